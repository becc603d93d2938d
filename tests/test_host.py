"""CPU tests of libnsffn.so: it loads, exports every C-ABI symbol of
include/ns_ffn.h, and its host-side logic (generator, layout conversion,
argument errors) is right.  No GPU call is made here."""
import ctypes

import numpy as np
import pytest

import ns_oracle as O
import nsffn as N


def test_library_exports_every_header_symbol():
    L = ctypes.CDLL(N.LIB_PATH)
    names = N.header_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert N.lib().ns_abi_version() == 1


def test_synth_is_deterministic_and_rangeable():
    a = N.synth_blocks(N.Q4_K, 5, 100)
    b = N.synth_blocks(N.Q4_K, 5, 100, nthreads=3)
    assert np.array_equal(a, b)
    # any sub-range reproduces the same blocks
    c = N.synth_blocks(N.Q4_K, 5, 10, first=40)
    assert np.array_equal(a.reshape(100, 144)[40:50].reshape(-1), c)
    assert not np.array_equal(a, N.synth_blocks(N.Q4_K, 6, 100))
    x1 = N.synth_normal_f32(9, 1000)
    assert np.array_equal(x1[500:], N.synth_normal_f32(9, 500, first=500))
    h = N.synth_normal_f16(9, 1000)
    assert np.array_equal(h, x1.astype(np.float16).view(np.uint16))


def test_synth_distributions():
    q4 = N.synth_blocks(N.Q4_K, 1, 20000).reshape(-1, 144)
    d = q4[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1)
    # |N(0,1)| * 1e-3 has mean sqrt(2/pi) * 1e-3
    assert abs(d.mean() / 1e-3 - np.sqrt(2 / np.pi)) < 0.02
    assert (d >= 0).all()
    qs = q4[:, 16:].reshape(-1)
    assert abs((qs & 15).mean() - 7.5) < 0.05
    q6 = N.synth_blocks(N.Q6_K, 2, 20000).reshape(-1, 210)
    sc = q6[:, 192:208].copy().view(np.int8).reshape(-1)
    assert sc.min() == -32 and sc.max() == 31
    x = N.synth_normal_f32(3, 200000)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    assert N.layer_seed(10, 0) == 10 and N.layer_seed(10, 1) == 10 ^ 0x9E3779B97F4A7C15


@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K])
def test_retile_matches_nsmffn_reorder_and_round_trips(qtype):
    cols, rows = 768, 192
    nb, bs = cols // 256, N.BLOCK_BYTES[qtype]
    rng = np.random.default_rng(qtype)
    src = rng.integers(0, 256, size=rows * nb * bs, dtype=np.uint8)
    ns = N.retile(src, qtype, cols, rows, N.ROW_MAJOR, N.NSMFFN)
    # the reference converter's mapping (metal_ffn.cpp:145-146), via the oracle's index
    L = O.lib()
    sb = src.reshape(rows * nb, bs)
    nsb = ns.reshape(rows * nb, bs)
    for r in range(rows):
        for b in range(nb):
            assert np.array_equal(nsb[L.nso_block_index(O.NSMFFN, r, b, nb)], sb[r * nb + b])
    cd = N.retile(ns, qtype, cols, rows, N.NSMFFN, N.CDNA4)
    assert not np.array_equal(cd, ns)
    assert np.array_equal(N.retile(cd, qtype, cols, rows, N.CDNA4, N.ROW_MAJOR), src)
    assert np.array_equal(N.retile(src, qtype, cols, rows, N.ROW_MAJOR, N.CDNA4), cd)


def test_cdna4_chunk_positions():
    # Q4_K: chunk c of row r%64 in slab region (slab*nb + kb)*64*144 at (c*64 + r%64)*16
    cols, rows = 512, 128
    nb = 2
    src = np.zeros(rows * nb * 144, dtype=np.uint8)
    blk = src.reshape(rows * nb, 144)
    blk[70 * nb + 1, 16 * 3 + 5] = 0xAB         # row 70, kb 1, chunk 3, byte 5
    cd = N.retile(src, N.Q4_K, cols, rows, N.ROW_MAJOR, N.CDNA4)
    region = (1 * nb + 1) * 64 * 144
    assert cd[region + (3 * 64 + 6) * 16 + 5] == 0xAB
    assert int(cd.sum()) == 0xAB
    # Q6_K d (bytes 208..209) sits after the 13 chunk planes
    src = np.zeros(rows * nb * 210, dtype=np.uint8)
    src.reshape(rows * nb, 210)[3 * nb + 0, 209] = 0x7F
    cd = N.retile(src, N.Q6_K, cols, rows, N.ROW_MAJOR, N.CDNA4)
    assert cd[13 * 1024 + 3 * 2 + 1] == 0x7F


def test_host_argument_errors():
    src = np.zeros(144 * 64, dtype=np.uint8)
    with pytest.raises(N.NsError) as e:
        N.retile(src, 13, 256, 64, N.ROW_MAJOR, N.NSMFFN)
    assert e.value.code == 1 and "type" in str(e.value)
    with pytest.raises(N.NsError) as e:
        N.retile(src, N.Q4_K, 300, 64, N.ROW_MAJOR, N.NSMFFN)
    assert e.value.code == 2
    with pytest.raises(N.NsError):
        N.retile(src, N.Q4_K, 256, 60, N.ROW_MAJOR, N.CDNA4)
