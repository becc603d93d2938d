"""CPU tests pinning the oracle (oracle/ns_oracle.c) before it is trusted.

Pins, per oracle function:
  f16<->f32      numpy float16 over all 65536 half patterns / 200k float patterns.
  q4k/q6k value  the reference's own quant.cpp (oracle/_ref, compiled from the
                 reference checkout, when present), the committed golden vectors
                 made from it (tests/golden/), and hand-built closed-form blocks.
  dot_row        oracle/_ref bit-exact; one-hot columns; linearity.
  gemv           bit-identical to dot_row for every row.
  gelu_tanh      gelu(0)=0, gelu(g)-gelu(-g)=g, large |g| -> relu, float64 formula.
  .nsmffn index  metal_ffn.cpp:145-146 known answers and bijection.
  FP16 mode      the oracle's FP16-mode functions (f16_tile_rows, gemm and
                 gate_up_geglu_prefill with acc_mode 1) restate this build's own
                 tile formulas and its single final rounding, so checks against
                 them are a self-consistency check of the kernels.  They are pinned
                 here by worked tile values, equality with the reference's
                 half(d*sc*q - dmin*m) form on power-of-two factors, the tile error
                 bound and the 2049+1 rounding case.  The reference's own FP16 mode
                 accumulates in Apple simdgroup half registers (metal:380, :487),
                 which nothing here can run: parity with that arithmetic is
                 unpinned.  The FP16 mode's parity evidence is its bound against
                 the FP32 oracle (the reference's CPU arithmetic), 1e-2.
"""
import os

import numpy as np
import pytest

import ns_oracle as O
from helpers import f16_bits, q4k_block, q6k_block

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz")


def _rng(seed=1234):
    return np.random.default_rng(seed)


def test_f16_to_f32_all_patterns():
    L = O.lib()
    h = np.arange(65536, dtype=np.uint32)
    got = np.array([L.nso_f16_to_f32(int(v)) for v in h], dtype=np.float32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rne():
    L = O.lib()
    rng = _rng()
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0**-25, 2.0**-24, 3 * 2.0**-25,
                         2.0**-14, 6.1e-5, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, np.inf, -np.inf],
                        dtype=np.float32).view(np.uint32)
    f = np.concatenate([bits, specials]).view(np.float32)
    f = f[~np.isnan(f)]
    got = np.array([L.nso_f32_to_f16(float(v)) for v in f], dtype=np.uint16)
    want = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def _random_blocks(qtype, n, seed):
    """Uniform random bytes with sane (finite) fp16 scale fields, plus extremes."""
    rng = _rng(seed)
    bs = 144 if qtype == O.Q4_K else 210
    b = rng.integers(0, 256, size=(n, bs), dtype=np.uint8)
    scale = rng.choice([1e-3, 0.5, 3.0e-6, 6.0e-8, 0.0, 65504.0], size=(n, 2)).astype(np.float16)
    if qtype == O.Q4_K:
        b[:, 0:2] = scale[:, 0:1].view(np.uint8)
        b[:, 2:4] = scale[:, 1:2].view(np.uint8)
    else:
        b[:, 208:210] = scale[:, 0:1].view(np.uint8)
    return np.ascontiguousarray(b.reshape(-1))


@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q6_K])
def test_values_match_reference_quant_cpp(qtype):
    if O.ref() is None:
        pytest.skip("oracle/_ref not built (reference checkout absent); golden vectors cover this")
    n = 64
    w = _random_blocks(qtype, n, seed=qtype)
    cols, rows = 512, n // 2
    mine = O.dequant_rows(qtype, O.ROW_MAJOR, w, cols, rows).reshape(-1)
    rc, theirs = O.ref_dequant(qtype, w, cols, rows, 0, cols * rows)
    assert rc == 0
    assert np.array_equal(mine.view(np.uint32), theirs.view(np.uint32))
    x = _rng(7).standard_normal(cols).astype(np.float32)
    for r in range(rows):
        rc, d = O.ref_dot_row(qtype, w, cols, rows, r, x)
        assert rc == 0
        assert np.float32(d).view(np.uint32) == np.float32(O.dot_row(qtype, O.ROW_MAJOR, w, cols, rows, r, x)).view(np.uint32)


def test_reference_rejects_out_of_range():
    if O.ref() is None:
        pytest.skip("oracle/_ref not built")
    w = _random_blocks(O.Q4_K, 2, 3)
    rc, _ = O.ref_dequant(O.Q4_K, w, 256, 2, 511, 2)  # element 512 is out of range
    assert rc != 0


def test_golden_vectors():
    g = np.load(GOLDEN, allow_pickle=False)
    for name, qtype in (("q4k", O.Q4_K), ("q6k", O.Q6_K)):
        w = np.ascontiguousarray(g[f"{name}_bytes"])
        cols, rows = int(g[f"{name}_shape"][0]), int(g[f"{name}_shape"][1])
        want = g[f"{name}_values"].reshape(rows, cols)
        got = O.dequant_rows(qtype, O.ROW_MAJOR, w, cols, rows)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
        x = g[f"{name}_x"]
        for r in range(rows):
            d = O.dot_row(qtype, O.ROW_MAJOR, w, cols, rows, r, x)
            assert np.float32(d).view(np.uint32) == g[f"{name}_dot"][r].view(np.uint32), (name, r)


def test_q4k_closed_forms():
    # d=1, dmin=0.5, scales sc_g = g+1, mins m_g = 2g, q = element index mod 16
    sc = [g + 1 for g in range(8)]
    m = [2 * g for g in range(8)]
    q = [i % 16 for i in range(256)]
    b = q4k_block(1.0, 0.5, sc, m, q)
    vals = np.array([O.lib().nso_q4k_value(b.ctypes.data, i) for i in range(256)], dtype=np.float32)
    want = np.array([1.0 * sc[i // 32] * q[i] - 0.5 * m[i // 32] for i in range(256)], dtype=np.float32)
    assert np.array_equal(vals, want)
    # high-bit scales (sc, m >= 16 exercise the 2-bit tops stored in scales[0..7])
    b = q4k_block(2.0, 1.0, [63, 17, 32, 48, 63, 17, 32, 48], [63, 0, 16, 47, 31, 62, 1, 33], [15] * 256)
    v = np.array([O.lib().nso_q4k_value(b.ctypes.data, 32 * g) for g in range(8)], dtype=np.float32)
    assert list(v) == [2.0 * s * 15 - mm for s, mm in zip([63, 17, 32, 48, 63, 17, 32, 48],
                                                          [63, 0, 16, 47, 31, 62, 1, 33])]
    # d = dmin = 0 -> zeros; fp16-subnormal d
    b = q4k_block(0.0, 0.0, [63] * 8, [63] * 8, [15] * 256)
    assert all(O.lib().nso_q4k_value(b.ctypes.data, i) == 0.0 for i in range(256))
    sub = float(np.float16(2.0**-20))
    b = q4k_block(sub, 0.0, [3] * 8, [0] * 8, [5] * 256)
    assert O.lib().nso_q4k_value(b.ctypes.data, 77) == np.float32(sub * 15)


def test_q6k_closed_forms():
    v = [i % 64 for i in range(256)]
    sc = [s - 8 for s in range(16)]
    b = q6k_block(0.25, sc, v)
    vals = np.array([O.lib().nso_q6k_value(b.ctypes.data, i) for i in range(256)], dtype=np.float32)
    want = []
    for i in range(256):
        half, p = divmod(i, 128)
        quarter, l = divmod(p, 32)
        want.append(0.25 * sc[half * 8 + l // 16 + quarter * 2] * (v[i] - 32))
    assert np.array_equal(vals, np.array(want, dtype=np.float32))
    # sc = -32, v = 0 -> d * 1024
    b = q6k_block(0.5, [-32] * 16, [0] * 256)
    assert O.lib().nso_q6k_value(b.ctypes.data, 200) == 512.0


@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q6_K])
def test_dot_row_one_hot_and_linearity(qtype):
    w = _random_blocks(qtype, 8, seed=11)
    cols, rows = 512, 4
    deq = O.dequant_rows(qtype, O.ROW_MAJOR, w, cols, rows)
    for k in (0, 37, 255, 256, 511):
        e = np.zeros(cols, dtype=np.float32)
        e[k] = 1.0
        for r in range(rows):
            assert O.dot_row(qtype, O.ROW_MAJOR, w, cols, rows, r, e) == deq[r, k]
    rng = _rng(5)
    x1, x2 = rng.standard_normal((2, cols)).astype(np.float32)
    for r in range(rows):
        a = O.dot_row(qtype, O.ROW_MAJOR, w, cols, rows, r, x1 + x2)
        b = O.dot_row(qtype, O.ROW_MAJOR, w, cols, rows, r, x1) + O.dot_row(qtype, O.ROW_MAJOR, w, cols, rows, r, x2)
        scale = np.sum(np.abs(deq[r]) * (np.abs(x1) + np.abs(x2)))
        assert abs(a - b) <= 1e-5 * scale


@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q6_K])
def test_gemv_equals_dot_row(qtype):
    w = _random_blocks(qtype, 64 * 4, seed=21)
    cols, rows = 1024, 64
    x = _rng(9).standard_normal(cols).astype(np.float32)
    y = O.gemv(qtype, O.ROW_MAJOR, w, cols, rows, x, nthreads=4)
    for r in range(rows):
        assert np.float32(y[r]).view(np.uint32) == np.float32(O.dot_row(qtype, O.ROW_MAJOR, w, cols, rows, r, x)).view(np.uint32)


def test_gelu_closed_forms():
    g = O.gelu_tanh
    assert g(0.0) == 0.0
    for v in (0.1, 1.0, 3.5, 20.0):
        assert abs((g(v) - g(-v)) - v) <= 4e-7 * max(1.0, v)
    assert g(30.0) == 30.0 and g(-30.0) == 0.0
    xs = np.linspace(-8, 8, 161)
    ref = 0.5 * xs * (1 + np.tanh(np.sqrt(2 / np.pi) * (xs + 0.044715 * xs**3)))
    got = np.array([g(float(v)) for v in xs])
    assert np.max(np.abs(got - ref)) <= 2e-6 * np.max(np.abs(ref))


def test_nsmffn_block_index():
    L = O.lib()
    # metal_ffn.cpp:145-146: target = ((row0/64)*blocks + block)*64 + row
    assert L.nso_block_index(O.NSMFFN, 0, 0, 15) == 0
    assert L.nso_block_index(O.NSMFFN, 1, 0, 15) == 1
    assert L.nso_block_index(O.NSMFFN, 0, 1, 15) == 64
    assert L.nso_block_index(O.NSMFFN, 65, 2, 15) == (1 * 15 + 2) * 64 + 1
    assert L.nso_block_index(O.ROW_MAJOR, 65, 2, 15) == 65 * 15 + 2
    nb, rows = 3, 128
    idx = {L.nso_block_index(O.NSMFFN, r, b, nb) for r in range(rows) for b in range(nb)}
    assert idx == set(range(rows * nb))


def test_fp16_mode_oracle_is_fp16_and_close():
    rng = _rng(3)
    cols, rows, batch = 512, 64, 5
    w = _random_blocks(O.Q4_K, rows * cols // 256, seed=4)
    # keep scales at the model's magnitude so fp16 cannot overflow
    wb = w.reshape(-1, 144)
    wb[:, 0:4] = np.array([1e-3, 1e-3], dtype=np.float16).view(np.uint8)
    x = f16_bits(rng.standard_normal((batch, cols)).astype(np.float16))
    y32 = O.gemm(O.Q4_K, O.ROW_MAJOR, w, cols, rows, batch, x, 0)
    y16 = O.gemm(O.Q4_K, O.ROW_MAJOR, w, cols, rows, batch, x, 1)
    assert not np.any(y16.view(np.uint32) & 0x1FFF)  # 11 significant bits
    assert np.max(np.abs(y16 - y32)) <= 4e-3 * np.max(np.abs(y32))


def test_round_f16p():
    """FP16-mode rounding equals fp16 RNE on the fp16 normal range and keeps
    magnitudes beyond it (no overflow)."""
    L = O.lib()
    rng = _rng(8)
    v = (rng.standard_normal(50_000) * np.exp(rng.uniform(-9, 11, 50_000))).astype(np.float32)
    v = v[(np.abs(v) >= 2.0**-14) & (np.abs(v) < 65504)]
    got = np.array([L.nso_round_f16p(float(a)) for a in v], dtype=np.float32)
    assert np.array_equal(got, v.astype(np.float16).astype(np.float32))
    big = np.float32(171474.9)
    r = L.nso_round_f16p(float(big))
    assert np.isfinite(r) and abs(r - big) <= big * 2.0**-11
    assert L.nso_round_f16p(1.0 + 2.0**-11) == 1.0 and L.nso_round_f16p(1.0 + 3 * 2.0**-11) == 1.0 + 2.0**-9


# ---- the RMSNorm family (metal:509-529) ---------------------------------------------

def test_rmsnorm_known_answers():
    """Closed forms: x = (3, 4, 0, 0) has mean square 25/4, so r = 0.4 exactly with eps = 0;
    a constant row c has r = 1/sqrt(c^2 + eps); a zero row with eps > 0 maps to zeros."""
    w = np.array([1.0, 2.0, -1.0, 0.5], dtype=np.float32)
    y = O.rmsnorm(np.array([3.0, 4.0, 0.0, 0.0], dtype=np.float32), w, eps=0.0)
    np.testing.assert_array_equal(y, np.float32([1.2, 3.2, 0.0, 0.0]))
    c, eps = np.float32(-2.5), np.float32(1e-3)
    y = O.rmsnorm(np.full(64, c, dtype=np.float32), np.ones(64, dtype=np.float32), eps=float(eps))
    expect = float(c) / np.sqrt(float(c) ** 2 + float(eps))
    assert np.allclose(y, expect, rtol=2e-7, atol=0)
    assert not np.any(O.rmsnorm(np.zeros(16, np.float32), np.ones(16, np.float32), eps=1e-6))


def test_rmsnorm_unit_rms_and_scale_invariance():
    """With w = 1 and eps = 0 the output has mean square 1; scaling x by 2^k leaves the
    output unchanged bit for bit (the sum scales by 4^k exactly, the root by 2^k)."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 3840)).astype(np.float32)
    ones = np.ones(3840, dtype=np.float32)
    y = O.rmsnorm(x, ones, eps=0.0)
    assert np.allclose(np.mean(y.astype(np.float64) ** 2, axis=1), 1.0, rtol=1e-5)
    w = rng.standard_normal(3840).astype(np.float32)
    for k in (-6, 3, 10):
        np.testing.assert_array_equal(O.rmsnorm(x * np.float32(2.0 ** k), w, eps=0.0), O.rmsnorm(x, w, eps=0.0))


def test_rmsnorm_add_and_then():
    """rms_add: a zero input with eps > 0 returns the residual (times scale) exactly; the
    residual enters additively.  The _then form equals rms_add followed by rms (mm:563)."""
    rng = np.random.default_rng(6)
    res = rng.standard_normal(256).astype(np.float32)
    w = rng.standard_normal(256).astype(np.float32)
    np.testing.assert_array_equal(O.rmsnorm(np.zeros(256, np.float32), w, residual=res, eps=1e-6), res)
    np.testing.assert_array_equal(O.rmsnorm(np.zeros(256, np.float32), w, residual=res, scale=0.5, eps=1e-6),
                                  res * np.float32(0.5))
    x = rng.standard_normal(256).astype(np.float32)
    y0 = O.rmsnorm(x, w, eps=1e-6)
    y1 = O.rmsnorm(x, w, residual=np.zeros(256, np.float32), eps=1e-6)
    np.testing.assert_array_equal(y1, y0)  # 0 + v == v
    nw = rng.standard_normal(256).astype(np.float32)
    y, nxt = O.rmsnorm(x, w, residual=res, scale=0.75, next_w=nw, eps=1e-6)
    np.testing.assert_array_equal(y, O.rmsnorm(x, w, residual=res, scale=0.75, eps=1e-6))
    np.testing.assert_array_equal(nxt, O.rmsnorm(y, nw, eps=1e-6))


# ---- the FP16 mode: fp16 tiles with a row scale, one rounding at the end ----------------

def _q4_rows(specs):
    """Q4_K rows from (d, dmin, sc[8], m[8], q[256]) per block: spec[r] = list of blocks."""
    return np.concatenate([np.concatenate([q4k_block(*blk) for blk in row]) for row in specs])


def test_f16_tile_equals_reference_half_form_on_power_of_two_factors():
    """With d and dmin powers of two, A = d*sc*2^24*c and B = -dmin*m*c are exact in fp16, so
    the tile is one rounding of c*(d*sc*q - dmin*m) and F/c equals the reference's
    half(d*sc*q - dmin*m) (metal:231) bit for bit.  Q6_K likewise with half(d*sc*(v-32))
    (metal:417-418).  Random quants and scales, factors 2^-12..2^-6."""
    rng = _rng(21)
    cols, rows = 512, 8
    specs = []
    for r in range(rows):
        blocks = []
        for b in range(cols // 256):
            blocks.append((2.0 ** -int(rng.integers(6, 13)), 2.0 ** -int(rng.integers(6, 13)),
                           rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256)))
        specs.append(blocks)
    w = _q4_rows(specs)
    tile, inv = O.f16_tile_rows(O.Q4_K, O.ROW_MAJOR, w, cols, rows)
    exact = O.dequant_rows(O.Q4_K, O.ROW_MAJOR, w, cols, rows)
    np.testing.assert_array_equal(tile * inv[:, None], exact.astype(np.float16).astype(np.float32))
    w6 = _random_blocks(O.Q6_K, rows * cols // 256, seed=22).reshape(-1, 210)
    w6[:, 208:210] = np.array([2.0 ** -int(e) for e in rng.integers(6, 13, len(w6))],
                              dtype=np.float16).view(np.uint8).reshape(-1, 2)
    w6 = w6.reshape(-1)
    tile, inv = O.f16_tile_rows(O.Q6_K, O.ROW_MAJOR, w6, cols, rows)
    exact = O.dequant_rows(O.Q6_K, O.ROW_MAJOR, w6, cols, rows)
    np.testing.assert_array_equal(tile * inv[:, None], exact.astype(np.float16).astype(np.float32))


def test_f16_tile_known_roundings():
    """Hand-computed values.  d = 1 + 2^-10, dmin = 0.5: M = d, ceil(log2 M) = 1, c = 2^-16,
    c*2^24 = 256.  Group 0 (sc = 63, m = 63): A = RNE16(63.0615234375 * 256 = 16143.75) = 16144
    (ulp 8); B = -0.5*63*2^-16 = -2016 * 2^-22 (exact).  q = 15: q*2^-24*A + B =
    0.013953208923339844 = 1828.875 ulps of 2^-17 -> RNE16 = 1829 * 2^-17.  q = 0 gives B
    itself; a block with d = dmin = 0 gives zeros."""
    sc = np.array([63, 1, 2, 3, 4, 5, 6, 7])
    m = np.array([63, 0, 0, 0, 0, 0, 0, 0])
    q = np.zeros(256, dtype=np.int64)
    q[0], q[1] = 15, 0
    w = _q4_rows([[(1.0 + 2.0 ** -10, 0.5, sc, m, q), (0.0, 0.0, np.zeros(8, int), np.zeros(8, int),
                                                        np.zeros(256, int))]])
    tile, inv = O.f16_tile_rows(O.Q4_K, O.ROW_MAJOR, w, 512, 1)
    assert inv[0] == 2.0 ** 16
    A = 16144.0
    B = -2016.0 * 2.0 ** -22
    v = 15 * 2.0 ** -24 * A + B
    assert v / 2.0 ** -17 == 1828.875
    assert tile[0, 0] == np.float32(1829 * 2.0 ** -17)
    assert tile[0, 1] == np.float32(B)
    assert not np.any(tile[0, 256:])
    # the row scale at and just past a power of two: M = 2 -> c*2^24 = 2^8; M = 2 + 2^-9 -> 2^7
    for dv, expect in ((2.0, 2.0 ** (15 + 1)), (2.0 + 2.0 ** -9, 2.0 ** (15 + 2)), (2.0 ** -24, 2.0 ** -9)):
        w1 = _q4_rows([[(dv, 0.0, sc, np.zeros(8, int), q)]])
        _, inv1 = O.f16_tile_rows(O.Q4_K, O.ROW_MAJOR, w1, 256, 1)
        assert inv1[0] == np.float32(expect), (dv, inv1[0])
    # a zero row: c = 1 and zero tiles
    wz = _q4_rows([[(0.0, 0.0, sc, m, q)]])
    tz, iz = O.f16_tile_rows(O.Q4_K, O.ROW_MAJOR, wz, 256, 1)
    assert iz[0] == 1.0 and not np.any(tz)


def test_f16_tile_q6k_row_scale_and_int8_extremes():
    """Q6_K rows take the power of two strictly above M: M = 2 gives E = 2, c = 2^-17 (a Q4_K row
    with M = 2 takes E = 1).  Hand-computed tiles for d = 2 and sc = -128, the scale llama.cpp's
    quantiser gives the largest group of every Q6_K block: A = RNE16(2 * -128 * 2^24 * 2^-17) =
    -2^15 (with E = 1 it would be -2^16, past fp16's range), B = RNE16(-32 * 2 * -128 * 2^-17) =
    2^-4; v = 0 gives B, v = 63 gives 63 * 2^-24 * -2^15 + 2^-4 = -31 * 2^-9 (exact), and F/c
    are the weights 8192 and -7936.  sc = 127 with v = 63: c*w = 2 * 127 * 31 * 2^-17 is 1968.5
    ulps of 2^-15, a tie that RNE16 takes to 1968: F/c = 7872 (the FP16 mode's one rounding)."""
    sc = np.full(16, 127)
    sc[0] = -128
    v = np.zeros(256, dtype=np.int64)
    v[1] = 63
    v[16] = 63  # group 1 (sc = 127)
    w = q6k_block(np.float16(2.0), sc, v)
    tile, inv = O.f16_tile_rows(O.Q6_K, O.ROW_MAJOR, w, 256, 1)
    assert inv[0] == 2.0 ** 17
    assert tile[0, 0] == np.float32(2.0 ** -4)
    assert tile[0, 1] == np.float32(-31 * 2.0 ** -9)
    assert tile[0, 0] * inv[0] == 8192.0 and tile[0, 1] * inv[0] == -7936.0
    assert tile[0, 16] == np.float32(1968 * 2.0 ** -15) and tile[0, 16] * inv[0] == 7872.0
    assert np.isfinite(tile).all()
    # away from powers of two the row scale is ceil(log2 M), as for Q4_K
    for dv, expect in ((2.0 + 2.0 ** -9, 2.0 ** 17), (1.5, 2.0 ** 16), (2.0 ** -24, 2.0 ** -8)):
        _, inv6 = O.f16_tile_rows(O.Q6_K, O.ROW_MAJOR, q6k_block(np.float16(dv), sc, v), 256, 1)
        assert inv6[0] == np.float32(expect), (dv, inv6[0])


def test_f16_tile_error_bound():
    """On BASELINE-distributed blocks, F/c differs from the exact weight w by at most the three
    roundings of A, B and F: |F/c - w| <= 2^-11 * (|d*sc*q| + |dmin*m| + |w|) * (1 + 2^-10)
    plus the subnormal step 2^-24/c, bounded here through |d*sc*q| <= |w| + 63|dmin| (Q6_K:
    |d*sc*v| + 32|d*sc| <= |w| + 64*32|d|).  A wrong row scale, a dropped B or a q off by one
    breaks this by the size of a weight."""
    nsffn = pytest.importorskip("nsffn")
    cols, rows = 3840, 64
    for qt in (O.Q4_K, O.Q6_K):
        w = nsffn.synth_weights(qt, 23 + qt, rows, cols)
        tile, inv = O.f16_tile_rows(qt, O.ROW_MAJOR, w, cols, rows)
        exact = O.dequant_rows(qt, O.ROW_MAJOR, w, cols, rows).astype(np.float64)
        got = tile.astype(np.float64) * inv[:, None]
        blocks = w.reshape(rows, cols // 256, 144 if qt == O.Q4_K else 210)
        if qt == O.Q4_K:
            side = 63 * np.abs(blocks[:, :, 2:4].copy().view(np.float16).astype(np.float64))  # 63|dmin|
            terms = 2 * np.abs(exact) + 2 * np.repeat(side[:, :, 0], 256, axis=1)
        else:
            dd = np.abs(blocks[:, :, 208:210].copy().view(np.float16).astype(np.float64))
            terms = 2 * np.abs(exact) + 64 * 32 * np.repeat(dd[:, :, 0], 256, axis=1)
        bound = 2.0 ** -11 * (1 + 2.0 ** -10) * terms + 2.0 ** -24 * inv[:, None].astype(np.float64)
        assert np.all(np.abs(got - exact) <= bound), qt


def test_fp16_mode_rounds_once_at_the_end():
    """Integer sums (every product and partial sum exact): one row whose block 0 sums to 2049
    and block 1 to 1.  x = 1 on both blocks: FP32 mode 2050; FP16 mode RNE11(2050) = 2050 (one
    rounding at the end; rounding per super-block would give RNE11(RNE11(2049) + 1) = 2048).
    x = 1 on block 0 only: FP32 2049, FP16 RNE11(2049) = 2048 (the tie goes to even)."""
    sc1, m0 = np.ones(8, int), np.zeros(8, int)
    q0 = np.zeros(256, dtype=np.int64)
    q0[:136] = 15
    q0[136] = 9
    q1 = np.zeros(256, dtype=np.int64)
    q1[0] = 1
    row0 = [(1.0, 0.0, sc1, m0, q0), (1.0, 0.0, sc1, m0, q1)]
    zero = [(0.0, 0.0, m0, m0, np.zeros(256, int))] * 2
    w = _q4_rows([row0, zero])
    x = np.zeros((2, 512), dtype=np.float16)
    x[0, :] = 1
    x[1, :256] = 1
    xb = f16_bits(x)
    y32 = O.gemm(O.Q4_K, O.ROW_MAJOR, w, 512, 2, 2, xb, 0)
    y16 = O.gemm(O.Q4_K, O.ROW_MAJOR, w, 512, 2, 2, xb, 1)
    assert y32[0, 0] == 2050 and y32[1, 0] == 2049
    assert y16[0, 0] == 2050 and y16[1, 0] == 2048
    assert not np.any(y32[:, 1]) and not np.any(y16[:, 1])
