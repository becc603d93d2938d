"""GPU known-answer tests of the FP16 accumulation mode (fast_swa, metal_engine.mm:565).

The FP16 mode multiplies fp16 weight tiles F = RNE16(q*2^-24*A + B) that carry a per-row
power of two c (neutron-star_amd/csrc/ns_tile16.hpp, restated in oracle/ns_oracle.c) and
rounds the fp32 sum, times 1/c, once to fp16 precision.  Two cases pin that on the GPU
exactly, through every prefill GEMM kernel (the CDNA4 kernel of ns_gemm_f16.hip and the
LDS-tile kernel that serves the NSMFFN and ROW_MAJOR layouts), with and without split K:

  * the schedule: integer sums, every product and partial sum exact in fp32, so any
    summation order gives the same value: block sums 2049 + 1 must give 2050 (one rounding
    at the end; per-block rounding would give 2048) and 2049 alone must give 2048;
  * the tiles: one-hot tokens make y[t][r] = F[r][k_t] / c_r, an fp16 value times a power
    of two, so the GPU must return the oracle's tile values bit for bit.
"""
import numpy as np
import pytest

import ns_oracle as O
import nsffn as N
from helpers import f16_bits, f16_value, q4k_block

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

LAYOUTS = [N.CDNA4, N.NSMFFN, N.ROW_MAJOR]
LNAME = {N.CDNA4: "cdna4", N.NSMFFN: "nsmffn", N.ROW_MAJOR: "rowmajor"}


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = N.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def dev(host, qtype, cols, rows, layout):
    img = host if layout == N.ROW_MAJOR else N.retile(host, qtype, cols, rows, N.ROW_MAJOR, layout)
    return torch.from_numpy(np.ascontiguousarray(img)).cuda()


def schedule_weights(rows=64):
    """Row 0: block 0 sums to 2049 against ones (136 quants of 15, one of 9, d = 1, sc = 1,
    no min), block 1 to 1; rows 1.. are zero blocks."""
    sc1, m0 = np.ones(8, int), np.zeros(8, int)
    q0 = np.zeros(256, dtype=np.int64)
    q0[:136] = 15
    q0[136] = 9
    q1 = np.zeros(256, dtype=np.int64)
    q1[0] = 1
    zero = q4k_block(0.0, 0.0, m0, m0, np.zeros(256, int))
    row0 = np.concatenate([q4k_block(1.0, 0.0, sc1, m0, q0), q4k_block(1.0, 0.0, sc1, m0, q1)])
    return np.concatenate([row0] + [np.concatenate([zero, zero])] * (rows - 1))


@pytest.mark.parametrize("kparts", [0, 2], ids=["plan", "split2"])
@pytest.mark.parametrize("layout", LAYOUTS, ids=LNAME.get)
def test_fp16_mode_rounds_once_at_the_end(ctx, tune, layout, kparts):
    if kparts:
        tune("gemm_kparts", kparts)
    cols, rows, batch = 512, 64, 8
    host = schedule_weights(rows)
    w = dev(host, N.Q4_K, cols, rows, layout)
    x = np.zeros((batch, cols), dtype=np.float16)
    x[0, :] = 1
    x[1, :256] = 1
    xd = torch.from_numpy(f16_bits(x).view(np.int16)).cuda()
    out = {}
    for fast in (False, True):
        y = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
        ctx.ffn_down(w, N.Q4_K, layout, cols, rows, batch, xd, y, half_input=True, fast_swa=fast)
        torch.cuda.synchronize()
        out[fast] = y.cpu().numpy()
    assert out[False][0, 0] == 2050 and out[False][1, 0] == 2049
    assert out[True][0, 0] == 2050 and out[True][1, 0] == 2048
    for fast in (False, True):
        rest = out[fast].copy()
        rest[0, 0] = rest[1, 0] = 0
        assert not np.any(rest), fast
    # the oracle gives the same answers
    ref = O.gemm(N.Q4_K, O.ROW_MAJOR, host, cols, rows, batch, f16_bits(x), 1)
    np.testing.assert_array_equal(out[True], ref)


@pytest.mark.parametrize("layout", LAYOUTS, ids=LNAME.get)
@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
def test_fp16_tiles_one_hot_bit_exact(ctx, qtype, layout):
    """Seeded BASELINE-distributed weights with one fp16-subnormal d block per row; token t is
    one-hot at k_t, so y[t][r] = F[r][k_t] / c_r exactly: bit-equal to the oracle's tiles."""
    cols, rows = 768, 128
    host = N.synth_weights(qtype, 81 + qtype, rows, cols).copy()
    bb = 144 if qtype == N.Q4_K else 210
    blocks = host.reshape(rows, cols // 256, bb)
    doff = 0 if qtype == N.Q4_K else 208
    blocks[::3, 1, doff:doff + 2] = np.array([2.0 ** -20], dtype=np.float16).view(np.uint8)
    host = blocks.reshape(-1)
    ks = [0, 1, 31, 32, 100, 255, 256, 300, 511, 512, 640, 767]
    batch = len(ks)
    x = np.zeros((batch, cols), dtype=np.float16)
    for t, k in enumerate(ks):
        x[t, k] = 1
    w = dev(host, qtype, cols, rows, layout)
    y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    ctx.ffn_down(w, qtype, layout, cols, rows, batch, torch.from_numpy(f16_bits(x).view(np.int16)).cuda(), y,
                 half_input=True, fast_swa=True)
    torch.cuda.synchronize()
    tile, inv = O.f16_tile_rows(qtype, O.ROW_MAJOR, host, cols, rows)
    want = (tile[:, ks] * inv[:, None]).T
    np.testing.assert_array_equal(y.cpu().numpy(), want)


@pytest.mark.parametrize("layout", LAYOUTS, ids=LNAME.get)
def test_fp16_gate_up_one_hot(ctx, layout):
    """The gate/up pair in the FP16 mode on one-hot tokens: h = fp16(gelu(g) * u) with g, u the
    rows' tile values (exact), within one fp16 rounding step of the oracle's GeGLU of them."""
    cols, rows = 512, 128
    hg = N.synth_weights(N.Q4_K, 91, rows, cols)
    hu = N.synth_weights(N.Q4_K, 92, rows, cols)
    ks = [0, 7, 63, 64, 200, 256, 400, 511]
    x = np.zeros((len(ks), cols), dtype=np.float16)
    for t, k in enumerate(ks):
        x[t, k] = 1
    h = torch.empty((len(ks), rows), dtype=torch.int16, device="cuda")
    ctx.gate_up_geglu_rm32(dev(hg, N.Q4_K, cols, rows, layout), dev(hu, N.Q4_K, cols, rows, layout), layout,
                           cols, rows, len(ks), torch.from_numpy(f16_bits(x).view(np.int16)).cuda(), h, True)
    torch.cuda.synchronize()
    got = f16_value(h.cpu().numpy().view(np.uint16))
    ref = O.gate_up_geglu_prefill(O.ROW_MAJOR, hg, hu, cols, rows, len(ks), f16_bits(x), 1)
    step = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -14))) - 10)
    assert np.all(np.abs(got - ref) <= step)


def _down_case(qtype, batch, seed):
    cols, rows = 15360, 3840
    host = N.synth_weights(qtype, seed, rows, cols)
    w = dev(host, qtype, cols, rows, N.CDNA4)
    xd = torch.from_numpy(N.synth_normal_f16(seed + 1, batch * cols).view(np.int16).reshape(batch, cols)).cuda()
    return cols, rows, w, xd


def _run_down(ctx, qtype, cols, rows, batch, w, xd, fast=True):
    y = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
    ctx.ffn_down(w, qtype, N.CDNA4, cols, rows, batch, xd, y, half_input=True, fast_swa=fast)
    torch.cuda.synchronize()
    return y.cpu().numpy()


MODES = {"fp16": True, "fp32": False}


@pytest.mark.parametrize("kparts", [0, 2, 8], ids=["plan", "split2", "split8"])
@pytest.mark.parametrize("batch", [1024, 300])
@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("mode", list(MODES))
def test_split_k_reduce_scatter_equals_last_arrival(ctx, tune, mode, qtype, batch, kparts):
    """The down projection (3840 x 15360, CDNA4), in either accumulation mode, finishes its
    split-K tiles either by a reduce-scatter (every part adds the parts of its own token
    sub-tiles; the default when the grid fits the device at once and, in the FP32 mode, when
    the parts number as many as a wave's token sub-tiles) or by the last part to arrive
    (tuning key gemm_rs 0).  Both add the same fp32 parts in part order, so the outputs are
    equal bit for bit."""
    if kparts:
        tune("gemm_kparts", kparts)
    cols, rows, w, xd = _down_case(qtype, batch, 0xD0 + batch)
    a = _run_down(ctx, qtype, cols, rows, batch, w, xd, MODES[mode])
    tune("gemm_rs", 0)
    b = _run_down(ctx, qtype, cols, rows, batch, w, xd, MODES[mode])
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("mode", list(MODES))
def test_split_k_reduce_scatter_bounded_wait(ctx, tune, mode, qtype):
    """The reduce-scatter's wait for the other parts is bounded.  Forced down to two polls from
    the host (every wave still exits normally), a part whose wait ran out writes its token
    sub-tiles (32 tokens each) as NaN and every other sub-tile is the normal result; the
    context's status reports the timeout (NS_ERR_TIMEOUT) exactly when a sub-tile ran out,
    once; the next launch with the default bound is whole again (the last part clears the
    counters) and reports nothing."""
    batch = 1024
    cols, rows, w, xd = _down_case(qtype, batch, 0xE0)
    want = _run_down(ctx, qtype, cols, rows, batch, w, xd, MODES[mode])
    ctx.status()
    tune("gemm_rs", 2)
    got = _run_down(ctx, qtype, cols, rows, batch, w, xd, MODES[mode])
    blocks = got.reshape(batch // 32, 32, rows // 256, 256).transpose(0, 2, 1, 3)
    nan_blocks = int(sum(np.isnan(blocks[a, c]).all() for a in range(blocks.shape[0])
                         for c in range(blocks.shape[1])))
    if nan_blocks:
        with pytest.raises(N.NsError, match="reduce-scatter") as e:
            ctx.status()
        assert e.value.code == 7  # NS_ERR_TIMEOUT
    ctx.status()  # reported once, then clear
    tune("gemm_rs", 1)
    again = _run_down(ctx, qtype, cols, rows, batch, w, xd, MODES[mode])
    ref = want.reshape(batch // 32, 32, rows // 256, 256).transpose(0, 2, 1, 3)
    for a in range(blocks.shape[0]):
        for c in range(blocks.shape[1]):
            if not np.isnan(blocks[a, c]).all():
                assert np.array_equal(blocks[a, c].view(np.uint32), ref[a, c].view(np.uint32)), (a, c)
    print(f"bounded wait: {nan_blocks} of {blocks.shape[0] * blocks.shape[1]} sub-tiles ran out")
    assert np.array_equal(again.view(np.uint32), want.view(np.uint32))
    ctx.status()
