"""GPU parity tests: the HIP path, called through the C ABI, against the CPU
oracle on identical seeded inputs.

Bars:
  dequantised weights      bit-exact (fp32 and its fp16 RNE)
  FP32-accumulation output rel_err <= 1e-3
  FP16-accumulation output rel_err <= 1e-2
rel_err (tests/helpers.py) = max over output rows of max|got-ref| / max|ref|.
"""
import numpy as np
import pytest

import ns_oracle as O
import nsffn as N
from helpers import f16_value, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL32, TOL16 = 1e-3, 1e-2
# FP16-mode outputs against the oracle's FP16 mode (the same tiles and one final rounding to
# 11 bits): they differ only by the fp32 summation order before that rounding, i.e. at most
# one fp16 rounding step of an output, 2^-11 < 1e-3 of the row's largest value.
TOL16_SAME = 1e-3
# The gate/up pair rounds g and u to 11 bits before GeGLU: a rounding step of g or u that
# flips between the two summation orders is amplified by GeGLU (by up to ~6 near its minimum,
# g ~ -2.5), plus h's own rounding; measured against the largest |h| of the columns compared.
TOL16_SAME_PAIR = 5e-3
LAYOUTS = [N.CDNA4, N.NSMFFN, N.ROW_MAJOR]
LNAME = {N.CDNA4: "cdna4", N.NSMFFN: "nsmffn", N.ROW_MAJOR: "rowmajor"}


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = N.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def dev_bytes(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()


def weights(qtype, seed, rows, cols, layout):
    """(oracle ROW_MAJOR bytes, device bytes in `layout`)."""
    host = N.synth_weights(qtype, seed, rows, cols)
    lay = host if layout == N.ROW_MAJOR else N.retile(host, qtype, cols, rows, N.ROW_MAJOR, layout)
    return host, dev_bytes(lay)


def f32(n, seed):
    return N.synth_normal_f32(seed, n)


# ---- dequantisation: bit-exact ------------------------------------------------

@pytest.mark.parametrize("layout", LAYOUTS, ids=LNAME.get)
@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
def test_dequant_bit_exact(ctx, qtype, layout):
    cols, rows = 1024, 192
    host, w = weights(qtype, 100 + qtype, rows, cols, layout)
    out32 = torch.empty((rows - 64, cols), dtype=torch.float32, device="cuda")
    out16 = torch.empty((rows - 64, cols), dtype=torch.int16, device="cuda")
    ctx.dequant(w, qtype, layout, cols, rows, 64, rows - 64, out32, out16)
    torch.cuda.synchronize()
    want = O.dequant_rows(qtype, O.ROW_MAJOR, host, cols, rows, 64, rows - 64)
    got32 = out32.cpu().numpy()
    assert np.array_equal(got32.view(np.uint32), want.view(np.uint32))
    got16 = out16.cpu().numpy().view(np.uint16)
    assert np.array_equal(got16, want.astype(np.float16).view(np.uint16))


# ---- decode GEMV ----------------------------------------------------------------

GEMV_CASES = [
    (N.Q4_K, 3840, 15360, "cfg0_q4k_gate"),
    (N.Q6_K, 15360, 3840, "cfg1a_q6k_down"),
    (N.Q4_K, 15360, 3840, "q4k_down"),
    (N.Q6_K, 256, 64, "tiny"),
    (N.Q4_K, 512, 192, "small"),
]


@pytest.mark.parametrize("layout", LAYOUTS, ids=LNAME.get)
@pytest.mark.parametrize("qtype,cols,rows,name", GEMV_CASES, ids=[c[3] for c in GEMV_CASES])
def test_gemv(ctx, qtype, cols, rows, name, layout):
    host, w = weights(qtype, 7, rows, cols, layout)
    x = f32(cols, 8)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.matmul(w, qtype, layout, cols, rows, 1, torch.from_numpy(x).cuda(), y)
    torch.cuda.synchronize()
    ref = O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, x)
    assert rel_err(y.cpu().numpy(), ref) <= TOL32


@pytest.mark.parametrize("qslab", ["1", "0"], ids=["k_wg_per_slab", "flattened"])
@pytest.mark.parametrize("qtype,rows,layout", [(N.Q6_K, 3840, N.CDNA4), (N.Q4_K, 3840, N.NSMFFN),
                                               (N.Q6_K, 3840 - 24, N.ROW_MAJOR)],
                         ids=["q6k_cdna4", "q4k_nsmffn", "q6k_rowmajor_ragged"])
def test_down_plans(ctx, tune, qslab, qtype, rows, layout):
    """The 60-block down projection under both grids of the one-unit instance:
    4 workgroups of 15 waves per slab (default) and the flattened split
    (NS_GEMV_QSLAB=0, 15 workgroups per slab); both meet the bar and repeat."""
    tune("gemv_qslab", qslab)
    cols = 15360
    host, w = weights(qtype, 41, rows, cols, layout)
    x = f32(cols, 42)
    ref = O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, x)
    ys = []
    for _ in range(2):
        y = torch.empty(rows, dtype=torch.float32, device="cuda")
        ctx.matmul(w, qtype, layout, cols, rows, 1, torch.from_numpy(x).cuda(), y)
        ys.append(y)
    torch.cuda.synchronize()
    assert rel_err(ys[0].cpu().numpy(), ref) <= TOL32
    assert torch.equal(ys[0], ys[1])


@pytest.mark.parametrize("layout", [N.CDNA4, N.ROW_MAJOR], ids=LNAME.get)
def test_lm_head_gemv(ctx, layout):
    """Config 1b: Q6_K 262144 x 3840 lm-head (row-major in the reference, mm:576)."""
    cols, rows = 3840, 262144
    host, w = weights(N.Q6_K, 9, rows, cols, layout)
    x = f32(cols, 10)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.matmul(w, N.Q6_K, layout, cols, rows, 1, torch.from_numpy(x).cuda(), y)
    torch.cuda.synchronize()
    ref = O.gemv(N.Q6_K, O.ROW_MAJOR, host, cols, rows, x)
    assert rel_err(y.cpu().numpy(), ref) <= TOL32


# ---- the streaming GEMV (the lm-head instance) ----------------------------------
# With at least two slabs per resident workgroup the streaming instance gives
# every slab its own 4-wave workgroup (parts meet in LDS); NS_GEMV_WAVES forces
# the flattened grid instead (slabs cut between waves and workgroups).  Both
# grids must meet the bar, and each must repeat bit for bit.

def _lm_head(ctx, layout, rows=262144):
    cols = 3840
    host, w = weights(N.Q6_K, 9, rows, cols, layout)
    x = f32(cols, 10)
    return host, w, x, cols, rows


def _run(ctx, qtype, w, layout, cols, rows, x):
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.matmul(w, qtype, layout, cols, rows, 1, torch.from_numpy(x).cuda(), y)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("waves", [None, "2048", "12288"], ids=["slab_per_wg", "resident", "cut_slabs"])
def test_stream_grids(ctx, tune, waves):
    if waves:
        tune("gemv_waves", waves)
    host, w, x, cols, rows = _lm_head(ctx, N.CDNA4)
    ref = O.gemv(N.Q6_K, O.ROW_MAJOR, host, cols, rows, x)
    y = _run(ctx, N.Q6_K, w, N.CDNA4, cols, rows, x)
    assert rel_err(y, ref) <= TOL32
    assert np.array_equal(_run(ctx, N.Q6_K, w, N.CDNA4, cols, rows, x).view(np.uint32), y.view(np.uint32))


def test_stream_repeated_launches(ctx):
    """Back-to-back launches on one stream give identical results (the hand-off
    counters of cut slabs return to zero after each launch)."""
    _, w, x, cols, rows = _lm_head(ctx, N.CDNA4)
    xd = torch.from_numpy(x).cuda()
    ys = [torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda") for _ in range(4)]
    for y in ys:
        ctx.matmul(w, N.Q6_K, N.CDNA4, cols, rows, 1, xd, y)
    torch.cuda.synchronize()
    assert not torch.isnan(ys[0]).any()
    assert all(torch.equal(ys[0], t) for t in ys[1:])


STREAM_CASES = [
    (N.Q6_K, 3840, 262144 - 37, N.ROW_MAJOR, "lm_head_ragged"),
    (N.Q4_K, 512, 192, N.CDNA4, "q4k_small"),
    (N.Q6_K, 256, 64, N.NSMFFN, "q6k_one_slab"),
    (N.Q4_K, 3840, 65536, N.NSMFFN, "q4k_wide"),
    (N.Q6_K, 768, 131072, N.CDNA4, "q6k_three_blocks"),
]


@pytest.mark.parametrize("qtype,cols,rows,layout,name", STREAM_CASES, ids=[c[4] for c in STREAM_CASES])
def test_stream_shapes(ctx, tune, qtype, cols, rows, layout, name):
    """The streaming instance forced (NS_GEMV_PF=1) on shapes from one slab to a
    ragged row-major lm-head, with fewer super-blocks per slab than waves."""
    tune("gemv_pf", "1")
    host, w = weights(qtype, 31, rows, cols, layout)
    x = f32(cols, 32)
    ref = O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, x)
    assert rel_err(_run(ctx, qtype, w, layout, cols, rows, x), ref) <= TOL32


def test_stream_gate_up_pair(ctx, tune):
    tune("gemv_pf", "1")
    cols, rows = 3840, 15360
    hg, wg = weights(N.Q4_K, 21, rows, cols, N.CDNA4)
    hu, wu = weights(N.Q4_K, 22, rows, cols, N.CDNA4)
    x = f32(cols, 23)
    ref = O.gate_up_geglu(O.ROW_MAJOR, hg, hu, cols, rows, x)
    h = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.gate_up_geglu_decode(wg, wu, N.CDNA4, cols, rows, torch.from_numpy(x).cuda(), h)
    torch.cuda.synchronize()
    assert rel_err(h.cpu().numpy(), ref) <= TOL32


def test_gemv_deterministic(ctx):
    cols, rows = 15360, 3840
    _, w = weights(N.Q6_K, 11, rows, cols, N.CDNA4)
    x = torch.from_numpy(f32(cols, 12)).cuda()
    ys = []
    for _ in range(3):
        y = torch.empty(rows, dtype=torch.float32, device="cuda")
        ctx.matmul(w, N.Q6_K, N.CDNA4, cols, rows, 1, x, y)
        ys.append(y)
    torch.cuda.synchronize()
    assert all(torch.equal(ys[0], t) for t in ys[1:])


@pytest.mark.parametrize("layout", LAYOUTS, ids=LNAME.get)
def test_gate_up_geglu_decode(ctx, layout):
    cols, rows = 3840, 15360
    hg, wg = weights(N.Q4_K, 21, rows, cols, layout)
    hu, wu = weights(N.Q4_K, 22, rows, cols, layout)
    x = f32(cols, 23)
    h = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.gate_up_geglu_decode(wg, wu, layout, cols, rows, torch.from_numpy(x).cuda(), h)
    torch.cuda.synchronize()
    ref = O.gate_up_geglu(O.ROW_MAJOR, hg, hu, cols, rows, x)
    assert rel_err(h.cpu().numpy(), ref) <= TOL32


def test_ffn_block_decode_two_layers(ctx):
    """Config 2 for two seeded layers: gate/up+GeGLU then the Q6_K down GEMV,
    each layer's output compared with the oracle fed the same input."""
    D, F = 3840, 15360
    x = f32(D, 31)
    for layer in range(2):
        s = N.layer_seed(1000, layer)
        hg, wg = weights(N.Q4_K, s + 1, F, D, N.CDNA4)
        hu, wu = weights(N.Q4_K, s + 2, F, D, N.CDNA4)
        hd, wd = weights(N.Q6_K, s + 3, D, F, N.CDNA4)
        xd = torch.from_numpy(x).cuda()
        h = torch.empty(F, dtype=torch.float32, device="cuda")
        y = torch.empty(D, dtype=torch.float32, device="cuda")
        ctx.gate_up_geglu_decode(wg, wu, N.CDNA4, D, F, xd, h)
        ctx.ffn_down(wd, N.Q6_K, N.CDNA4, F, D, 1, h, y, half_input=False, fast_swa=False)
        torch.cuda.synchronize()
        h_ref = O.gate_up_geglu(O.ROW_MAJOR, hg, hu, D, F, x)
        assert rel_err(h.cpu().numpy(), h_ref) <= TOL32
        y_ref = O.gemv(N.Q6_K, O.ROW_MAJOR, hd, F, D, h.cpu().numpy())
        yg = y.cpu().numpy()
        assert rel_err(yg, y_ref) <= TOL32
        x = (yg / np.sqrt(np.mean(yg.astype(np.float64) ** 2))).astype(np.float32)


# ---- prefill GEMM ---------------------------------------------------------------

PREFILL_SMALL = [(512, 128, 5), (1024, 192, 33), (768, 128, 200), (256, 64, 2)]


@pytest.mark.parametrize("layout", [N.CDNA4, N.NSMFFN], ids=LNAME.get)
@pytest.mark.parametrize("acc", [N.ACC_FP32, N.ACC_FP16], ids=["fp32acc", "fp16acc"])
@pytest.mark.parametrize("cols,rows,batch", PREFILL_SMALL)
def test_prefill_gate_up_small(ctx, cols, rows, batch, acc, layout):
    hg, wg = weights(N.Q4_K, 41, rows, cols, layout)
    hu, wu = weights(N.Q4_K, 42, rows, cols, layout)
    x = N.synth_normal_f16(43, batch * cols).reshape(batch, cols)
    h = torch.empty((batch, rows), dtype=torch.int16, device="cuda")
    ctx.gate_up_geglu_rm32(wg, wu, layout, cols, rows, batch, dev_u16(x), h, fast_swa=(acc == N.ACC_FP16))
    torch.cuda.synchronize()
    got = f16_value(h.cpu().numpy().view(np.uint16))
    ref32 = O.gate_up_geglu_prefill(O.ROW_MAJOR, hg, hu, cols, rows, batch, x, 0)
    assert rel_err(got, ref32) <= (TOL32 if acc == N.ACC_FP32 else TOL16)
    if acc == N.ACC_FP16:
        ref16 = O.gate_up_geglu_prefill(O.ROW_MAJOR, hg, hu, cols, rows, batch, x, 1)
        assert rel_err(got, ref16) <= TOL16_SAME_PAIR


@pytest.mark.parametrize("layout", [N.CDNA4, N.NSMFFN], ids=LNAME.get)
@pytest.mark.parametrize("acc", [N.ACC_FP32, N.ACC_FP16], ids=["fp32acc", "fp16acc"])
@pytest.mark.parametrize("qtype", [N.Q6_K, N.Q4_K], ids=["q6k", "q4k"])
@pytest.mark.parametrize("cols,rows,batch", PREFILL_SMALL)
def test_prefill_down_small(ctx, cols, rows, batch, qtype, acc, layout):
    hw, w = weights(qtype, 51, rows, cols, layout)
    x = N.synth_normal_f16(52, batch * cols).reshape(batch, cols)
    y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    ctx.ffn_down(w, qtype, layout, cols, rows, batch, dev_u16(x), y, half_input=True,
                 fast_swa=(acc == N.ACC_FP16))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref32 = O.gemm(qtype, O.ROW_MAJOR, hw, cols, rows, batch, x, 0)
    if batch <= 4:
        # mm:289: fp16 input at batch <= 4 goes to matmul's small-batch kernels, FP32 in both modes
        assert rel_err(got, ref32) <= TOL32
        return
    assert rel_err(got, ref32) <= (TOL32 if acc == N.ACC_FP32 else TOL16)
    if acc == N.ACC_FP16:
        assert not np.any(got.view(np.uint32) & 0x1FFF)  # fp16 precision: 11 significant bits
        ref16 = O.gemm(qtype, O.ROW_MAJOR, hw, cols, rows, batch, x, 1)
        assert rel_err(got, ref16) <= TOL16_SAME


# Forced split-K: every part count path of both Q4_K kernels (register-fragment,
# LDS-tile) and the Q6_K kernel, on ragged token and row tiles.  Parts of 1 or 2
# super-blocks each; the last workgroup of a tile adds them in part order.
SPLIT_CASES = [("q4k-reg", N.Q4_K, "1"), ("q4k-lds", N.Q4_K, "0"), ("q6k-lds", N.Q6_K, "1")]


@pytest.mark.parametrize("kparts", ["3", "5"])
@pytest.mark.parametrize("acc", [N.ACC_FP32, N.ACC_FP16], ids=["fp32acc", "fp16acc"])
@pytest.mark.parametrize("name,qtype,reg", SPLIT_CASES, ids=[c[0] for c in SPLIT_CASES])
def test_prefill_split_k(ctx, tune, name, qtype, reg, acc, kparts):
    tune("gemm_kparts", kparts)
    tune("gemm_q4_reg", reg)
    cols, rows, batch = 2048, 320, 200
    fast = acc == N.ACC_FP16
    tol = TOL16 if fast else TOL32
    x = N.synth_normal_f16(71, batch * cols).reshape(batch, cols)
    hw, w = weights(qtype, 72, rows, cols, N.CDNA4)
    y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    ctx.ffn_down(w, qtype, N.CDNA4, cols, rows, batch, dev_u16(x), y, half_input=True, fast_swa=fast)
    if qtype == N.Q4_K:
        hu, wu = weights(N.Q4_K, 73, rows, cols, N.CDNA4)
        h = torch.empty((batch, rows), dtype=torch.int16, device="cuda")
        ctx.gate_up_geglu_rm32(w, wu, N.CDNA4, cols, rows, batch, dev_u16(x), h, fast_swa=fast)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert rel_err(got, O.gemm(qtype, O.ROW_MAJOR, hw, cols, rows, batch, x, 0)) <= tol
    if fast:
        assert not np.any(got.view(np.uint32) & 0x1FFF)
        assert rel_err(got, O.gemm(qtype, O.ROW_MAJOR, hw, cols, rows, batch, x, 1)) <= 4e-3
    if qtype == N.Q4_K:
        hh = f16_value(h.cpu().numpy().view(np.uint16))
        assert rel_err(hh, O.gate_up_geglu_prefill(O.ROW_MAJOR, hw, hu, cols, rows, batch, x, 0)) <= tol


def _row_slice(host, qtype, cols, r0, nrows):
    bpr = (cols // 256) * N.BLOCK_BYTES[qtype]
    return np.ascontiguousarray(host[r0 * bpr:(r0 + nrows) * bpr])


@pytest.mark.parametrize("layout", [N.CDNA4, N.ROW_MAJOR], ids=LNAME.get)
@pytest.mark.parametrize("qtype", [N.Q6_K, N.Q4_K], ids=["q6k", "q4k"])
@pytest.mark.parametrize("batch", [5, 64, 300])
def test_matmul_fp32_input_above_batch4(ctx, batch, qtype, layout):
    """mm:274: fp32 input above batch 4 takes the MMA GEMM, whose tile loader rounds each x value
    to half (metal:235).  The result equals the fp16-input call on x rounded to nearest even (numpy's
    float16 conversion) bit for bit, and is within the FP32 bar of the oracle's GEMM on those
    values."""
    cols, rows = 1024, 320
    hw, w = weights(qtype, 81 + batch, rows, cols, layout)
    x = N.synth_normal_f32(82 + batch, batch * cols).reshape(batch, cols)
    xh = x.astype(np.float16)
    y32 = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
    y16 = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
    ctx.matmul(w, qtype, layout, cols, rows, batch, torch.from_numpy(x).cuda(), y32)
    ctx.matmul(w, qtype, layout, cols, rows, batch, dev_u16(xh.view(np.uint16)), y16, half_input=True)
    torch.cuda.synchronize()
    got = y32.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), y16.cpu().numpy().view(np.uint32))
    assert rel_err(got, O.gemm(qtype, O.ROW_MAJOR, hw, cols, rows, batch, xh.view(np.uint16), 0)) <= TOL32


@pytest.mark.parametrize("acc", [N.ACC_FP32, N.ACC_FP16], ids=["fp32acc", "fp16acc"])
def test_prefill_ffn_full_size(ctx, acc):
    """Config 3 at full size (batch 1024, 3840 -> 15360 -> 3840).  The GPU runs
    the whole block; the oracle checks 128-row samples of H and of Y (the down
    check feeds the oracle the GPU's fp16 H, isolating each GEMM)."""
    D, F, B = 3840, 15360, 1024
    hg, wg = weights(N.Q4_K, 61, F, D, N.CDNA4)
    hu, wu = weights(N.Q4_K, 62, F, D, N.CDNA4)
    hd, wd = weights(N.Q6_K, 63, D, F, N.CDNA4)
    x = N.synth_normal_f16(64, B * D).reshape(B, D)
    h = torch.empty((B, F), dtype=torch.int16, device="cuda")
    y = torch.empty((B, D), dtype=torch.float32, device="cuda")
    fast = acc == N.ACC_FP16
    ctx.gate_up_geglu_rm32(wg, wu, N.CDNA4, D, F, B, dev_u16(x), h, fast_swa=fast)
    ctx.ffn_down(wd, N.Q6_K, N.CDNA4, F, D, B, h, y, half_input=True, fast_swa=fast)
    torch.cuda.synchronize()
    hh = h.cpu().numpy().view(np.uint16)
    yy = y.cpu().numpy()
    assert np.isfinite(f16_value(hh)).all() and np.isfinite(yy).all()
    tol = TOL32 if acc == N.ACC_FP32 else TOL16
    for r0 in (0, 7040, F - 128):
        gs, us = _row_slice(hg, N.Q4_K, D, r0, 128), _row_slice(hu, N.Q4_K, D, r0, 128)
        ref = O.gate_up_geglu_prefill(O.ROW_MAJOR, gs, us, D, 128, B, x, 0)
        assert rel_err(f16_value(hh[:, r0:r0 + 128]), ref) <= tol
        if fast:
            ref16 = O.gate_up_geglu_prefill(O.ROW_MAJOR, gs, us, D, 128, B, x, 1)
            assert rel_err(f16_value(hh[:, r0:r0 + 128]), ref16) <= TOL16_SAME_PAIR
    for r0 in (0, 1984, D - 128):
        ds = _row_slice(hd, N.Q6_K, F, r0, 128)
        ref = O.gemm(N.Q6_K, O.ROW_MAJOR, ds, F, 128, B, hh, 0)
        assert rel_err(yy[:, r0:r0 + 128], ref) <= tol
        if fast:
            assert rel_err(yy[:, r0:r0 + 128], O.gemm(N.Q6_K, O.ROW_MAJOR, ds, F, 128, B, hh, 1)) <= TOL16_SAME


@pytest.mark.parametrize("acc", [N.ACC_FP32, N.ACC_FP16], ids=["fp32acc", "fp16acc"])
def test_prefill_q4k_down_full_size(ctx, acc):
    """The Q4_K down projection of the Q4_K_M mix (odd layers of config 4) at full size:
    15360 -> 3840 at batch 1024, 128-row samples against the oracle in the same mode."""
    D, F, B = 3840, 15360, 1024
    hd, wd = weights(N.Q4_K, 65, D, F, N.CDNA4)
    x = N.synth_normal_f16(66, B * F).reshape(B, F)
    y = torch.empty((B, D), dtype=torch.float32, device="cuda")
    fast = acc == N.ACC_FP16
    ctx.ffn_down(wd, N.Q4_K, N.CDNA4, F, D, B, dev_u16(x), y, half_input=True, fast_swa=fast)
    torch.cuda.synchronize()
    yy = y.cpu().numpy()
    assert np.isfinite(yy).all()
    for r0 in (0, 1984, D - 128):
        ds = _row_slice(hd, N.Q4_K, F, r0, 128)
        assert rel_err(yy[:, r0:r0 + 128], O.gemm(N.Q4_K, O.ROW_MAJOR, ds, F, 128, B, x, 0)) <= (TOL16 if fast else TOL32)
        if fast:
            assert rel_err(yy[:, r0:r0 + 128], O.gemm(N.Q4_K, O.ROW_MAJOR, ds, F, 128, B, x, 1)) <= TOL16_SAME


@pytest.mark.parametrize("acc", [N.ACC_FP32, N.ACC_FP16], ids=["fp32acc", "fp16acc"])
@pytest.mark.parametrize("batch", [512, 256])
def test_prefill_q6k_down_many_parts(ctx, batch, acc):
    """The down projection below batch 1024 splits K into 8 parts (fewer token tiles): the
    last workgroup adds them four at a time.  128-row samples against the oracle in the same
    mode, and the values do not depend on the part count beyond fp32 rounding (kparts 4)."""
    D, F = 3840, 15360
    hd, wd = weights(N.Q6_K, 67, D, F, N.CDNA4)
    x = N.synth_normal_f16(68, batch * F).reshape(batch, F)
    fast = acc == N.ACC_FP16
    y = torch.empty((batch, D), dtype=torch.float32, device="cuda")
    ctx.ffn_down(wd, N.Q6_K, N.CDNA4, F, D, batch, dev_u16(x), y, half_input=True, fast_swa=fast)
    torch.cuda.synchronize()
    yy = y.cpu().numpy()
    assert np.isfinite(yy).all()
    for r0 in (0, D - 128):
        ds = _row_slice(hd, N.Q6_K, F, r0, 128)
        ref = O.gemm(N.Q6_K, O.ROW_MAJOR, ds, F, 128, batch, x, 1 if fast else 0)
        assert rel_err(yy[:, r0:r0 + 128], ref) <= (TOL16_SAME if fast else TOL32)


# ---- device layout conversion and argument errors -------------------------------

@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
def test_retile_device_matches_host(ctx, qtype):
    cols, rows = 768, 192
    host = N.synth_weights(qtype, 71, rows, cols)
    src = dev_bytes(host)
    for to in (N.NSMFFN, N.CDNA4):
        dst = torch.empty_like(src)
        N.retile_device(src, dst, qtype, cols, rows, N.ROW_MAJOR, to)
        torch.cuda.synchronize()
        assert np.array_equal(dst.cpu().numpy(), N.retile(host, qtype, cols, rows, N.ROW_MAJOR, to))


def test_argument_errors(ctx):
    _, w = weights(N.Q4_K, 81, 64, 256, N.CDNA4)
    x = torch.zeros(256, dtype=torch.float32, device="cuda")
    y = torch.zeros(64, dtype=torch.float32, device="cuda")
    with pytest.raises(N.NsError) as e:
        ctx.matmul(w, N.Q4_K, N.CDNA4, 300, 64, 1, x, y)
    assert e.value.code == 2
    with pytest.raises(N.NsError) as e:
        ctx.matmul(w[1:], N.Q4_K, N.CDNA4, 256, 64, 1, x, y)
    assert "misaligned" in str(e.value)
    with pytest.raises(N.NsError) as e:  # fp16 input at batch 1 is no regime of matmul (mm:269-275)
        ctx.matmul(w, N.Q4_K, N.CDNA4, 256, 64, 1, x, y, half_input=True)
    assert e.value.code == 4


# ---- the reference's own values on the GPU ----------------------------------------------

@pytest.mark.parametrize("layout", LAYOUTS, ids=LNAME.get)
@pytest.mark.parametrize("name,qtype", [("q4k", N.Q4_K), ("q6k", N.Q6_K)])
def test_golden_vectors_on_gpu(ctx, name, qtype, layout):
    """tests/golden/quant_golden.npz holds values and dot_row results written by the reference's
    own quant.cpp (oracle/_ref): seeded blocks plus extremes (zero and maximal scales, fp16-
    subnormal d, sc = -32).  The GPU's dequant must equal the values bit for bit and its GEMV
    must be within the FP32 bar of the reference's dots.  Slab layouts get the 2 golden rows
    padded to one 64-row slab with zero blocks."""
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "quant_golden.npz"))
    cols, rows = (int(v) for v in z[f"{name}_shape"])
    raw = z[f"{name}_bytes"]
    bb = 144 if qtype == N.Q4_K else 210
    prow = rows if layout == N.ROW_MAJOR else 64
    host = np.zeros(prow * (cols // 256) * bb, dtype=np.uint8)
    host[:raw.size] = raw
    img = host if layout == N.ROW_MAJOR else N.retile(host, qtype, cols, prow, N.ROW_MAJOR, layout)
    w = torch.from_numpy(np.ascontiguousarray(img)).cuda()
    out = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    ctx.dequant(w, qtype, layout, cols, prow, 0, rows, out_f32=out)
    y = torch.empty(prow, dtype=torch.float32, device="cuda")
    ctx.matmul(w, qtype, layout, cols, prow, 1, torch.from_numpy(z[f"{name}_x"]).cuda(), y)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().reshape(-1).view(np.uint32), z[f"{name}_values"].view(np.uint32))
    dots = z[f"{name}_dot"].astype(np.float64)
    got = y.cpu().numpy()[:rows].astype(np.float64)
    assert np.max(np.abs(got - dots)) <= TOL32 * np.max(np.abs(dots))
