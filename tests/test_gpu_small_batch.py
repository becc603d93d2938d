"""GPU parity tests of the batch 2-4 regime (MTP verification): matmul, ffn_down
and gate_up_geglu stream the weights once for every token (metal:102-177;
dispatch at metal_engine.mm:273, :282).  Each token's output is checked against
the oracle's GEMV of that token (fp16 inputs enter the oracle as their exact
fp32 values); FP32 accumulation, rel_err <= 1e-3.
"""
import numpy as np
import pytest

import ns_oracle as O
import nsffn as N
from helpers import f16_value, q6k_block, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL32 = 1e-3
LNAME = {N.CDNA4: "cdna4", N.NSMFFN: "nsmffn", N.ROW_MAJOR: "rowmajor"}


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = N.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def weights(qtype, seed, rows, cols, layout):
    host = N.synth_weights(qtype, seed, rows, cols)
    lay = host if layout == N.ROW_MAJOR else N.retile(host, qtype, cols, rows, N.ROW_MAJOR, layout)
    return host, torch.from_numpy(np.ascontiguousarray(lay)).cuda()


def tokens(seed, batch, cols, half):
    """(device input, the fp32 values the oracle multiplies)."""
    if half:
        bits = N.synth_normal_f16(seed, batch * cols).reshape(batch, cols)
        return torch.from_numpy(bits.view(np.int16)).cuda(), f16_value(bits).astype(np.float32)
    x = N.synth_normal_f32(seed, batch * cols).reshape(batch, cols)
    return torch.from_numpy(x).cuda(), x


@pytest.mark.parametrize("half", [False, True], ids=["f32in", "f16in"])
@pytest.mark.parametrize("batch", [2, 3, 4])
@pytest.mark.parametrize("layout", [N.CDNA4, N.NSMFFN, N.ROW_MAJOR], ids=LNAME.get)
@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
def test_matmul_small_batch(ctx, qtype, layout, batch, half):
    cols = 1024
    rows = 200 if layout == N.ROW_MAJOR else 192  # ragged last slab in the row-major layout
    host, w = weights(qtype, 90 + batch, rows, cols, layout)
    xd, xf = tokens(91 + batch, batch, cols, half)
    y = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
    ctx.matmul(w, qtype, layout, cols, rows, batch, xd, y, half_input=half)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    for t in range(batch):
        assert rel_err(got[t], O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, xf[t])) <= TOL32, t


@pytest.mark.parametrize("batch", [1, 2, 3, 4])
@pytest.mark.parametrize("layout", [N.CDNA4, N.NSMFFN, N.ROW_MAJOR], ids=LNAME.get)
def test_gate_up_geglu_small_batch(ctx, layout, batch):
    cols = 768
    rows = 136 if layout == N.ROW_MAJOR else 128
    hg, wg = weights(N.Q4_K, 95, rows, cols, layout)
    hu, wu = weights(N.Q4_K, 96, rows, cols, layout)
    xd, xf = tokens(97 + batch, batch, cols, True)
    h = torch.zeros((batch, rows), dtype=torch.int16, device="cuda")
    ctx.gate_up_geglu(wg, wu, layout, cols, rows, batch, xd, h)
    torch.cuda.synchronize()
    got = f16_value(h.cpu().numpy().view(np.uint16))
    for t in range(batch):
        assert rel_err(got[t], O.gate_up_geglu(O.ROW_MAJOR, hg, hu, cols, rows, xf[t])) <= TOL32, t


def test_ffn_down_small_batch_half_input(ctx):
    """ffn_down with fp16 input and batch 3 takes matmul's small-batch path (mm:289)."""
    cols, rows, batch = 2048, 256, 3
    host, w = weights(N.Q6_K, 98, rows, cols, N.CDNA4)
    xd, xf = tokens(99, batch, cols, True)
    y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    ctx.ffn_down(w, N.Q6_K, N.CDNA4, cols, rows, batch, xd, y, half_input=True, fast_swa=True)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    for t in range(batch):
        assert rel_err(got[t], O.gemv(N.Q6_K, O.ROW_MAJOR, host, cols, rows, xf[t])) <= TOL32, t


def _row_slice(host, qtype, cols, r0, nrows):
    bpr = (cols // 256) * N.BLOCK_BYTES[qtype]
    return np.ascontiguousarray(host[r0 * bpr:(r0 + nrows) * bpr])


def test_lm_head_batch4(ctx):
    """The full 262144-row Q6_K lm-head for 4 fp32 tokens (MTP verification of 3
    drafted tokens): sampled rows against the oracle, and every row against four
    single-token GEMVs of the same kernel family (same per-token FMA order)."""
    D, V, B = 3840, 262144, 4
    host, w = weights(N.Q6_K, 0x1B, V, D, N.CDNA4)
    xd, xf = tokens(0x1C, B, D, False)
    y = torch.empty((B, V), dtype=torch.float32, device="cuda")
    ctx.matmul(w, N.Q6_K, N.CDNA4, D, V, B, xd, y)
    y1 = torch.empty((B, V), dtype=torch.float32, device="cuda")
    for t in range(B):
        ctx.matmul(w, N.Q6_K, N.CDNA4, D, V, 1, xd[t], y1[t])
    torch.cuda.synchronize()
    got, single = y.cpu().numpy(), y1.cpu().numpy()
    for t in range(B):
        assert rel_err(got[t], single[t]) <= 1e-5, t
    for r0 in (0, 131072 - 64, V - 128):
        sl = _row_slice(host, N.Q6_K, D, r0, 128)
        for t in range(B):
            assert rel_err(got[t, r0:r0 + 128], O.gemv(N.Q6_K, O.ROW_MAJOR, sl, D, 128, xf[t])) <= TOL32, (r0, t)


# ---- the MFMA form (ns_gemv_mfma.hip, CDNA4 layout; mt_mfma = 0 selects the VALU kernel) ----

def _both_kernels(ctx, tune, fn):
    """fn() run on the MFMA kernel and on the VALU kernel (host copies)."""
    a = fn()
    tune("mt_mfma", 0)
    b = fn()
    tune("mt_mfma", 1)
    return a, b


@pytest.mark.parametrize("half", [False, True], ids=["f32in", "f16in"])
@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
def test_mfma_matches_valu_kernel_full_size(ctx, tune, qtype, half):
    """Full-size shapes of the model (15360 x 3840 and the 60-block down, which splits its
    columns over four workgroups), batch 3: the MFMA form against the oracle and within
    1e-5 of the VALU kernel, whose per-token FMA order is the single-token GEMV's."""
    for rows, cols in ((15360, 3840), (3840, 15360)):
        host, w = weights(qtype, 0x5A + rows % 7, rows, cols, N.CDNA4)
        xd, xf = tokens(0x5B, 3, cols, half)

        def run():
            y = torch.full((3, rows), float("nan"), dtype=torch.float32, device="cuda")
            ctx.matmul(w, qtype, N.CDNA4, cols, rows, 3, xd, y, half_input=half)
            torch.cuda.synchronize()
            return y.cpu().numpy()
        got, valu = _both_kernels(ctx, tune, run)
        assert rel_err(got, valu) <= 1e-5, (rows, cols)
        for t in range(3):
            sl = _row_slice(host, qtype, cols, rows - 128, 128)
            assert rel_err(got[t, rows - 128:], O.gemv(qtype, O.ROW_MAJOR, sl, cols, 128, xf[t])) <= TOL32, (rows, t)


@pytest.mark.parametrize("parts", [1, 2, 3, 5])
def test_mfma_column_parts(ctx, tune, parts):
    """Every column split of one workgroup (and four workgroups per slab for the 60-block
    down) gives the oracle's values: the gate/up pair and the Q6_K down at batch 4."""
    tune("mt_parts", parts)
    cols, rows = 3840, 256
    hg, wg = weights(N.Q4_K, 0x61, rows, cols, N.CDNA4)
    hu, wu = weights(N.Q4_K, 0x62, rows, cols, N.CDNA4)
    xd, xf = tokens(0x63, 4, cols, True)
    h = torch.zeros((4, rows), dtype=torch.int16, device="cuda")
    ctx.gate_up_geglu(wg, wu, N.CDNA4, cols, rows, 4, xd, h)
    hd, w6 = weights(N.Q6_K, 0x64, 256, 15360, N.CDNA4)
    xd6, xf6 = tokens(0x65, 4, 15360, True)
    y = torch.empty((4, 256), dtype=torch.float32, device="cuda")
    ctx.ffn_down(w6, N.Q6_K, N.CDNA4, 15360, 256, 4, xd6, y, half_input=True, fast_swa=False)
    torch.cuda.synchronize()
    got = f16_value(h.cpu().numpy().view(np.uint16))
    yg = y.cpu().numpy()
    for t in range(4):
        assert rel_err(got[t], O.gate_up_geglu(O.ROW_MAJOR, hg, hu, cols, rows, xf[t])) <= TOL32, t
        assert rel_err(yg[t], O.gemv(N.Q6_K, O.ROW_MAJOR, hd, 15360, 256, xf6[t])) <= TOL32, t


def test_mfma_q6k_full_range_scales(ctx):
    """Real Q6_K tensors carry int8 scales up to +-127 (the synthetic ones stay in -32..31):
    every scale and every 6-bit value at its extremes, against the oracle."""
    cols, rows = 1024, 128
    rng = np.random.default_rng(0x66)
    nb = rows * cols // 256
    blocks = []
    for i in range(nb):
        sc = rng.integers(-128, 128, 16)
        sc[i % 16] = -128 if i % 2 else 127
        v = rng.integers(0, 64, 256)
        v[:8] = 63
        v[8:16] = 0
        blocks.append(q6k_block(np.float16(rng.uniform(1e-4, 2e-3)), sc, v))
    host = np.concatenate(blocks)
    w = torch.from_numpy(N.retile(host, N.Q6_K, cols, rows, N.ROW_MAJOR, N.CDNA4)).cuda()
    for half in (False, True):
        xd, xf = tokens(0x67, 4, cols, half)
        y = torch.empty((4, rows), dtype=torch.float32, device="cuda")
        ctx.matmul(w, N.Q6_K, N.CDNA4, cols, rows, 4, xd, y, half_input=half)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        for t in range(4):
            assert rel_err(got[t], O.gemv(N.Q6_K, O.ROW_MAJOR, host, cols, rows, xf[t])) <= TOL32, (half, t)


@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
def test_mfma_fp32_tokens_beyond_fp16_range(ctx, qtype):
    """fp32 tokens far outside fp16's range (|x| up to 3e7, one token tiny): the per-token
    power-of-two scale keeps the fp16 split exact in range; values against the oracle."""
    cols, rows = 1024, 192
    host, w = weights(qtype, 0x68, rows, cols, N.CDNA4)
    x = N.synth_normal_f32(0x69, 4 * cols).reshape(4, cols).copy()
    x[0] *= 3e5
    x[1, 5] = 3e7
    x[2] *= 1e-6
    xd = torch.from_numpy(x).cuda()
    y = torch.empty((4, rows), dtype=torch.float32, device="cuda")
    ctx.matmul(w, qtype, N.CDNA4, cols, rows, 4, xd, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    for t in range(4):
        assert rel_err(got[t], O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, x[t])) <= TOL32, t


@pytest.mark.parametrize("down_type", [N.Q6_K, N.Q4_K], ids=["q6down", "q4down"])
@pytest.mark.parametrize("batch", [2, 4])
def test_ffn_block_decode_small_batch_full_size(ctx, batch, down_type):
    """The FFN block at decode with 2-4 fp32 tokens, at the model's shape (3840 x 15360, CDNA4):
    matmul(gate) and matmul(up) each stream their weights once for every token, gemma_geglu
    forms h, then the down projection's small-batch kernel (mm:570-573).  Per token, h against
    the oracle's gate/up GeGLU and y against the oracle's GEMV of that h, FP32 bar 1e-3."""
    D, F = 3840, 15360
    hg, wg = weights(N.Q4_K, 0x70 + batch, F, D, N.CDNA4)
    hu, wu = weights(N.Q4_K, 0x71 + batch, F, D, N.CDNA4)
    hd, wd = weights(down_type, 0x72 + batch, D, F, N.CDNA4)
    xd, xf = tokens(0x73 + batch, batch, D, False)
    mid = torch.full((batch, F), float("nan"), dtype=torch.float32, device="cuda")
    out = torch.full((batch, D), float("nan"), dtype=torch.float32, device="cuda")
    ctx.ffn_block(wg, wu, wd, down_type, N.CDNA4, D, F, batch, xd.reshape(-1), mid.reshape(-1), out.reshape(-1),
                  prefill=False, swa=True)
    ctx.status()
    h = mid.cpu().numpy()
    y = out.cpu().numpy()
    for t in range(batch):
        assert rel_err(h[t], O.gate_up_geglu(O.ROW_MAJOR, hg, hu, D, F, xf[t])) <= TOL32, t
        assert rel_err(y[t], O.gemv(down_type, O.ROW_MAJOR, hd, F, D, h[t])) <= TOL32, t


def test_geglu_elementwise(ctx):
    """ns_geglu (gemma_geglu / _f16, metal:530-531) against the oracle's GeGLU per element, on a
    ragged count; fp32 out within 1e-5 of the oracle (the row-max relative error), fp16 out the
    round-to-nearest-even of the fp32 value."""
    n = 15360 * 3 + 5
    g = N.synth_normal_f32(0x80, n) * 3
    u = N.synth_normal_f32(0x81, n)
    gd, ud = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    y = torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")
    yh = torch.zeros((n,), dtype=torch.int16, device="cuda")
    ctx.geglu(gd, ud, n, y)
    ctx.geglu(gd, ud, n, yh, half_out=True)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = np.array([O.gelu_tanh(float(v)) for v in g], dtype=np.float32) * u
    assert rel_err(got, ref) <= 1e-5
    assert np.array_equal(yh.cpu().numpy().view(np.uint16), got.astype(np.float16).view(np.uint16))
