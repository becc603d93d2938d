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
from helpers import f16_value, rel_err

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
