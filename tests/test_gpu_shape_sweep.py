"""Seeded sweep of irregular shapes through every regime, against the CPU oracle.

The fixed-shape parity tests follow BASELINE's configs.  This sweep draws shapes
that those do not reach: one super-block per row, super-block counts that are
prime or just past a power of two, one to 130 slabs, ragged last slabs in the
row-major layout (the only layout without the 64-row rule, metal_ffn.cpp:74).
Each shape runs through the decode GEMV (both kernel instances, and the
planner's own choice), the batch 2-4 kernels (fp32 and fp16 tokens) and the
prefill GEMM (both accumulation modes).  Bars as in test_gpu_parity.py: FP32
accumulation rel_err <= 1e-3, FP16 accumulation <= 1e-2.
"""
import numpy as np
import pytest

import ns_oracle as O
import nsffn as N
from helpers import f16_value, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL32, TOL16 = 1e-3, 1e-2
LAYOUTS = [N.CDNA4, N.NSMFFN, N.ROW_MAJOR]
LNAME = {N.CDNA4: "cdna4", N.NSMFFN: "nsmffn", N.ROW_MAJOR: "rowmajor"}
QNAME = {N.Q4_K: "q4k", N.Q6_K: "q6k"}


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        qtype = [N.Q4_K, N.Q6_K][int(rng.integers(2))]
        layout = LAYOUTS[int(rng.integers(3))]
        nb = int(rng.choice([1, 2, 3, 5, 7, 15, 16, 17, 33, 60]))
        nslab = int(rng.choice([1, 2, 3, 5, 9, 17, 40, 130]))
        rows = nslab * 64
        if layout == N.ROW_MAJOR and nslab > 1 and rng.random() < 0.7:
            rows -= int(rng.integers(1, 64))
        out.append((qtype, layout, nb * 256, rows))
    return out


CASES = _cases(24, 2026)
IDS = [f"{QNAME[q]}-{LNAME[l]}-{c}x{r}" for q, l, c, r in CASES]


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = N.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def _weights(qtype, seed, rows, cols, layout):
    host = N.synth_weights(qtype, seed, rows, cols)
    lay = host if layout == N.ROW_MAJOR else N.retile(host, qtype, cols, rows, N.ROW_MAJOR, layout)
    return host, torch.from_numpy(np.ascontiguousarray(lay)).cuda()


@pytest.mark.parametrize("qtype,layout,cols,rows", CASES, ids=IDS)
def test_gemv_sweep(ctx, tune, qtype, layout, cols, rows):
    host, w = _weights(qtype, 300 + rows, rows, cols, layout)
    x = N.synth_normal_f32(301 + cols, cols)
    ref = O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, x)
    xd = torch.from_numpy(x).cuda()
    for pf in (None, "0", "1"):  # the planner's choice, one unit per wave, streaming
        if pf is None:
            tune("gemv_pf", -1)
        else:
            tune("gemv_pf", pf)
        y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
        ctx.matmul(w, qtype, layout, cols, rows, 1, xd, y)
        torch.cuda.synchronize()
        assert rel_err(y.cpu().numpy(), ref) <= TOL32, pf


@pytest.mark.parametrize("qtype,layout,cols,rows", CASES[:12], ids=IDS[:12])
def test_small_batch_sweep(ctx, qtype, layout, cols, rows):
    host, w = _weights(qtype, 310 + rows, rows, cols, layout)
    for batch, half in ((2, True), (3, False), (4, True), (4, False)):
        if half:
            bits = N.synth_normal_f16(311 + batch, batch * cols).reshape(batch, cols)
            xd = torch.from_numpy(bits.view(np.int16)).cuda()
            xf = f16_value(bits).astype(np.float32)
        else:
            xf = N.synth_normal_f32(312 + batch, batch * cols).reshape(batch, cols)
            xd = torch.from_numpy(xf).cuda()
        y = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
        ctx.matmul(w, qtype, layout, cols, rows, batch, xd, y, half_input=half)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        for t in range(batch):
            assert rel_err(got[t], O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, xf[t])) <= TOL32, (batch, t)


@pytest.mark.parametrize("qtype,layout,cols,rows", CASES[12:], ids=IDS[12:])
def test_prefill_sweep(ctx, qtype, layout, cols, rows):
    host, w = _weights(qtype, 320 + rows, rows, cols, layout)
    for batch in (5, 37):
        x = N.synth_normal_f16(321 + batch, batch * cols).reshape(batch, cols)
        xd = torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()
        for fast in (False, True):
            y = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
            ctx.ffn_down(w, qtype, layout, cols, rows, batch, xd, y, half_input=True, fast_swa=fast)
            torch.cuda.synchronize()
            got = y.cpu().numpy()
            ref = O.gemm(qtype, O.ROW_MAJOR, host, cols, rows, batch, x, 1 if fast else 0)
            assert rel_err(got, ref) <= (TOL16 if fast else TOL32), (batch, fast)


@pytest.mark.parametrize("layout,cols,rows", [(l, c, r) for q, l, c, r in CASES[:8]],
                         ids=[f"{LNAME[l]}-{c}x{r}" for q, l, c, r in CASES[:8]])
def test_gate_up_sweep(ctx, layout, cols, rows):
    """The Q4_K gate/up pair with GeGLU at batch 1 (decode), 3 and 37 (prefill, FP32 mode)."""
    hg, wg = _weights(N.Q4_K, 330 + rows, rows, cols, layout)
    hu, wu = _weights(N.Q4_K, 331 + rows, rows, cols, layout)
    x1 = N.synth_normal_f32(332, cols)
    h1 = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.gate_up_geglu_decode(wg, wu, layout, cols, rows, torch.from_numpy(x1).cuda(), h1)
    torch.cuda.synchronize()
    assert rel_err(h1.cpu().numpy(), O.gate_up_geglu(O.ROW_MAJOR, hg, hu, cols, rows, x1)) <= TOL32
    for batch in (3, 37):
        x = N.synth_normal_f16(333 + batch, batch * cols).reshape(batch, cols)
        h = torch.zeros((batch, rows), dtype=torch.int16, device="cuda")
        xd = torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()
        if batch <= 4:
            ctx.gate_up_geglu(wg, wu, layout, cols, rows, batch, xd, h)
        else:
            ctx.gate_up_geglu_rm32(wg, wu, layout, cols, rows, batch, xd, h, False)
        torch.cuda.synchronize()
        got = f16_value(h.cpu().numpy().view(np.uint16))
        ref = O.gate_up_geglu_prefill(O.ROW_MAJOR, hg, hu, cols, rows, batch, x, 0)
        assert rel_err(got, ref) <= TOL32, batch
