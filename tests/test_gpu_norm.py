"""GPU parity of the FFN neighbours (metal:509-529; mm:291-296, called at mm:563, :574, :576)
and of the decode gate/up GEMV with the RMSNorm ahead of it fused in, against the CPU oracle.  RMSNorm outputs: fp32 within 2e-6 of the largest output (the GPU sums with
FMAs in a different order); fp16 outputs within one fp16 step of the oracle's value.  The
fused gate/up: FP32 bar, rel_err <= 1e-3.
"""
import numpy as np
import pytest

import ns_oracle as O
import nsffn as N
from helpers import f16_value, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

LNAME = {N.CDNA4: "cdna4", N.NSMFFN: "nsmffn", N.ROW_MAJOR: "rowmajor"}
EPS = 1e-6


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = N.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def vec(seed, n, shift=0.0):
    return (np.random.default_rng(seed).standard_normal(n) + shift).astype(np.float32)


def assert_f16_close(got_bits, ref32):
    """Every fp16 output within one fp16 step of the oracle's fp32 value, plus 4e-6 of the
    row's largest value: where the residual cancels the normed term, the fp32 value itself
    carries that absolute rounding (the GPU fuses the add), which near zero exceeds a step."""
    got = np.atleast_2d(f16_value(got_bits).astype(np.float64))
    ref = np.atleast_2d(np.asarray(ref32, dtype=np.float64))
    step = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    slack = 4e-6 * np.max(np.abs(ref), axis=1, keepdims=True)
    assert np.all(np.abs(got - ref) <= step + slack), float(np.max((np.abs(got - ref) - slack) / step))


@pytest.mark.parametrize("width", [3840, 1000, 1])
def test_rmsnorm(ctx, width):
    rows = 3
    x, w = vec(1, rows * width).reshape(rows, width), vec(2, width, 1.0)
    y = torch.empty((rows, width), dtype=torch.float32, device="cuda")
    yh = torch.empty((rows, width), dtype=torch.int16, device="cuda")
    ctx.rmsnorm(dev(x), dev(w), rows, width, EPS, y)
    ctx.rmsnorm(dev(x), dev(w), rows, width, EPS, yh, half_out=True)
    torch.cuda.synchronize()
    ref = O.rmsnorm(x, w, eps=EPS)
    assert rel_err(y.cpu().numpy(), ref) <= 2e-6
    assert_f16_close(yh.cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("scaled", [False, True])
def test_rmsnorm_add(ctx, scaled):
    rows, width = 2, 3840
    x, w, res = vec(3, rows * width).reshape(rows, width), vec(4, width), vec(5, rows * width).reshape(rows, width)
    scale = np.float32([0.625])
    y = torch.empty((rows, width), dtype=torch.float32, device="cuda")
    ctx.rmsnorm_add(dev(x), dev(w), dev(res), dev(scale) if scaled else None, rows, width, EPS, y)
    torch.cuda.synchronize()
    ref = O.rmsnorm(x, w, residual=res, scale=float(scale[0]) if scaled else None, eps=EPS)
    assert rel_err(y.cpu().numpy(), ref) <= 2e-6
    # in place over the residual (each element is read before it is written)
    yr = dev(res)
    ctx.rmsnorm_add(dev(x), dev(w), yr, dev(scale) if scaled else None, rows, width, EPS, yr)
    torch.cuda.synchronize()
    assert rel_err(yr.cpu().numpy(), ref) <= 2e-6


@pytest.mark.parametrize("half_next", [False, True])
def test_rmsnorm_add_then(ctx, half_next):
    """rms_add_then_half (mm:296; half_next) and rms_add followed by rms (mm:563)."""
    rows, width = 4, 3840
    x, w, res, nw = (vec(6, rows * width).reshape(rows, width), vec(7, width),
                     vec(8, rows * width).reshape(rows, width), vec(9, width, 1.0))
    scale = np.float32([1.5])
    y = torch.empty((rows, width), dtype=torch.float32, device="cuda")
    nxt = torch.empty((rows, width), dtype=torch.int16 if half_next else torch.float32, device="cuda")
    ctx.rmsnorm_add_then(dev(x), dev(w), dev(res), dev(scale), dev(nw), rows, width, EPS, y, nxt, half_next)
    torch.cuda.synchronize()
    ry, rn = O.rmsnorm(x, w, residual=res, scale=1.5, next_w=nw, eps=EPS)
    assert rel_err(y.cpu().numpy(), ry) <= 2e-6
    if half_next:
        assert_f16_close(nxt.cpu().numpy().view(np.uint16), rn)
    else:
        assert rel_err(nxt.cpu().numpy(), rn) <= 4e-6


def weights(seed, rows, cols, layout):
    host = N.synth_weights(N.Q4_K, seed, rows, cols)
    lay = host if layout == N.ROW_MAJOR else N.retile(host, N.Q4_K, cols, rows, N.ROW_MAJOR, layout)
    return host, dev(lay)


@pytest.mark.parametrize("force_pf", [None, "1"], ids=["auto", "prefetch"])
@pytest.mark.parametrize("layout", [N.CDNA4, N.NSMFFN, N.ROW_MAJOR], ids=LNAME.get)
@pytest.mark.parametrize("shape", [(768, 128), (3840, 15360)], ids=["small", "gemma"])
def test_rms_gate_up_geglu_decode(ctx, layout, shape, force_pf, tune):
    """rms (mm:563) fused ahead of the pair GEMV.  The default grid (one super-block per wave,
    whole slabs) takes the barrier-free form; the prefetching instance the workgroup form."""
    if force_pf:
        tune("gemv_pf", force_pf)
    cols, rows = shape
    if layout == N.ROW_MAJOR and rows == 128:
        rows = 136  # ragged last slab
    hg, wg = weights(31, rows, cols, layout)
    hu, wu = weights(32, rows, cols, layout)
    x, nw = vec(33, cols, 0.5), vec(34, cols)
    h = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    ctx.rms_gate_up_geglu_decode(wg, wu, layout, cols, rows, dev(x), dev(nw), EPS, h)
    torch.cuda.synchronize()
    xn = O.rmsnorm(x, nw, eps=EPS)
    ref = O.gate_up_geglu(O.ROW_MAJOR, hg, hu, cols, rows, xn)
    assert rel_err(h.cpu().numpy(), ref) <= 1e-3


def test_rms_fused_equals_rms_then_gate_up(ctx):
    """The fused entry against the standalone rms followed by the plain pair GEMV."""
    cols, rows = 3840, 15360
    _, wg = weights(41, rows, cols, N.CDNA4)
    _, wu = weights(42, rows, cols, N.CDNA4)
    x, nw = dev(vec(43, cols, 0.3)), dev(vec(46, cols, 1.0))
    h1 = torch.empty(rows, dtype=torch.float32, device="cuda")
    h2 = torch.empty(rows, dtype=torch.float32, device="cuda")
    xn = torch.empty(cols, dtype=torch.float32, device="cuda")
    ctx.rms_gate_up_geglu_decode(wg, wu, N.CDNA4, cols, rows, x, nw, EPS, h1)
    ctx.rmsnorm(x, nw, 1, cols, EPS, xn)
    ctx.gate_up_geglu_decode(wg, wu, N.CDNA4, cols, rows, xn, h2)
    torch.cuda.synchronize()
    assert rel_err(h1.cpu().numpy(), h2.cpu().numpy()) <= 1e-5


@pytest.mark.parametrize("force_pf", ["0", "1"], ids=["one_unit", "prefetch"])
@pytest.mark.parametrize("layout", [N.CDNA4, N.NSMFFN, N.ROW_MAJOR], ids=LNAME.get)
@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
def test_gemv_both_instances(ctx, qtype, layout, force_pf, tune):
    """The decode GEMV with each kernel instance forced (NS_GEMV_PF), on shapes with more
    than 16 super-blocks per row, so slabs are cut between workgroups in both."""
    tune("gemv_pf", force_pf)
    cols, rows = 5120, (200 if layout == N.ROW_MAJOR else 192)
    host = N.synth_weights(qtype, 61, rows, cols)
    w = dev(host if layout == N.ROW_MAJOR else N.retile(host, qtype, cols, rows, N.ROW_MAJOR, layout))
    x = vec(62, cols)
    y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    ctx.matmul(w, qtype, layout, cols, rows, 1, dev(x), y)
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, x)) <= 1e-3
