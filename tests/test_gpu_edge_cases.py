"""GPU parity on the special cases of the block formats, through every kernel family.

The dequantisation of these cases is pinned bit-exact elsewhere (test_oracle.py,
test_gpu_parity.py::test_dequant_bit_exact).  The matmul kernels do not dequantise
element by element: the GEMVs factor d, dmin, the scales and the group sums of x, and
the GEMMs hold sc*q integers with d applied on the accumulators (and a rescale factor
z = d/e < 1 for Q4_K blocks with d < dmin/1024).  Here every row mixes:

  Q4_K  random; d = dmin = 0; d = 0; dmin = 0; all scales 0 (w = -dmin*m); q = 15 with
        sc = m = 63; fp16-subnormal d; d far below dmin (the z < 1 path)
  Q6_K  random; d = 0; every scale -32 with v = 0 (w = 1024*d); scales at +31/-32 with
        v at 0/63; fp16-subnormal d; v = 63 everywhere

Also: x constant over each scale group (isolates the scale and min sums), the largest
batch the reference accepts (2048, config.cpp:124), and a float64 brute force of the
tiny shapes (rows 64, cols 256/512, batch 1/5/33) as a third reference.
"""
import numpy as np
import pytest

import ns_oracle as O
import nsffn as N
from helpers import f16_value, q4k_block, q6k_block, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL32, TOL16 = 1e-3, 1e-2


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = N.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def q4_kind(rng, kind):
    sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    d, dmin = abs(rng.normal()) * 1e-3, abs(rng.normal()) * 1e-3
    if kind == 1:
        d = dmin = 0.0
    elif kind == 2:
        d = 0.0
    elif kind == 3:
        dmin = 0.0
    elif kind == 4:
        sc = np.zeros(8, dtype=np.int64)
    elif kind == 5:
        sc, m, q = np.full(8, 63), np.full(8, 63), np.full(256, 15)
    elif kind == 6:
        d = 3.0e-6  # fp16 subnormal
    elif kind == 7:
        d, dmin = 2.0e-7, 4.0e-3  # d < dmin / 1024
    return q4k_block(d, dmin, sc, m, q)


def q6_kind(rng, kind):
    sc = rng.integers(-32, 32, 16)
    v = rng.integers(0, 64, 256)
    d = abs(rng.normal()) * 1e-3
    if kind == 1:
        d = 0.0
    elif kind == 2:
        sc, v = np.full(16, -32), np.zeros(256, dtype=np.int64)
    elif kind == 3:
        sc = np.where(np.arange(16) % 2 == 0, 31, -32)
        v = np.where(np.arange(256) % 3 == 0, 63, 0)
    elif kind == 4:
        d = 3.0e-6
    elif kind == 5:
        v = np.full(256, 63)
    return q6k_block(d, sc, v)


def special_matrix(qtype, rows, cols, seed):
    """Row-major blocks; block (r, b) has kind (r + b) % nkinds, so every row mixes kinds."""
    rng = np.random.default_rng(seed)
    nb = cols // 256
    nk, make = (8, q4_kind) if qtype == N.Q4_K else (6, q6_kind)
    return np.concatenate([make(rng, (r + b) % nk) for r in range(rows) for b in range(nb)])


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def laid(host, qtype, rows, cols, layout):
    return dev(host if layout == N.ROW_MAJOR else N.retile(host, qtype, cols, rows, N.ROW_MAJOR, layout))


LAYOUTS = [N.CDNA4, N.NSMFFN]
LNAME = {N.CDNA4: "cdna4", N.NSMFFN: "nsmffn", N.ROW_MAJOR: "rowmajor"}


@pytest.mark.parametrize("layout", [N.CDNA4, N.NSMFFN, N.ROW_MAJOR], ids=LNAME.get)
@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
def test_special_blocks_gemv_and_small_batch(ctx, qtype, layout):
    rows, cols = 128, 1024
    host = special_matrix(qtype, rows, cols, 7 + qtype)
    w = laid(host, qtype, rows, cols, layout)
    x = N.synth_normal_f32(11, 3 * cols).reshape(3, cols)
    y1 = torch.empty(rows, dtype=torch.float32, device="cuda")
    y3 = torch.empty((3, rows), dtype=torch.float32, device="cuda")
    ctx.matmul(w, qtype, layout, cols, rows, 1, dev(x[0]), y1)
    ctx.matmul(w, qtype, layout, cols, rows, 3, dev(x), y3)
    torch.cuda.synchronize()
    assert rel_err(y1.cpu().numpy(), O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, x[0])) <= TOL32
    got3 = y3.cpu().numpy()
    for t in range(3):
        assert rel_err(got3[t], O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, x[t])) <= TOL32, t


# Q4_K has two GEMM kernels (register-fragment, LDS-tile); Q6_K has one
GEMM_KERNELS = [(N.Q4_K, "1"), (N.Q4_K, "0"), (N.Q6_K, "1")]


@pytest.mark.parametrize("acc", [N.ACC_FP32, N.ACC_FP16], ids=["fp32acc", "fp16acc"])
@pytest.mark.parametrize("layout", LAYOUTS, ids=LNAME.get)
@pytest.mark.parametrize("qtype,reg", GEMM_KERNELS, ids=["q4k-reg", "q4k-lds", "q6k"])
def test_special_blocks_gemm(ctx, tune, qtype, reg, layout, acc):
    tune("gemm_q4_reg", reg)
    rows, cols, batch = 128, 1024, 40
    host = special_matrix(qtype, rows, cols, 17 + qtype)
    w = laid(host, qtype, rows, cols, layout)
    xb = N.synth_normal_f16(19, batch * cols).reshape(batch, cols)
    y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    fast = acc == N.ACC_FP16
    ctx.ffn_down(w, qtype, layout, cols, rows, batch, dev(xb.view(np.int16)), y, half_input=True, fast_swa=fast)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.isfinite(got).all()
    assert rel_err(got, O.gemm(qtype, O.ROW_MAJOR, host, cols, rows, batch, xb, 0)) <= (TOL16 if fast else TOL32)
    if fast:
        assert rel_err(got, O.gemm(qtype, O.ROW_MAJOR, host, cols, rows, batch, xb, 1)) <= 4e-3


@pytest.mark.parametrize("layout", LAYOUTS, ids=LNAME.get)
def test_special_blocks_gate_up(ctx, layout):
    """Decode pair, small-batch pair and the prefill pair (FP32 mode) on special Q4_K blocks."""
    rows, cols = 128, 768
    hg, hu = special_matrix(N.Q4_K, rows, cols, 23), special_matrix(N.Q4_K, rows, cols, 24)
    wg, wu = laid(hg, N.Q4_K, rows, cols, layout), laid(hu, N.Q4_K, rows, cols, layout)
    x = N.synth_normal_f32(25, cols)
    h = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.gate_up_geglu_decode(wg, wu, layout, cols, rows, dev(x), h)
    xb = N.synth_normal_f16(26, 40 * cols).reshape(40, cols)
    hp = torch.empty((40, rows), dtype=torch.int16, device="cuda")
    ctx.gate_up_geglu_rm32(wg, wu, layout, cols, rows, 40, dev(xb.view(np.int16)), hp, False)
    hs = torch.empty((3, rows), dtype=torch.int16, device="cuda")
    ctx.gate_up_geglu(wg, wu, layout, cols, rows, 3, dev(xb[:3].view(np.int16)), hs)
    torch.cuda.synchronize()
    assert rel_err(h.cpu().numpy(), O.gate_up_geglu(O.ROW_MAJOR, hg, hu, cols, rows, x)) <= TOL32
    ref = O.gate_up_geglu_prefill(O.ROW_MAJOR, hg, hu, cols, rows, 40, xb, 0)
    assert rel_err(f16_value(hp.cpu().numpy().view(np.uint16)), ref) <= TOL32
    assert rel_err(f16_value(hs.cpu().numpy().view(np.uint16)), ref[:3]) <= TOL32


@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
def test_x_constant_per_group(ctx, qtype):
    """x constant over each 32-wide (Q4_K) or 16-wide (Q6_K) scale group: the dot
    reduces to the scale and min sums the GEMVs factor out."""
    rows, cols = 192, 2048
    host = N.synth_weights(qtype, 31, rows, cols)
    g = 32 if qtype == N.Q4_K else 16
    x = np.repeat(N.synth_normal_f32(32, cols // g), g).astype(np.float32)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.matmul(laid(host, qtype, rows, cols, N.CDNA4), qtype, N.CDNA4, cols, rows, 1, dev(x), y)
    torch.cuda.synchronize()
    ref = O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, x)
    assert rel_err(y.cpu().numpy(), ref) <= TOL32
    # and against the factored closed form in float64: sum_g x_g * sum_{k in g} w_k
    wd = O.dequant_rows(qtype, O.ROW_MAJOR, host, cols, rows).astype(np.float64).reshape(rows, cols // g, g)
    closed = wd.sum(axis=2) @ x[::g].astype(np.float64)
    assert rel_err(y.cpu().numpy(), closed) <= TOL32


@pytest.mark.parametrize("acc", [N.ACC_FP32, N.ACC_FP16], ids=["fp32acc", "fp16acc"])
def test_max_batch_2048(ctx, acc):
    """The largest batch the reference accepts (config.cpp:124): both halves of the block."""
    cols, rows, batch = 512, 256, 2048
    hg, hu = N.synth_weights(N.Q4_K, 41, rows, cols), N.synth_weights(N.Q4_K, 42, rows, cols)
    hd = N.synth_weights(N.Q6_K, 43, cols, rows)
    xb = N.synth_normal_f16(44, batch * cols).reshape(batch, cols)
    h = torch.empty((batch, rows), dtype=torch.int16, device="cuda")
    y = torch.empty((batch, cols), dtype=torch.float32, device="cuda")
    fast = acc == N.ACC_FP16
    tol = TOL16 if fast else TOL32
    ctx.gate_up_geglu_rm32(laid(hg, N.Q4_K, rows, cols, N.CDNA4), laid(hu, N.Q4_K, rows, cols, N.CDNA4), N.CDNA4,
                           cols, rows, batch, dev(xb.view(np.int16)), h, fast)
    ctx.ffn_down(laid(hd, N.Q6_K, cols, rows, N.CDNA4), N.Q6_K, N.CDNA4, rows, cols, batch, h, y, True, fast)
    torch.cuda.synchronize()
    hh = h.cpu().numpy().view(np.uint16)
    assert rel_err(f16_value(hh), O.gate_up_geglu_prefill(O.ROW_MAJOR, hg, hu, cols, rows, batch, xb, 0)) <= tol
    assert rel_err(y.cpu().numpy(), O.gemm(N.Q6_K, O.ROW_MAJOR, hd, rows, cols, batch, hh, 0)) <= tol


@pytest.mark.parametrize("batch", [1, 5, 33])
@pytest.mark.parametrize("cols", [256, 512])
@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
def test_tiny_shapes_float64_brute_force(ctx, qtype, cols, batch):
    """rows 64: the GPU (GEMV, small-batch or GEMM by batch) and the oracle, each
    against a float64 product of the dequantised weights."""
    rows = 64
    host = N.synth_weights(qtype, 51 + cols, rows, cols)
    wd = O.dequant_rows(qtype, O.ROW_MAJOR, host, cols, rows).astype(np.float64).reshape(rows, cols)
    w = laid(host, qtype, rows, cols, N.CDNA4)
    y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    if batch == 1:
        x = N.synth_normal_f32(52, cols)
        ctx.matmul(w, qtype, N.CDNA4, cols, rows, 1, dev(x), y)
        xs, oracle = x[None, :].astype(np.float64), O.gemv(qtype, O.ROW_MAJOR, host, cols, rows, x)[None, :]
    else:
        xb = N.synth_normal_f16(53, batch * cols).reshape(batch, cols)
        ctx.ffn_down(w, qtype, N.CDNA4, cols, rows, batch, dev(xb.view(np.int16)), y, half_input=True, fast_swa=False)
        xs, oracle = f16_value(xb).astype(np.float64), O.gemm(qtype, O.ROW_MAJOR, host, cols, rows, batch, xb, 0)
    torch.cuda.synchronize()
    brute = xs @ wd.T
    assert rel_err(oracle, brute) <= 1e-5
    assert rel_err(y.cpu().numpy(), brute) <= TOL32
