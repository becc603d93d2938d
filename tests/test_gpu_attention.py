"""GPU parity of the rest of a layer's matmul time on the same machinery (the survey's next
row after the FFN neighbours): the token embedding lookup (gemma_q6k_embedding, metal:503-505),
the fused Q/K/V projections (qkv, mm:311; metal:442-454) and the prefill GEMM on row-major
weights (matmul, mm:274: the reference's swizzled kernels, as attention tensors stay row-major).

The embedding is bit-exact: scale * the quant.cpp value, one fp32 rounding, compared with the
oracle's dequantised row times the same fp32 scale.  Projections: FP32 bar, rel_err <= 1e-3.
"""
import numpy as np
import pytest

import ns_oracle as O
import nsffn as N
from helpers import rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

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


@pytest.mark.parametrize("layout", [N.ROW_MAJOR, N.NSMFFN, N.CDNA4], ids=LNAME.get)
@pytest.mark.parametrize("qtype", [N.Q6_K, N.Q4_K], ids=["q6k", "q4k"])
def test_embedding_bit_exact(ctx, qtype, layout):
    cols, rows = 3840, 1024
    host, w = weights(qtype, 0xE1, rows, cols, layout)
    ids = np.array([0, rows - 1, 517, 3, 3, 900], dtype=np.int32)
    scale = np.float32(np.sqrt(3840.0))
    out = torch.empty((len(ids), cols), dtype=torch.float32, device="cuda")
    ctx.embedding(w, qtype, layout, cols, rows, torch.from_numpy(ids).cuda(), len(ids), float(scale), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for t, r in enumerate(ids):
        want = scale * O.dequant_rows(qtype, O.ROW_MAJOR, host, cols, rows, int(r), 1)[0]
        np.testing.assert_array_equal(got[t].view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_embedding_rejects_out_of_range_ids(ctx):
    cols, rows = 512, 128
    _, w = weights(N.Q6_K, 0xE2, rows, cols, N.ROW_MAJOR)
    ids = torch.tensor([5, -1, rows, 7], dtype=torch.int32, device="cuda")
    out = torch.zeros((4, cols), dtype=torch.float32, device="cuda")
    ctx.embedding(w, N.Q6_K, N.ROW_MAJOR, cols, rows, ids, 4, 1.0, out)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.isnan(o[1]).all() and np.isnan(o[2]).all() and np.isfinite(o[0]).all() and np.isfinite(o[3]).all()


@pytest.mark.parametrize("batch", [3, 40])
@pytest.mark.parametrize("v", ["q4", "q6", "tied"])
@pytest.mark.parametrize("layout", [N.ROW_MAJOR, N.CDNA4], ids=LNAME.get)
def test_qkv(ctx, layout, v, batch):
    cols, q_rows, kv_rows = 768, 512, 256
    if layout == N.ROW_MAJOR:
        q_rows, kv_rows = 520, 200  # ragged: the row-major layout has no 64-row rule
    hq, wq = weights(N.Q4_K, 0xA1, q_rows, cols, layout)
    hk, wk = weights(N.Q4_K, 0xA2, kv_rows, cols, layout)
    vt = N.Q6_K if v == "q6" else N.Q4_K
    hv, wv = weights(vt, 0xA3, kv_rows, cols, layout) if v != "tied" else (hk, None)
    bits = N.synth_normal_f16(0xA4, batch * cols).reshape(batch, cols)
    x = torch.from_numpy(bits.view(np.int16)).cuda()
    q = torch.full((batch, q_rows), float("nan"), dtype=torch.float32, device="cuda")
    k = torch.full((batch, kv_rows), float("nan"), dtype=torch.float32, device="cuda")
    vo = torch.full((batch, kv_rows), float("nan"), dtype=torch.float32, device="cuda")
    ctx.qkv(wq, wk, wv, vt, layout, cols, q_rows, kv_rows, batch, x, q, k, vo)
    torch.cuda.synchronize()
    assert rel_err(q.cpu().numpy(), O.gemm(N.Q4_K, O.ROW_MAJOR, hq, cols, q_rows, batch, bits, 0)) <= 1e-3
    assert rel_err(k.cpu().numpy(), O.gemm(N.Q4_K, O.ROW_MAJOR, hk, cols, kv_rows, batch, bits, 0)) <= 1e-3
    assert rel_err(vo.cpu().numpy(), O.gemm(vt, O.ROW_MAJOR, hv, cols, kv_rows, batch, bits, 0)) <= 1e-3
    if v == "tied":
        assert torch.equal(vo, k)


@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
def test_prefill_matmul_row_major(ctx, qtype):
    """matmul at batch > 4 with fp16 input on a row-major tensor (mm:274), ragged rows."""
    cols, rows, batch = 1024, 328, 70
    host, w = weights(qtype, 0xB1, rows, cols, N.ROW_MAJOR)
    bits = N.synth_normal_f16(0xB2, batch * cols).reshape(batch, cols)
    y = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
    ctx.matmul(w, qtype, N.ROW_MAJOR, cols, rows, batch, torch.from_numpy(bits.view(np.int16)).cuda(), y,
               half_input=True)
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), O.gemm(qtype, O.ROW_MAJOR, host, cols, rows, batch, bits, 0)) <= 1e-3


@pytest.mark.parametrize("fast_swa", [False, True], ids=["fp32acc", "fp16acc"])
def test_prefill_gate_up_row_major(ctx, fast_swa):
    """The gate/up pair GEMM on row-major tensors (ragged rows), both accumulation modes."""
    cols, rows, batch = 768, 136, 48
    hg, wg = weights(N.Q4_K, 0xC1, rows, cols, N.ROW_MAJOR)
    hu, wu = weights(N.Q4_K, 0xC2, rows, cols, N.ROW_MAJOR)
    bits = N.synth_normal_f16(0xC3, batch * cols).reshape(batch, cols)
    h = torch.zeros((batch, rows), dtype=torch.int16, device="cuda")
    ctx.gate_up_geglu_rm32(wg, wu, N.ROW_MAJOR, cols, rows, batch, torch.from_numpy(bits.view(np.int16)).cuda(), h,
                           fast_swa)
    torch.cuda.synchronize()
    got = h.cpu().numpy().view(np.uint16).view(np.float16).astype(np.float32)
    ref = O.gate_up_geglu_prefill(O.ROW_MAJOR, hg, hu, cols, rows, batch, bits, 0)
    assert rel_err(got, ref) <= (1e-2 if fast_swa else 1e-3)


def test_qkv_rejects_decode_batch(ctx):
    cols = 256
    _, wq = weights(N.Q4_K, 1, 64, cols, N.CDNA4)
    x = torch.zeros((1, cols), dtype=torch.int16, device="cuda")
    out = torch.empty((1, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(N.NsError, match="batch >= 2"):
        ctx.qkv(wq, wq, None, N.Q4_K, N.CDNA4, cols, 64, 64, 1, x, out, out, out)
