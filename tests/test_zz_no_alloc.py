"""GPU test of ns_matmul_noalloc (the entry point that allocates nothing): through the C ABI
its outputs equal ns_matmul's bit for bit, on two calls in a row with the second on a
smaller input (the static scratch keeps the first call's contents), for the decode GEMV
whose slabs are cut between workgroups (the 60-block down projection), the 262,144-row
lm-head, and the batch 2-4 kernels; shapes past the static scratch are refused."""
import numpy as np
import pytest

import nsffn as N

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = N.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def cdna4(qtype, seed, rows, cols):
    host = N.synth_weights(qtype, seed, rows, cols)
    return torch.from_numpy(N.retile(host, qtype, cols, rows, N.ROW_MAJOR, N.CDNA4)).cuda()


CASES = [  # (first call, second call on a smaller input): (qtype, rows, cols, batch, half)
    ((N.Q6_K, 262144, 3840, 1, False), (N.Q6_K, 3840, 15360, 1, False)),
    ((N.Q6_K, 3840, 15360, 1, False), (N.Q4_K, 3840, 3840, 1, False)),
    ((N.Q4_K, 15360, 3840, 4, True), (N.Q6_K, 3840, 15360, 2, True)),
    ((N.Q6_K, 262144, 3840, 4, False), (N.Q4_K, 15360, 3840, 3, False)),
]


@pytest.mark.parametrize("first,second", CASES, ids=["lmhead-down", "down-q4", "mt4-mt2", "lmhead4-mt3"])
def test_noalloc_matches_matmul(ctx, first, second):
    for k, (qtype, rows, cols, batch, half) in enumerate((first, second)):
        w = cdna4(qtype, 300 + k, rows, cols)
        if half:
            x = torch.from_numpy(N.synth_normal_f16(310 + k, batch * cols).view(np.int16)).cuda()
        else:
            x = torch.from_numpy(N.synth_normal_f32(310 + k, batch * cols)).cuda()
        ref = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
        got = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
        ctx.matmul(w, qtype, N.CDNA4, cols, rows, batch, x, ref, half_input=half)
        N.matmul_noalloc(w, qtype, N.CDNA4, cols, rows, batch, x, got, half_input=half)
        torch.cuda.synchronize()
        assert not torch.isnan(ref).any()
        assert torch.equal(got, ref), (k, qtype, rows, cols, batch)


PREFILL_CASES = [  # (first call, second call on a smaller input): (qtype, rows, cols, batch)
    ((N.Q6_K, 3840, 15360, 1024), (N.Q4_K, 15360, 3840, 300)),
    ((N.Q4_K, 3840, 15360, 256), (N.Q6_K, 3840, 15360, 5)),
]


@pytest.mark.parametrize("first,second", PREFILL_CASES, ids=["q6down1024-q4gate300", "q4down256-q6down5"])
def test_noalloc_prefill_matches_matmul_with_one_k_part(ctx, first, second):
    """Above batch 4 the static scratch cannot hold the default plan's split-K parts (a
    batch-1024 Q6_K down needs ~63 MB): the GEMM runs with one K part, as ns_matmul does with
    the gemm_kparts 1 tuning, and equals it bit for bit; the status stays clear."""
    for k, (qtype, rows, cols, batch) in enumerate((first, second)):
        w = cdna4(qtype, 320 + k, rows, cols)
        x = torch.from_numpy(N.synth_normal_f16(330 + k, batch * cols).view(np.int16)).cuda()
        ref = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
        got = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
        ctx.set_tuning("gemm_kparts", 1)
        try:
            ctx.matmul(w, qtype, N.CDNA4, cols, rows, batch, x, ref, half_input=True)
        finally:
            ctx.set_tuning("gemm_kparts", 0)
        N.matmul_noalloc(w, qtype, N.CDNA4, cols, rows, batch, x, got, half_input=True)
        N.noalloc_status()
        assert not torch.isnan(ref).any()
        assert torch.equal(got, ref), (k, qtype, rows, cols, batch)


def test_noalloc_refuses_shapes_past_the_scratch():
    """A batch-1024 Q4_K down projection (15360 columns) needs ~8.3 M floats of x group sums
    and rescaled copy, above the 4 M of the static scratch, even with one K part."""
    rows, cols, batch = 3840, 15360, 1024
    w = torch.zeros(rows * (cols // 256) * 144, dtype=torch.uint8, device="cuda")
    x = torch.zeros(batch * cols, dtype=torch.int16, device="cuda")
    y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    with pytest.raises(N.NsError, match="static scratch"):
        N.matmul_noalloc(w, N.Q4_K, N.CDNA4, cols, rows, batch, x, y, half_input=True)
    N.noalloc_status()
