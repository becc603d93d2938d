"""GPU tests of the wait-free mode (ns_ctx_set_wait_free) and of the context's status word
(ns_ctx_status, the counterpart of the reference's finish_command, mm:231-243).

A context in the wait-free mode runs launches in which no workgroup waits for another: the
split-K prefill GEMMs finish by the last part to arrive instead of the reduce-scatter, and the
decode FFN block runs as its two launches.  Each split reduction adds the same fp32 parts in
the same order, so the outputs equal the default context's bit for bit, in both accumulation
modes; and default runs leave the status clear.
"""
import numpy as np
import pytest

import nsffn as N

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

D, F = 3840, 15360


@pytest.fixture(scope="module")
def ctxs():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    a, b = N.Context(0), N.Context(0)
    b.set_wait_free(True)
    yield a, b
    torch.cuda.synchronize()
    a.close()
    b.close()


def cdna4(qtype, seed, rows, cols):
    host = N.synth_weights(qtype, seed, rows, cols)
    return torch.from_numpy(N.retile(host, qtype, cols, rows, N.ROW_MAJOR, N.CDNA4)).cuda()


def f16(seed, n):
    return torch.from_numpy(N.synth_normal_f16(seed, n).view(np.int16)).cuda()


def same_bits(a, b):
    return torch.equal(a.view(torch.int32), b.view(torch.int32))


@pytest.mark.parametrize("qtype", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("fast", [False, True], ids=["fp32", "fp16"])
@pytest.mark.parametrize("batch", [1024, 300])
def test_prefill_down_wait_free_equals_default(ctxs, qtype, fast, batch):
    """The split-K down projection (3840 x 15360): reduce-scatter (default) and last arrival
    (wait-free) give the same bits."""
    w = cdna4(qtype, 0x51 + qtype, D, F)
    x = f16(0x52 + batch, batch * F)
    outs = []
    for c in ctxs:
        y = torch.full((batch, D), float("nan"), dtype=torch.float32, device="cuda")
        c.ffn_down(w, qtype, N.CDNA4, F, D, batch, x, y, half_input=True, fast_swa=fast)
        c.status()
        outs.append(y)
    assert torch.isfinite(outs[0]).all()
    assert same_bits(outs[0], outs[1])


@pytest.mark.parametrize("fast", [False, True], ids=["fp32", "fp16"])
def test_prefill_gate_up_wait_free_equals_default(ctxs, fast):
    batch = 512
    wg, wu = cdna4(N.Q4_K, 0x61, F, D), cdna4(N.Q4_K, 0x62, F, D)
    x = f16(0x63, batch * D)
    outs = []
    for c in ctxs:
        h = torch.zeros((batch, F), dtype=torch.int16, device="cuda")
        c.gate_up_geglu_rm32(wg, wu, N.CDNA4, D, F, batch, x, h, fast)
        c.status()
        outs.append(h)
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("down_type", [N.Q4_K, N.Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("norm", [False, True], ids=["x", "rms"])
def test_decode_block_wait_free_equals_default(ctxs, down_type, norm):
    """The one-launch decode block (default) equals its two launches (wait-free) bit for bit."""
    wg, wu, wd = cdna4(N.Q4_K, 0x71, F, D), cdna4(N.Q4_K, 0x72, F, D), cdna4(down_type, 0x73, D, F)
    x = torch.from_numpy(N.synth_normal_f32(0x74, D)).cuda()
    nw = torch.from_numpy(N.synth_normal_f32(0x75, D)).cuda() if norm else None
    outs = []
    for c in ctxs:
        h = torch.full((F,), float("nan"), dtype=torch.float32, device="cuda")
        y = torch.full((D,), float("nan"), dtype=torch.float32, device="cuda")
        c.ffn_block_decode(wg, wu, wd, down_type, N.CDNA4, D, F, x, h, y, norm_weight=nw, eps=1e-6)
        c.status()
        outs.append((h, y))
    assert torch.isfinite(outs[0][1]).all()
    assert same_bits(outs[0][0], outs[1][0]) and same_bits(outs[0][1], outs[1][1])


def test_status_on_a_null_context_is_an_argument_error():
    with pytest.raises(N.NsError) as e:
        N.check(N.lib().ns_ctx_status(None, None))
    assert e.value.code == 1
