"""GPU tests of the FFN stack (BASELINE configs 2 and 4) through the C ABI.

  * standardised rescale between layers (ns_standardize): invariants (one scale per
    token, unit RMS) and fp16 rounding of the scaled values;
  * config 2: the decode FFN block over 48 distinct seeded full-size layers,
    every layer's h and y checked against the oracle fed the same input;
  * config 4's per-layer accumulation-mode rule (fast_swa_ffn = prefill && swa &&
    !exact_ffn, metal_engine.mm:565) on a small prefill stack with the Q4_K_M
    down mix, every layer checked against the oracle in its own mode.
"""
import numpy as np
import pytest

import ns_oracle as O
import nsffn as N
from helpers import f16_value, rel_err

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


def cdna4(host, qtype, rows, cols):
    return torch.from_numpy(N.retile(host, qtype, cols, rows, N.ROW_MAJOR, N.CDNA4)).cuda()


def test_standardize(ctx):
    """Invariants of the inter-layer step: per token the output is one affine map of
    the input, (y - m) * c with m the mean, and has zero mean and unit RMS; the fp16
    output is the round-to-nearest-even of the fp32 one (within one ulp, as the two
    launches may round the scale differently); a constant row maps to zeros."""
    batch, cols = 6, 3840
    y = N.synth_normal_f32(3, batch * cols).reshape(batch, cols) * np.arange(1, batch + 1)[:, None] * 37.0
    y += np.arange(batch)[:, None] * 1000.0  # large common components, as between layers of the stack
    y[5] = 7.25                               # a constant row
    y = y.astype(np.float32)
    yd = torch.from_numpy(y).cuda()
    o32 = torch.empty((batch, cols), dtype=torch.float32, device="cuda")
    o16 = torch.empty((batch, cols), dtype=torch.int16, device="cuda")
    ctx.standardize(yd, batch, cols, o32, False)
    ctx.standardize(yd, batch, cols, o16, True)
    torch.cuda.synchronize()
    a = o32.cpu().numpy().astype(np.float64)
    assert not a[5].any() and np.isfinite(a).all()
    a, y64 = a[:5], y[:5].astype(np.float64)
    m = y64.mean(axis=1, keepdims=True)
    c = np.sum(a * (y64 - m), axis=1, keepdims=True) / np.sum((y64 - m) ** 2, axis=1, keepdims=True)
    assert np.max(np.abs(a - (y64 - m) * c)) < 2e-5                  # one affine map per token
    assert np.max(np.abs(a.mean(axis=1))) < 2e-5                      # zero mean
    assert np.allclose(np.sqrt(np.mean(a * a, axis=1)), 1.0, rtol=5e-6)  # unit RMS
    h = o16.cpu().numpy().view(np.uint16)
    want = o32.cpu().numpy().astype(np.float16).view(np.uint16)
    assert np.max(np.abs(h.astype(np.int64) - want.astype(np.int64))) <= 1


def test_config2_decode_48_distinct_layers(ctx):
    """Config 2 at full size: x -> gate/up+GeGLU -> Q6_K down, 48 distinct seeded
    layers, FP32; each layer is checked against the oracle fed the GPU's own
    input, and the next layer takes the standardised rescale of this layer's output."""
    D, F = 3840, 15360
    x = torch.from_numpy(N.synth_normal_f32(0x21, D)).cuda()
    h = torch.empty(F, dtype=torch.float32, device="cuda")
    y = torch.empty(D, dtype=torch.float32, device="cuda")
    worst = 0.0
    for layer in range(48):
        s = N.layer_seed(0xC2, layer)
        hg, hu, hd = (N.synth_weights(N.Q4_K, s + 1, F, D), N.synth_weights(N.Q4_K, s + 2, F, D),
                      N.synth_weights(N.Q6_K, s + 3, D, F))
        wg, wu, wd = cdna4(hg, N.Q4_K, F, D), cdna4(hu, N.Q4_K, F, D), cdna4(hd, N.Q6_K, D, F)
        ctx.ffn_block(wg, wu, wd, N.Q6_K, N.CDNA4, D, F, 1, x, h, y, prefill=False, swa=True)
        torch.cuda.synchronize()
        xh, hh, yh = x.cpu().numpy(), h.cpu().numpy(), y.cpu().numpy()
        e1 = rel_err(hh, O.gate_up_geglu(O.ROW_MAJOR, hg, hu, D, F, xh))
        e2 = rel_err(yh, O.gemv(N.Q6_K, O.ROW_MAJOR, hd, F, D, hh))
        assert e1 <= TOL32 and e2 <= TOL32, (layer, e1, e2)
        worst = max(worst, e1, e2)
        xn = torch.empty(D, dtype=torch.float32, device="cuda")
        ctx.standardize(y, 1, D, xn, False)
        x = xn
    print(f"config 2, 48 layers: worst rel_err {worst:.2e}")


def test_stack_prefill_mode_rule(ctx):
    """Six layers of a small stack in prefill: down is Q6_K on even layers and Q4_K
    on odd ones, layer 5 is global (FP32 mode), the others local (FP16 mode), and
    exact_ffn forces FP32 everywhere.  Every layer's H and Y are checked against
    the oracle in that layer's mode, given the GPU's own input."""
    D, F, B = 512, 1024, 40
    for exact in (False, True):
        x = torch.from_numpy(N.synth_normal_f16(0x41, B * D).view(np.int16).reshape(B, D)).cuda()
        hp = torch.empty((B, F), dtype=torch.int16, device="cuda")
        yp = torch.empty((B, D), dtype=torch.float32, device="cuda")
        for layer in range(6):
            s = N.layer_seed(0xC4, layer)
            dt = N.Q6_K if layer % 2 == 0 else N.Q4_K
            glob = layer % 6 == 5
            hg, hu, hd = (N.synth_weights(N.Q4_K, s + 1, F, D), N.synth_weights(N.Q4_K, s + 2, F, D),
                          N.synth_weights(dt, s + 3, D, F))
            wg, wu, wd = cdna4(hg, N.Q4_K, F, D), cdna4(hu, N.Q4_K, F, D), cdna4(hd, dt, D, F)
            ctx.ffn_block(wg, wu, wd, dt, N.CDNA4, D, F, B, x, hp, yp, prefill=True, swa=not glob, exact_ffn=exact)
            torch.cuda.synchronize()
            xh = x.cpu().numpy().view(np.uint16)
            hh = hp.cpu().numpy().view(np.uint16)
            yh = yp.cpu().numpy()
            fast = (not glob) and not exact
            mode = 1 if fast else 0
            tol = TOL16 if fast else TOL32
            assert rel_err(f16_value(hh), O.gate_up_geglu_prefill(O.ROW_MAJOR, hg, hu, D, F, B, xh, 0)) <= tol
            assert rel_err(yh, O.gemm(dt, O.ROW_MAJOR, hd, F, D, B, hh, 0)) <= tol
            if fast:
                assert rel_err(yh, O.gemm(dt, O.ROW_MAJOR, hd, F, D, B, hh, mode)) <= 4e-3
            # FP16 mode leaves fp16 precision (13 low fraction bits clear); FP32 mode does not
            assert (not np.any(yh.view(np.uint32) & 0x1FFF)) == fast, (layer, exact)
            xn = torch.empty((B, D), dtype=torch.int16, device="cuda")
            ctx.standardize(yp, B, D, xn, True)
            x = xn


@pytest.mark.parametrize("nlayers", [6, 48])
def test_decode_step_graph_replay_matches_eager(ctx, nlayers):
    """A decode step of the stack (config 4: Q4_K_M down mix, standardised between
    layers, lm-head at the end) captured once into a HIP graph and replayed three
    times, with eager work and synchronisations between replays; every replay's
    logits must equal the eager step's bit for bit."""
    D, F, V = 3840, 15360, 65536
    layers = []
    for l in range(nlayers):
        s = N.layer_seed(0x6A, l)
        dt = N.Q6_K if l % 2 == 0 else N.Q4_K
        layers.append((cdna4(N.synth_weights(N.Q4_K, s + 1, F, D), N.Q4_K, F, D),
                       cdna4(N.synth_weights(N.Q4_K, s + 2, F, D), N.Q4_K, F, D),
                       cdna4(N.synth_weights(dt, s + 3, D, F), dt, D, F), dt))
    lm = cdna4(N.synth_weights(N.Q6_K, 0x6B, V, D), N.Q6_K, V, D)
    x0 = torch.from_numpy(N.synth_normal_f32(0x6C, D)).cuda()
    xd = x0.clone()
    h = torch.empty(F, dtype=torch.float32, device="cuda")
    y = torch.empty(D, dtype=torch.float32, device="cuda")
    xs = torch.empty(D, dtype=torch.float32, device="cuda")
    logits = torch.empty(V, dtype=torch.float32, device="cuda")

    def step():
        inp = xd
        for l, (g, u, d, dt) in enumerate(layers):
            ctx.ffn_block(g, u, d, dt, N.CDNA4, D, F, 1, inp, h, y, prefill=False, swa=l % 6 != 5)
            ctx.standardize(y, 1, D, xs, False)
            inp = xs
        ctx.matmul(lm, N.Q6_K, N.CDNA4, D, V, 1, xs, logits)
        xd.copy_(xs)

    step()
    torch.cuda.synchronize()
    xd.copy_(x0)
    step()
    torch.cuda.synchronize()
    eager, eager_x = logits.clone(), xd.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for r in range(3):
        xd.copy_(x0)
        logits.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits, eager) and torch.equal(xd, eager_x), f"replay {r}"
        step()  # eager work between replays
        torch.cuda.synchronize()
