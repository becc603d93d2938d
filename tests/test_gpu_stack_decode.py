"""GPU tests of the multi-layer decode launch (ns_ffn_stack_decode): the decode FFN blocks of
consecutive layers (the engine's per-layer decode FFN, metal_engine.mm:563-573, repeated; config
4's decode stack) in one launch.

  * 48 distinct full-size layers in config 4's Q4_K_M mix (Q6_K down on even layers, Q4_K on
    odd ones) with the RMSNorm folded in (per-layer sign vectors as norm weights): y equals 48
    calls of ns_ffn_block_decode bit for bit (whose parity with the oracle is checked layer by
    layer in test_gpu_stack.py and test_gpu_block.py), and the last layer equals the oracle
    applied to the launch's own y after 47 layers, FP32 bar 1e-3;
  * shapes with 1, 2, 3 and 4 column parts and 1-15 compute waves, with and without the norm,
    bit for bit against the per-layer blocks and the last layer against the oracle; a shape the
    launch does not take (16 waves) runs the per-layer blocks;
  * more layers than one launch's table holds (70): chained launches;
  * y aliasing x, repeated launches (the counters reset), HIP graph replays;
  * the bounded waits, forced down to one poll from the host: y is NaN, the context's status
    reports NS_ERR_TIMEOUT once, and the next launch is exact again;
  * the wait-free context runs one block per layer: the same bits;
  * launches of different lengths and shapes alternating on one context (the epoch), and a shape
    that grows the context's tagged buffers.
"""
import numpy as np
import pytest

import ns_oracle as O
import nsffn as N
from helpers import rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL32 = 1e-3
EPS = 1e-6


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = N.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def signs(seed, n):
    return np.where(N.synth_normal_f32(seed, n) < 0, -1.0, 1.0).astype(np.float32)


def make_stack(seed, L, D, F, norm=True, host=False):
    """L layers: gate/up Q4_K, down Q6_K on even layers and Q4_K on odd ones; CDNA4 on the
    device.  With host, also the row-major host weights of the last layer."""
    wg, wu, wd, dts, nws, last = [], [], [], [], [], None
    for l in range(L):
        s = N.layer_seed(seed, l)
        dt = N.Q6_K if l % 2 == 0 else N.Q4_K
        hs = (N.synth_weights(N.Q4_K, s + 1, F, D), N.synth_weights(N.Q4_K, s + 2, F, D),
              N.synth_weights(dt, s + 3, D, F))
        dev = []
        for hw, (q, rows, cols) in zip(hs, ((N.Q4_K, F, D), (N.Q4_K, F, D), (dt, D, F))):
            src = torch.from_numpy(hw).cuda()
            dst = torch.empty_like(src)
            N.retile_device(src, dst, q, cols, rows, N.ROW_MAJOR, N.CDNA4)
            dev.append(dst)
        wg.append(dev[0])
        wu.append(dev[1])
        wd.append(dev[2])
        dts.append(dt)
        nws.append(torch.from_numpy(signs(s + 5, D)).cuda() if norm else None)
        if host and l == L - 1:
            last = hs
    torch.cuda.synchronize()
    return wg, wu, wd, dts, (nws if norm else None), last


def run_stack(ctx, st, D, F, x, L=None):
    wg, wu, wd, dts, nws, _ = st
    L = len(wg) if L is None else L
    h = torch.full((F,), float("nan"), dtype=torch.float32, device="cuda")
    y = torch.full((D,), float("nan"), dtype=torch.float32, device="cuda")
    ctx.ffn_stack_decode(wg[:L], wu[:L], wd[:L], dts[:L], N.CDNA4, D, F, x, h, y,
                         norm_weights=None if nws is None else nws[:L], eps=EPS)
    return h, y


def run_blocks(ctx, st, D, F, x):
    wg, wu, wd, dts, nws, _ = st
    h = torch.full((F,), float("nan"), dtype=torch.float32, device="cuda")
    ys = [torch.full((D,), float("nan"), dtype=torch.float32, device="cuda") for _ in range(2)]
    inp = x
    for l in range(len(wg)):
        out = ys[l % 2]
        ctx.ffn_block_decode(wg[l], wu[l], wd[l], dts[l], N.CDNA4, D, F, inp, h, out,
                             norm_weight=None if nws is None else nws[l], eps=EPS)
        inp = out
    return h, inp


def bits(t):
    return t.cpu().numpy().view(np.uint32)


def check_last_layer(st, D, F, x_prev, h, y, norm):
    """The last layer's h and y against the oracle, given the launch's own y after L-1 layers."""
    hg, hu, hd = st[5]
    dt = st[3][-1]
    xp = x_prev.cpu().numpy()
    n = O.rmsnorm(xp, st[4][-1].cpu().numpy(), eps=EPS) if norm else xp
    hh = h.cpu().numpy()
    e1 = rel_err(hh, O.gate_up_geglu(O.ROW_MAJOR, hg, hu, D, F, n))
    e2 = rel_err(y.cpu().numpy(), O.gemv(dt, O.ROW_MAJOR, hd, F, D, hh))
    assert e1 <= TOL32 and e2 <= TOL32, (e1, e2)


def test_stack_48_layers_full_size(ctx):
    D, F, L = 3840, 15360, 48
    st = make_stack(0xD4, L, D, F, norm=True, host=True)
    x = torch.from_numpy(N.synth_normal_f32(0xD5, D)).cuda()
    h1, y1 = run_stack(ctx, st, D, F, x)
    h2, y2 = run_blocks(ctx, st, D, F, x)
    _, y47 = run_stack(ctx, st, D, F, x, L=L - 1)
    ctx.status()
    assert np.isfinite(y1.cpu().numpy()).all()
    assert np.array_equal(bits(y1), bits(y2)) and np.array_equal(bits(h1), bits(h2))
    check_last_layer(st, D, F, y47, h1, y1, True)


SHAPES = [(3840, 15360), (1024, 4096), (768, 1536), (512, 512), (256, 768), (3584, 7168)]


@pytest.mark.parametrize("norm", [False, True], ids=["x", "rms"])
@pytest.mark.parametrize("D,F", SHAPES, ids=[f"{d}x{f}" for d, f in SHAPES])
def test_stack_shapes_equal_blocks(ctx, D, F, norm):
    # without the norm the synthetic chain grows ~100x per layer and overflows fp32 by layer 5
    L = 5 if norm else 2
    st = make_stack(0xD6 + D, L, D, F, norm=norm, host=True)
    x = torch.from_numpy(N.synth_normal_f32(0xD7, D)).cuda()
    h1, y1 = run_stack(ctx, st, D, F, x)
    h2, y2 = run_blocks(ctx, st, D, F, x)
    _, y4 = run_stack(ctx, st, D, F, x, L=L - 1)
    ctx.status()
    assert np.isfinite(y1.cpu().numpy()).all()
    assert np.array_equal(bits(y1), bits(y2)) and np.array_equal(bits(h1), bits(h2))
    check_last_layer(st, D, F, y4, h1, y1, norm)


def test_stack_unsupported_shape_runs_blocks(ctx):
    """4096 columns need 16 compute waves plus the control wave: one block per layer instead."""
    D, F, L = 4096, 8192, 3
    st = make_stack(0xD8, L, D, F, norm=True)
    x = torch.from_numpy(N.synth_normal_f32(0xD9, D)).cuda()
    h1, y1 = run_stack(ctx, st, D, F, x)
    h2, y2 = run_blocks(ctx, st, D, F, x)
    assert np.isfinite(y1.cpu().numpy()).all()
    assert np.array_equal(bits(y1), bits(y2)) and np.array_equal(bits(h1), bits(h2))


def test_stack_more_layers_than_one_launch(ctx):
    """70 layers: the table of one launch holds 64, so two launches chain through y."""
    D, F, L = 512, 1024, 70
    st = make_stack(0xDA, L, D, F, norm=True)
    x = torch.from_numpy(N.synth_normal_f32(0xDB, D)).cuda()
    h1, y1 = run_stack(ctx, st, D, F, x)
    h2, y2 = run_blocks(ctx, st, D, F, x)
    assert np.isfinite(y1.cpu().numpy()).all()
    assert np.array_equal(bits(y1), bits(y2)) and np.array_equal(bits(h1), bits(h2))


def test_stack_in_place_repeated_and_graph(ctx):
    """y aliasing x, three launches in a row (the counters reset after each), and a captured
    graph of two launches replayed three times with host work between, each replay equal to
    the eager result."""
    D, F, L = 3840, 15360, 6
    st = make_stack(0xDC, L, D, F, norm=True)
    x0 = torch.from_numpy(N.synth_normal_f32(0xDD, D)).cuda()
    _, want = run_stack(ctx, st, D, F, x0)
    wg, wu, wd, dts, nws, _ = st
    h = torch.empty(F, dtype=torch.float32, device="cuda")
    for _ in range(3):
        xy = x0.clone()
        ctx.ffn_stack_decode(wg, wu, wd, dts, N.CDNA4, D, F, xy, h, xy, norm_weights=nws, eps=EPS)
        assert np.array_equal(bits(xy), bits(want))
    # two consecutive launches: the second continues from the first's y
    xy = x0.clone()
    ctx.ffn_stack_decode(wg, wu, wd, dts, N.CDNA4, D, F, xy, h, xy, norm_weights=nws, eps=EPS)
    ctx.ffn_stack_decode(wg, wu, wd, dts, N.CDNA4, D, F, xy, h, xy, norm_weights=nws, eps=EPS)
    eager = xy.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    buf = x0.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ctx.ffn_stack_decode(wg, wu, wd, dts, N.CDNA4, D, F, buf, h, buf, norm_weights=nws, eps=EPS)
            ctx.ffn_stack_decode(wg, wu, wd, dts, N.CDNA4, D, F, buf, h, buf, norm_weights=nws, eps=EPS)
    torch.cuda.current_stream().wait_stream(s)
    for r in range(3):
        buf.copy_(x0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(buf), bits(eager)), r
        _ = torch.randn(1000, device="cuda").sum().item()  # eager work between replays
    ctx.status()


def test_stack_bounded_wait(ctx, tune):
    """Every wait bounded: forced down to one poll from the host (every wave still exits
    normally), a wait runs out, y is all NaN and the status reports it once; the next launch
    with the default bound is exact (the last workgroup out reset the counters)."""
    D, F, L = 3840, 15360, 4
    st = make_stack(0xDE, L, D, F, norm=True)
    x = torch.from_numpy(N.synth_normal_f32(0xDF, D)).cuda()
    _, want = run_stack(ctx, st, D, F, x)
    ctx.status()
    tune("block_spin", 1)
    _, got = run_stack(ctx, st, D, F, x)
    g = got.cpu().numpy()
    if np.isnan(g).any():
        assert np.isnan(g).all()
        with pytest.raises(N.NsError, match="multi-layer decode") as e:
            ctx.status()
        assert e.value.code == 7  # NS_ERR_TIMEOUT
    else:
        assert np.array_equal(g.view(np.uint32), bits(want))
    ctx.status()
    tune("block_spin", 0)
    _, again = run_stack(ctx, st, D, F, x)
    assert np.array_equal(bits(again), bits(want))
    ctx.status()


def test_stack_wait_free_and_tuning_equal(ctx, tune):
    D, F, L = 3840, 15360, 4
    st = make_stack(0xE0, L, D, F, norm=True)
    x = torch.from_numpy(N.synth_normal_f32(0xE1, D)).cuda()
    _, want = run_stack(ctx, st, D, F, x)
    tune("stack_fused", 0)
    _, per_layer = run_stack(ctx, st, D, F, x)
    tune("stack_fused", 1)
    wf = N.Context(0)
    try:
        wf.set_wait_free(True)
        _, free = run_stack(wf, st, D, F, x)
        wf.status()
    finally:
        torch.cuda.synchronize()
        wf.close()
    assert np.array_equal(bits(per_layer), bits(want)) and np.array_equal(bits(free), bits(want))


def test_stack_argument_errors(ctx):
    D, F = 512, 1024
    st = make_stack(0xE2, 2, D, F, norm=True)
    wg, wu, wd, dts, nws, _ = st
    x = torch.zeros(D, dtype=torch.float32, device="cuda")
    h = torch.zeros(F, dtype=torch.float32, device="cuda")
    with pytest.raises(N.NsError, match="h overlaps"):
        ctx.ffn_stack_decode(wg, wu, wd, dts, N.CDNA4, D, F, x, h, h, norm_weights=nws)
    with pytest.raises(N.NsError):
        ctx.ffn_stack_decode([], [], [], [], N.CDNA4, D, F, x, h, x)
    with pytest.raises(N.NsError, match="type"):
        ctx.ffn_stack_decode(wg, wu, wd, [N.Q4_K, 3], N.CDNA4, D, F, x, h, x, norm_weights=nws)


def test_stack_epochs_across_launch_lengths(ctx):
    """Launches of different lengths and shapes alternate on one context (the epoch advances per
    launch, the tagged buffers are shared): every launch equals its per-layer blocks, so no
    launch reads a value an earlier one left behind."""
    big = make_stack(0xE4, 6, 3840, 15360, norm=True)
    small = make_stack(0xE6, 3, 1024, 4096, norm=True)
    xb = torch.from_numpy(N.synth_normal_f32(0xE5, 3840)).cuda()
    xs = torch.from_numpy(N.synth_normal_f32(0xE7, 1024)).cuda()
    for st, D, F, x, Ls in ((big, 3840, 15360, xb, (1, 6, 2)), (small, 1024, 4096, xs, (3, 1)),
                            (big, 3840, 15360, xb, (6, 1))):
        for L in Ls:
            sub = tuple(v[:L] if isinstance(v, list) else v for v in st)
            _, y1 = run_stack(ctx, sub, D, F, x)
            _, y2 = run_blocks(ctx, sub, D, F, x)
            assert np.array_equal(bits(y1), bits(y2)), (D, L)
    ctx.status()


def test_stack_grows_its_tagged_buffers(ctx):
    """A shape past the model's (16384 ffn rows: 256 workgroups, one per CU) grows the context's
    tagged h buffer; the result equals the per-layer blocks."""
    D, F, L = 2048, 16384, 3
    st = make_stack(0xE8, L, D, F, norm=True)
    x = torch.from_numpy(N.synth_normal_f32(0xE9, D)).cuda()
    h1, y1 = run_stack(ctx, st, D, F, x)
    h2, y2 = run_blocks(ctx, st, D, F, x)
    ctx.status()
    assert np.isfinite(y1.cpu().numpy()).all()
    assert np.array_equal(bits(y1), bits(y2)) and np.array_equal(bits(h1), bits(h2))
