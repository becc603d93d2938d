"""GPU parity of the decode FFN block in one launch (ns_ffn_block_decode: rms at mm:563 when a
norm weight is given, gate/up + GeGLU at mm:571, down at mm:573).

  * h and y against the CPU oracle (O.rmsnorm, O.gate_up_geglu, O.gemv), FP32 bar
    rel_err <= 1e-3, for both down types, with and without the norm, at the model's shape,
    at 4096 columns (16 waves per workgroup) and at smaller shapes whose column parts number
    1, 2, 3 and 4;
  * at the model's shape (3840 x 15360) bit for bit against the same block as two launches
    (tuning key block_fused 0: the pair GEMV, then the down GEMV): the one-launch kernel keeps
    their arithmetic and order per row;
  * repeated launches (the kernel resets its own counters), y aliasing x, a shape and a layout
    the kernel does not take (the two-launch path runs instead), overlapping h rejected, and a
    HIP graph of several blocks replayed against the eager result.
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
TNAME = {N.Q4_K: "q4k", N.Q6_K: "q6k"}


@pytest.fixture(scope="module")
def ctx():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = N.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def layer(seed, D, F, dt, layout=N.CDNA4):
    """Host weights (row-major) and device weights in `layout` of one block."""
    hs = (N.synth_weights(N.Q4_K, seed + 1, F, D), N.synth_weights(N.Q4_K, seed + 2, F, D),
          N.synth_weights(dt, seed + 3, D, F))
    dims = ((N.Q4_K, F, D), (N.Q4_K, F, D), (dt, D, F))
    devs = []
    for h, (q, rows, cols) in zip(hs, dims):
        lay = h if layout == N.ROW_MAJOR else N.retile(h, q, cols, rows, N.ROW_MAJOR, layout)
        devs.append(torch.from_numpy(np.ascontiguousarray(lay)).cuda())
    return hs, devs


def norm_vec(seed, n):
    return (np.random.default_rng(seed).standard_normal(n) + 1.0).astype(np.float32)


def run(ctx, devs, dt, D, F, x, nw, layout=N.CDNA4):
    h = torch.full((F,), float("nan"), dtype=torch.float32, device="cuda")
    y = torch.full((D,), float("nan"), dtype=torch.float32, device="cuda")
    ctx.ffn_block_decode(devs[0], devs[1], devs[2], dt, layout, D, F, x, h, y, norm_weight=nw, eps=EPS)
    torch.cuda.synchronize()
    return h.cpu().numpy(), y.cpu().numpy()


def oracle(hs, dt, D, F, x, nw):
    xn = x if nw is None else O.rmsnorm(x, nw, eps=EPS)
    h = O.gate_up_geglu(O.ROW_MAJOR, hs[0], hs[1], D, F, xn)
    return h, O.gemv(dt, O.ROW_MAJOR, hs[2], F, D, h)


@pytest.mark.parametrize("norm", [False, True], ids=["plain", "rms"])
@pytest.mark.parametrize("dt", [N.Q6_K, N.Q4_K], ids=TNAME.get)
@pytest.mark.parametrize("shape", [(3840, 15360), (4096, 8192), (1024, 4096), (512, 512), (256, 768), (768, 1536)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_block_decode_matches_oracle(ctx, shape, dt, norm):
    D, F = shape
    hs, devs = layer(N.layer_seed(0xB0, D + F + dt), D, F, dt)
    x = N.synth_normal_f32(0xB1 + D, D)
    nw = norm_vec(0xB2, D) if norm else None
    h, y = run(ctx, devs, dt, D, F, torch.from_numpy(x).cuda(), None if nw is None else torch.from_numpy(nw).cuda())
    href, _ = oracle(hs, dt, D, F, x, nw)
    assert np.isfinite(h).all() and np.isfinite(y).all()
    assert rel_err(h, href) <= TOL32
    # the down projection checked on the GPU's own h, as the two-launch tests do
    assert rel_err(y, O.gemv(dt, O.ROW_MAJOR, hs[2], F, D, h)) <= TOL32


@pytest.mark.parametrize("norm", [False, True], ids=["plain", "rms"])
@pytest.mark.parametrize("dt", [N.Q6_K, N.Q4_K], ids=TNAME.get)
def test_block_decode_equals_two_launches(ctx, tune, dt, norm):
    """Model shape: the one-launch block equals the two launches bit for bit, in h and y."""
    D, F = 3840, 15360
    _, devs = layer(N.layer_seed(0xB3, dt), D, F, dt)
    x = torch.from_numpy(N.synth_normal_f32(0xB4, D)).cuda()
    nw = torch.from_numpy(norm_vec(0xB5, D)).cuda() if norm else None
    h1, y1 = run(ctx, devs, dt, D, F, x, nw)
    tune("block_fused", 0)
    h2, y2 = run(ctx, devs, dt, D, F, x, nw)
    assert np.array_equal(h1.view(np.uint32), h2.view(np.uint32))
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


def test_block_decode_repeats_and_aliasing(ctx):
    """Ten launches in a row on one stream (the counters reset themselves: each result equals
    the first), then a chain of five blocks with y written over x, equal to the same chain
    with separate buffers."""
    D, F, dt = 3840, 15360, N.Q6_K
    _, devs = layer(N.layer_seed(0xB6, 0), D, F, dt)
    x0 = torch.from_numpy(N.synth_normal_f32(0xB7, D)).cuda()
    nw = torch.from_numpy(norm_vec(0xB8, D)).cuda()
    h = torch.empty(F, dtype=torch.float32, device="cuda")
    ys = [torch.empty(D, dtype=torch.float32, device="cuda") for _ in range(10)]
    for y in ys:
        ctx.ffn_block_decode(devs[0], devs[1], devs[2], dt, N.CDNA4, D, F, x0, h, y, norm_weight=nw, eps=EPS)
    torch.cuda.synchronize()
    for i, y in enumerate(ys[1:]):
        assert torch.equal(y, ys[0]), i + 1
    xa = x0.clone()
    xb = x0.clone()
    yb = torch.empty(D, dtype=torch.float32, device="cuda")
    for _ in range(5):
        ctx.ffn_block_decode(devs[0], devs[1], devs[2], dt, N.CDNA4, D, F, xa, h, xa, norm_weight=nw, eps=EPS)
        ctx.ffn_block_decode(devs[0], devs[1], devs[2], dt, N.CDNA4, D, F, xb, h, yb, norm_weight=nw, eps=EPS)
        xb, yb = yb, xb
    torch.cuda.synchronize()
    assert torch.isfinite(xa).all() and torch.equal(xa, xb)


@pytest.mark.parametrize("case", ["parts_not_whole", "nsmffn_layout", "rowmajor_layout"])
def test_block_decode_fallback(ctx, case):
    """Shapes and layouts the one-launch kernel does not take run as two launches: 768 x 1024
    (4 down super-blocks per row do not split into parts of 3) and the two other layouts."""
    D, F = (768, 1024) if case == "parts_not_whole" else (512, 1024)
    layout = {"parts_not_whole": N.CDNA4, "nsmffn_layout": N.NSMFFN, "rowmajor_layout": N.ROW_MAJOR}[case]
    dt = N.Q6_K
    hs, devs = layer(N.layer_seed(0xB9, D), D, F, dt, layout)
    x, nw = N.synth_normal_f32(0xBA, D), norm_vec(0xBB, D)
    h, y = run(ctx, devs, dt, D, F, torch.from_numpy(x).cuda(), torch.from_numpy(nw).cuda(), layout)
    href, _ = oracle(hs, dt, D, F, x, nw)
    assert rel_err(h, href) <= TOL32
    assert rel_err(y, O.gemv(dt, O.ROW_MAJOR, hs[2], F, D, h)) <= TOL32


def test_block_decode_rejects_overlapping_h(ctx):
    D, F, dt = 512, 1024, N.Q6_K
    _, devs = layer(N.layer_seed(0xBC, 0), D, F, dt)
    buf = torch.zeros(F + D, dtype=torch.float32, device="cuda")
    y = torch.empty(D, dtype=torch.float32, device="cuda")
    tail = buf[F - 64:F - 64 + D]  # its first 64 floats are h's last
    with pytest.raises(N.NsError, match="h overlaps x"):
        ctx.ffn_block_decode(devs[0], devs[1], devs[2], dt, N.CDNA4, D, F, tail, buf[:F], y)
    with pytest.raises(N.NsError, match="h overlaps y"):
        ctx.ffn_block_decode(devs[0], devs[1], devs[2], dt, N.CDNA4, D, F, y, buf[:F], tail)
    ctx.ffn_block_decode(devs[0], devs[1], devs[2], dt, N.CDNA4, D, F, buf[F:], buf[:F], y)  # adjacent is fine
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()


def test_block_decode_graph_replay(ctx):
    """Eight blocks (alternating Q6_K / Q4_K downs, the norm in each, y over x) captured into a
    HIP graph and replayed three times with eager work between: every replay equals the eager
    chain bit for bit."""
    D, F = 3840, 15360
    blocks = []
    for l in range(8):
        dt = N.Q6_K if l % 2 == 0 else N.Q4_K
        _, devs = layer(N.layer_seed(0xBD, l), D, F, dt)
        blocks.append((devs, dt, torch.from_numpy(norm_vec(0xBE + l, D)).cuda()))
    x0 = torch.from_numpy(N.synth_normal_f32(0xBF, D)).cuda()
    x = x0.clone()
    h = torch.empty(F, dtype=torch.float32, device="cuda")

    def chain():
        for devs, dt, nw in blocks:
            ctx.ffn_block_decode(devs[0], devs[1], devs[2], dt, N.CDNA4, D, F, x, h, x, norm_weight=nw, eps=EPS)

    chain()
    torch.cuda.synchronize()
    eager = x.clone()
    x.copy_(x0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain()
    for r in range(3):
        x.copy_(x0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(x, eager), f"replay {r}"
        x.copy_(x0)
        chain()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(x, eager)


def test_block_decode_bounded_wait(tune, ctx):
    """The down workgroups' wait for h is bounded.  With the bound forced down to one poll
    (from the host: every wave still exits normally), a slab whose wait ran out is written
    as NaN and every other slab is the normal result; the context's status reports the
    timeout exactly when a slab ran out (ns_ctx_status, NS_ERR_TIMEOUT), once; the next
    launch with the default bound is whole again (the kernel clears its counters) and
    reports nothing."""
    D, F, dt = 3840, 15360, N.Q6_K
    _, devs = layer(N.layer_seed(0xC0, 0), D, F, dt)
    x = torch.from_numpy(N.synth_normal_f32(0xC1, D)).cuda()
    _, want = run(ctx, devs, dt, D, F, x, None)
    ctx.status()
    tune("block_spin", 1)
    _, got = run(ctx, devs, dt, D, F, x, None)
    slabs = got.reshape(-1, 64)
    ran_out = int(np.isnan(slabs[:, 0]).sum())
    if ran_out:
        with pytest.raises(N.NsError, match="decode FFN block") as e:
            ctx.status()
        assert e.value.code == 7  # NS_ERR_TIMEOUT
    ctx.status()  # reported once, then clear
    tune("block_spin", 0)
    _, again = run(ctx, devs, dt, D, F, x, None)
    for s, row in enumerate(slabs):
        assert np.isnan(row).all() or np.array_equal(row.view(np.uint32), want.reshape(-1, 64)[s].view(np.uint32)), s
    print(f"bounded wait: {ran_out} of {len(slabs)} slabs ran out")
    assert np.array_equal(again.view(np.uint32), want.view(np.uint32))
    ctx.status()
