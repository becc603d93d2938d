"""Prefill inputs whose 32-wide groups sum past fp16's range.

The FP32-mode Q4_K GEMMs take the min term -dmin * sum_g m_g * S_g(x) as MFMAs over
the group sums S_g of x, held as fp16 hi + lo.  An fp16 activation reaches 65504,
so a group of 32 can sum to 2^21: large activations (the down projection's input is
the fp16 GeGLU output) must not turn those sums into inf.  Each test puts one group
of every token at +-2100 (|S_g| = 67200) and checks the result against the oracle,
which sums exactly.
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


def big_group_tokens(seed, batch, cols, tokens=None):
    """fp16 bits [batch][cols]: N(0,1) with one 32-wide group at +-2100 in each of `tokens`
    (default: every token)."""
    x = N.synth_normal_f16(seed, batch * cols).reshape(batch, cols).view(np.float16).copy()
    rng = np.random.default_rng(seed)
    for t in (range(batch) if tokens is None else tokens):
        g = int(rng.integers(0, cols // 32))
        x[t, 32 * g:32 * g + 32] = np.float16(2100.0 if t % 2 else -2100.0)
    return x.view(np.uint16)


@pytest.mark.parametrize("layout", [N.CDNA4, N.NSMFFN, N.ROW_MAJOR], ids=LNAME.get)
def test_q4k_prefill_large_group_sums(ctx, layout):
    cols, rows, batch = 2048, 256, 72
    host = N.synth_weights(N.Q4_K, 0x90, rows, cols)
    lay = host if layout == N.ROW_MAJOR else N.retile(host, N.Q4_K, cols, rows, N.ROW_MAJOR, layout)
    w = torch.from_numpy(np.ascontiguousarray(lay)).cuda()
    xb = big_group_tokens(0x91, batch, cols)
    y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    ctx.ffn_down(w, N.Q4_K, layout, cols, rows, batch, torch.from_numpy(xb.view(np.int16)).cuda(), y,
                 half_input=True, fast_swa=False)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.isfinite(got).all()
    assert rel_err(got, O.gemm(N.Q4_K, O.ROW_MAJOR, host, cols, rows, batch, xb, 0)) <= 1e-3


@pytest.mark.parametrize("layout", [N.CDNA4, N.ROW_MAJOR], ids=LNAME.get)
def test_q4k_prefill_some_tokens_rescaled(ctx, tune, layout):
    """Rescaled tokens in some 256-token blocks only (the first 128-token tile of block 0,
    the second tile of block 1 and the ragged tail), so tiles read x and the copy side by
    side; at several split-K counts."""
    cols, rows, batch = 2048, 256, 600
    host = N.synth_weights(N.Q4_K, 0x95, rows, cols)
    lay = host if layout == N.ROW_MAJOR else N.retile(host, N.Q4_K, cols, rows, N.ROW_MAJOR, layout)
    w = torch.from_numpy(np.ascontiguousarray(lay)).cuda()
    xb = big_group_tokens(0x96, batch, cols, tokens=[5, 127, 390, 599])
    want = O.gemm(N.Q4_K, O.ROW_MAJOR, host, cols, rows, batch, xb, 0)
    xd = torch.from_numpy(xb.view(np.int16)).cuda()
    for kparts in (0, 1, 4):
        tune("gemm_kparts", kparts)
        y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
        ctx.ffn_down(w, N.Q4_K, layout, cols, rows, batch, xd, y, half_input=True, fast_swa=False)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.isfinite(got).all(), kparts
        assert rel_err(got, want) <= 1e-3, kparts
        for t in (0, 200, 300, 598):  # tokens without a large group, in flagged and unflagged blocks
            assert rel_err(got[t], want[t]) <= 1e-3, (kparts, t)


@pytest.mark.parametrize("layout", [N.CDNA4, N.ROW_MAJOR], ids=LNAME.get)
def test_gate_up_prefill_large_group_sums(ctx, layout):
    """The pair at FP32 mode.  d and dmin are divided by 1024 so that h = gelu(g) * u stays
    within fp16 (|h| <= 2822 here; at 1/64 it reaches 7e5, which the fp16 output holds as inf
    in the reference too)."""
    cols, rows, batch = 1024, 256, 40
    hosts = []
    for seed in (0x92, 0x93):
        blk = N.synth_weights(N.Q4_K, seed, rows, cols).reshape(-1, 144).copy()
        for off in (0, 2):  # d and dmin / 1024
            v = blk[:, off:off + 2].copy().view(np.float16)
            blk[:, off:off + 2] = (v / np.float16(1024)).astype(np.float16).view(np.uint8)
        hosts.append(blk.reshape(-1))
    devs = []
    for h in hosts:
        lay = h if layout == N.ROW_MAJOR else N.retile(h, N.Q4_K, cols, rows, N.ROW_MAJOR, layout)
        devs.append(torch.from_numpy(np.ascontiguousarray(lay)).cuda())
    xb = big_group_tokens(0x94, batch, cols)
    out = torch.empty((batch, rows), dtype=torch.int16, device="cuda")
    ctx.gate_up_geglu_rm32(devs[0], devs[1], layout, cols, rows, batch, torch.from_numpy(xb.view(np.int16)).cuda(),
                           out, False)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.float16).astype(np.float32)
    ref = O.gate_up_geglu_prefill(O.ROW_MAJOR, hosts[0], hosts[1], cols, rows, batch, xb, 0)
    assert np.abs(ref).max() < 65504
    assert np.isfinite(got).all()
    assert rel_err(got, ref) <= 1e-3
