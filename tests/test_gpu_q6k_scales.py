"""Q6_K tensors with the int8 scales real GGUF files carry.

The generator of BASELINE's configs draws Q6_K scales in -32..31, but a Q6_K
super-block as llama.cpp quantises it puts its largest group at a scale near
+-127 (or -128), so real tensors reach the whole int8 range.  Every path that
reads Q6_K weights is run here on blocks whose scales span -128..127 (each
block has one group at -128 or 127, and six-bit values at 0 and 63), against
the oracle: the prefill GEMM in both accumulation modes and every layout, the
decode GEMV, the one-launch decode block, batch 2-4, the dequantisation check
hook and the embedding (bit-exact).  Bars as elsewhere:
FP32 mode 1e-3, FP16 mode 1e-2 against the FP32 oracle and 1e-3 against the
FP16-mode oracle.
"""
import numpy as np
import pytest

import ns_oracle as O
import nsffn as N
from helpers import f16_value, q6k_block, rel_err

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


def full_range_q6k(seed, rows, cols, d_lo=1e-4, d_hi=2e-3):
    """Row-major Q6_K blocks: scales uniform in -128..127 with one group of each block at
    -128 or 127, six-bit values uniform with runs at 63 and 0, |d| uniform in [d_lo, d_hi] with
    either sign (llama.cpp's Q6_K quantiser stores d = 1/iscale with iscale = -128/max, so d is
    usually negative)."""
    rng = np.random.default_rng(seed)
    nb = rows * cols // 256
    blocks = []
    for i in range(nb):
        sc = rng.integers(-128, 128, 16)
        sc[i % 16] = -128 if i % 2 else 127
        v = rng.integers(0, 64, 256)
        v[(i % 8) * 32:(i % 8) * 32 + 8] = 63
        v[(i % 8) * 32 + 8:(i % 8) * 32 + 16] = 0
        d = rng.uniform(d_lo, d_hi) * (-1.0 if rng.random() < 0.75 else 1.0)
        blocks.append(q6k_block(np.float16(d), sc, v))
    return np.concatenate(blocks)


def on_device(host, cols, rows, layout):
    lay = host if layout == N.ROW_MAJOR else N.retile(host, N.Q6_K, cols, rows, N.ROW_MAJOR, layout)
    return torch.from_numpy(np.ascontiguousarray(lay)).cuda()


@pytest.mark.parametrize("layout", [N.CDNA4, N.NSMFFN, N.ROW_MAJOR], ids=LNAME.get)
@pytest.mark.parametrize("fast", [False, True], ids=["fp32acc", "fp16acc"])
def test_prefill_down_full_range_scales(ctx, layout, fast):
    cols, rows, batch = 2048, 256, 96
    host = full_range_q6k(0x7A, rows, cols)
    w = on_device(host, cols, rows, layout)
    xb = N.synth_normal_f16(0x7B, batch * cols).reshape(batch, cols)
    y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    ctx.ffn_down(w, N.Q6_K, layout, cols, rows, batch, torch.from_numpy(xb.view(np.int16)).cuda(), y,
                 half_input=True, fast_swa=fast)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.isfinite(got).all()
    ref32 = O.gemm(N.Q6_K, O.ROW_MAJOR, host, cols, rows, batch, xb, 0)
    if fast:
        assert rel_err(got, ref32) <= 1e-2
        assert rel_err(got, O.gemm(N.Q6_K, O.ROW_MAJOR, host, cols, rows, batch, xb, 1)) <= 1e-3
    else:
        assert rel_err(got, ref32) <= 1e-3


def test_prefill_down_full_range_scales_power_of_two_d(ctx):
    """A row whose largest d is a power of two, with sc = -128: a row scale of 2^-(15 + ceil(log2 M))
    would make d*c_r exactly 2^-15 and the FP16-mode tile factor A = d*sc*2^24*c_r = -2^16, one
    past fp16's range; the Q6_K row scale takes the power of two strictly above M instead."""
    cols, rows, batch = 1024, 128, 64
    host = full_range_q6k(0x7C, rows, cols)
    blk = host.reshape(-1, 210).copy()
    blk[:, 208:210] = np.frombuffer(np.float16(2.0 ** -10).tobytes(), dtype=np.uint8)  # every d = 2^-10
    blk[:, 192:208] = np.where(np.arange(16) % 3 == 0, np.uint8(0x80), blk[:, 192:208])  # sc -128
    host = blk.reshape(-1)
    for layout in (N.CDNA4, N.ROW_MAJOR):
        w = on_device(host, cols, rows, layout)
        xb = N.synth_normal_f16(0x7D, batch * cols).reshape(batch, cols)
        for fast in (False, True):
            y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
            ctx.ffn_down(w, N.Q6_K, layout, cols, rows, batch, torch.from_numpy(xb.view(np.int16)).cuda(), y,
                         half_input=True, fast_swa=fast)
            torch.cuda.synchronize()
            got = y.cpu().numpy()
            assert np.isfinite(got).all(), (LNAME[layout], fast)
            ref = O.gemm(N.Q6_K, O.ROW_MAJOR, host, cols, rows, batch, xb, 1 if fast else 0)
            assert rel_err(got, ref) <= 1e-3, (LNAME[layout], fast)


@pytest.mark.parametrize("layout", [N.CDNA4, N.NSMFFN, N.ROW_MAJOR], ids=LNAME.get)
def test_decode_gemv_full_range_scales(ctx, layout):
    cols, rows = 3840, 512
    host = full_range_q6k(0x7E, rows, cols)
    w = on_device(host, cols, rows, layout)
    x = N.synth_normal_f32(0x7F, cols)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.matmul(w, N.Q6_K, layout, cols, rows, 1, torch.from_numpy(x).cuda(), y)
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), O.gemv(N.Q6_K, O.ROW_MAJOR, host, cols, rows, x)) <= 1e-3


@pytest.mark.parametrize("batch", [2, 4])
def test_small_batch_down_full_range_scales(ctx, batch):
    cols, rows = 2048, 256
    host = full_range_q6k(0x80, rows, cols)
    for layout in (N.CDNA4, N.NSMFFN):
        w = on_device(host, cols, rows, layout)
        xb = N.synth_normal_f16(0x81, batch * cols).reshape(batch, cols)
        y = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
        ctx.ffn_down(w, N.Q6_K, layout, cols, rows, batch, torch.from_numpy(xb.view(np.int16)).cuda(), y,
                     half_input=True, fast_swa=False)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        xf = f16_value(xb).astype(np.float32)
        for t in range(batch):
            assert rel_err(got[t], O.gemv(N.Q6_K, O.ROW_MAJOR, host, cols, rows, xf[t])) <= 1e-3, (LNAME[layout], t)


def test_decode_block_full_range_scales(ctx):
    """The one-launch decode block at the model's shape with a full-range Q6_K down."""
    D, F = 3840, 15360
    g = N.synth_weights(N.Q4_K, 0x82, F, D)
    u = N.synth_weights(N.Q4_K, 0x83, F, D)
    dn = full_range_q6k(0x84, D, F)
    dev = [torch.from_numpy(N.retile(a, t, c, r, N.ROW_MAJOR, N.CDNA4)).cuda()
           for a, t, c, r in ((g, N.Q4_K, D, F), (u, N.Q4_K, D, F), (dn, N.Q6_K, F, D))]
    x = N.synth_normal_f32(0x85, D)
    h = torch.empty(F, dtype=torch.float32, device="cuda")
    y = torch.empty(D, dtype=torch.float32, device="cuda")
    ctx.ffn_block_decode(dev[0], dev[1], dev[2], N.Q6_K, N.CDNA4, D, F, torch.from_numpy(x).cuda(), h, y)
    torch.cuda.synchronize()
    href = O.gate_up_geglu(O.ROW_MAJOR, g, u, D, F, x)
    yref = O.gemv(N.Q6_K, O.ROW_MAJOR, dn, F, D, href.astype(np.float32))
    assert rel_err(y.cpu().numpy(), yref) <= 1e-3


@pytest.mark.parametrize("layout", [N.CDNA4, N.NSMFFN, N.ROW_MAJOR], ids=LNAME.get)
def test_dequant_and_embedding_full_range_scales(ctx, layout):
    """The check hook and the token embedding stay bit-exact at int8 scales -128..127."""
    cols, rows = 1024, 128
    host = full_range_q6k(0x86, rows, cols)
    w = on_device(host, cols, rows, layout)
    out32 = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    out16 = torch.empty((rows, cols), dtype=torch.int16, device="cuda")
    ctx.dequant(w, N.Q6_K, layout, cols, rows, 0, rows, out32, out16)
    ids = np.array([0, rows - 1, 77, 77], dtype=np.int32)
    scale = np.float32(np.sqrt(3840.0))
    emb = torch.empty((len(ids), cols), dtype=torch.float32, device="cuda")
    ctx.embedding(w, N.Q6_K, layout, cols, rows, torch.from_numpy(ids).cuda(), len(ids), float(scale), emb)
    torch.cuda.synchronize()
    want = O.dequant_rows(N.Q6_K, O.ROW_MAJOR, host, cols, rows)
    assert np.array_equal(out32.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert np.array_equal(out16.cpu().numpy().view(np.uint16), want.astype(np.float16).view(np.uint16))
    got = emb.cpu().numpy()
    for t, r in enumerate(ids):
        np.testing.assert_array_equal(got[t].view(np.uint32), (scale * want[r]).astype(np.float32).view(np.uint32))
