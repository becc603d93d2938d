"""Shared test helpers: tolerance metric and block builders."""
import numpy as np


def rel_err(got, ref):
    """Max relative error as fixed for this build: for every output row (token),
    max_i |got_i - ref_i| / max_i |ref_i|; the worst row is returned.  A plain
    element-wise ratio is ill-conditioned on near-zero outputs."""
    got = np.atleast_2d(np.asarray(got, dtype=np.float64))
    ref = np.atleast_2d(np.asarray(ref, dtype=np.float64))
    assert got.shape == ref.shape, (got.shape, ref.shape)
    num = np.max(np.abs(got - ref), axis=1)
    den = np.maximum(np.max(np.abs(ref), axis=1), 1e-30)
    return float(np.max(num / den))


def f16_bits(x):
    return np.asarray(x, dtype=np.float16).view(np.uint16)


def f16_value(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def q4k_block(d, dmin, sc, m, q):
    """Pack a Q4_K block from fp16 d/dmin, 8 six-bit scales/mins and 256 nibbles
    (inverse of the unpack in src/native/quant.cpp:11)."""
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = f16_bits(np.float16(d)).reshape(1).view(np.uint8)
    b[2:4] = f16_bits(np.float16(dmin)).reshape(1).view(np.uint8)
    s = np.zeros(12, dtype=np.int64)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    b[4:16] = s.astype(np.uint8)
    q = np.asarray(q, dtype=np.int64)
    for g in range(8):
        for l in range(32):
            i = (g // 2) * 32 + l
            if g & 1:
                b[16 + i] |= (q[g * 32 + l] & 15) << 4
            else:
                b[16 + i] |= q[g * 32 + l] & 15
    return b


def q6k_block(d, sc, v):
    """Pack a Q6_K block from fp16 d, 16 int8 scales and 256 six-bit values
    (inverse of src/native/quant.cpp:13-18)."""
    b = np.zeros(210, dtype=np.uint8)
    v = np.asarray(v, dtype=np.int64)
    for i in range(256):
        half, p = divmod(i, 128)
        quarter, l = divmod(p, 32)
        lo, hi = v[i] & 15, v[i] >> 4
        lq = half * 64 + l + (32 if quarter in (1, 3) else 0)
        b[lq] |= lo << (4 if quarter >= 2 else 0)
        b[128 + half * 32 + l] |= hi << (2 * quarter)
    b[192:208] = np.asarray(sc, dtype=np.int8).view(np.uint8)
    b[208:210] = f16_bits(np.float16(d)).reshape(1).view(np.uint8)
    return b
