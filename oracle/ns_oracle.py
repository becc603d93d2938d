"""ctypes binding of the CPU oracle (oracle/libns_oracle.so) and of oracle/_ref.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU baseline.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libns_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libns_ref_quant.so")

Q4_K, Q6_K = 12, 14
ROW_MAJOR, NSMFFN = 0, 1

_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        vp, u64, i32, f32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_float
        L.nso_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.nso_f16_to_f32.restype = f32
        L.nso_f32_to_f16.argtypes = [f32]
        L.nso_f32_to_f16.restype = ctypes.c_uint16
        L.nso_round_f16p.argtypes = [f32]
        L.nso_round_f16p.restype = f32
        L.nso_q4k_value.argtypes = [vp, ctypes.c_uint32]
        L.nso_q4k_value.restype = f32
        L.nso_q6k_value.argtypes = [vp, ctypes.c_uint32]
        L.nso_q6k_value.restype = f32
        L.nso_block_index.argtypes = [i32, u64, u64, u64]
        L.nso_block_index.restype = u64
        L.nso_dequant_row.argtypes = [i32, i32, vp, u64, u64, u64, vp]
        L.nso_dot_row.argtypes = [i32, i32, vp, u64, u64, u64, vp]
        L.nso_dot_row.restype = f32
        L.nso_gemv.argtypes = [i32, i32, vp, u64, u64, vp, vp, i32]
        L.nso_gelu_tanh.argtypes = [f32]
        L.nso_gelu_tanh.restype = f32
        L.nso_gate_up_geglu.argtypes = [i32, vp, vp, u64, u64, vp, vp, i32]
        L.nso_gemm.argtypes = [i32, i32, vp, u64, u64, u64, vp, i32, vp, i32]
        L.nso_gate_up_geglu_prefill.argtypes = [i32, vp, vp, u64, u64, u64, vp, i32, vp, i32]
        L.nso_rmsnorm.argtypes = [vp, vp, vp, vp, vp, u64, u64, f32, vp, vp]
        _lib = L
    return _lib


def ref():
    """The reference's own quant.cpp (compiled by oracle/Makefile), or None."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        R = ctypes.CDLL(REF_PATH)
        vp, u64, i32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int
        R.nsref_dequant.argtypes = [i32, vp, u64, u64, u64, u64, vp]
        R.nsref_dot_row.argtypes = [i32, vp, u64, u64, u64, vp, vp]
        _ref = R
    return _ref


def _p(a):
    return None if a is None else a.ctypes.data


def _nt(n):
    return n or max(1, min(16, os.cpu_count() or 1))


def dequant_rows(qtype, layout, w, cols, rows, row0=0, nrows=None):
    nrows = rows - row0 if nrows is None else nrows
    out = np.empty((nrows, cols), dtype=np.float32)
    for i in range(nrows):
        rc = lib().nso_dequant_row(qtype, layout, _p(w), cols, rows, row0 + i, _p(out[i]))
        assert rc == 0
    return out


def dot_row(qtype, layout, w, cols, rows, row, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().nso_dot_row(qtype, layout, _p(w), cols, rows, row, _p(x))


def gemv(qtype, layout, w, cols, rows, x, nthreads=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    assert lib().nso_gemv(qtype, layout, _p(w), cols, rows, _p(x), _p(y), _nt(nthreads)) == 0
    return y


def gate_up_geglu(layout, wg, wu, cols, rows, x, nthreads=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    h = np.empty(rows, dtype=np.float32)
    assert lib().nso_gate_up_geglu(layout, _p(wg), _p(wu), cols, rows, _p(x), _p(h), _nt(nthreads)) == 0
    return h


def gemm(qtype, layout, w, cols, rows, batch, x_f16, acc_mode, nthreads=None):
    x_f16 = np.ascontiguousarray(x_f16, dtype=np.uint16)
    out = np.empty((batch, rows), dtype=np.float32)
    assert lib().nso_gemm(qtype, layout, _p(w), cols, rows, batch, _p(x_f16), acc_mode, _p(out),
                          _nt(nthreads)) == 0
    return out


def gate_up_geglu_prefill(layout, wg, wu, cols, rows, batch, x_f16, acc_mode, nthreads=None):
    x_f16 = np.ascontiguousarray(x_f16, dtype=np.uint16)
    h = np.empty((batch, rows), dtype=np.float32)
    assert lib().nso_gate_up_geglu_prefill(layout, _p(wg), _p(wu), cols, rows, batch, _p(x_f16), acc_mode,
                                           _p(h), _nt(nthreads)) == 0
    return h


def gelu_tanh(g):
    return lib().nso_gelu_tanh(g)


def rmsnorm(x, w, residual=None, scale=None, next_w=None, eps=1e-6):
    """metal:509-529 per row of x ([rows][width] or [width]): returns y, or (y, next) with next_w.
    scale is a Python float (the reference reads it from a one-float tensor)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    rows, width = x2.shape
    w = np.ascontiguousarray(w, dtype=np.float32)
    res = None if residual is None else np.ascontiguousarray(residual, dtype=np.float32).reshape(rows, width)
    sc = None if scale is None else np.array([scale], dtype=np.float32)
    nw = None if next_w is None else np.ascontiguousarray(next_w, dtype=np.float32)
    y = np.empty((rows, width), dtype=np.float32)
    nxt = np.empty((rows, width), dtype=np.float32) if nw is not None else None
    assert lib().nso_rmsnorm(_p(x2), _p(w), _p(res), _p(sc), _p(nw), rows, width, eps, _p(y), _p(nxt)) == 0
    if nw is None:
        return y.reshape(shape)
    return y.reshape(shape), nxt.reshape(shape)


def ref_dequant(qtype, w, cols, rows, first, count):
    out = np.empty(count, dtype=np.float32)
    rc = ref().nsref_dequant(qtype, _p(w), cols, rows, first, count, _p(out))
    return rc, out


def ref_dot_row(qtype, w, cols, rows, row, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(1, dtype=np.float32)
    rc = ref().nsref_dot_row(qtype, _p(w), cols, rows, row, _p(x), _p(out))
    return rc, out[0]
