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
REF_GGUF_PATH = os.path.join(HERE, "_ref", "libns_ref_gguf.so")

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
        L.nso_f16_tile_row.argtypes = [i32, i32, vp, u64, u64, u64, vp, vp]
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


def f16_tile_rows(qtype, layout, w, cols, rows, row0=0, nrows=None):
    """FP16-mode tiles of rows [row0, row0+nrows): (tiles [nrows][cols], inv_c [nrows])."""
    nrows = rows - row0 if nrows is None else nrows
    out = np.empty((nrows, cols), dtype=np.float32)
    inv = np.empty(nrows, dtype=np.float32)
    for i in range(nrows):
        rc = lib().nso_f16_tile_row(qtype, layout, _p(w), cols, rows, row0 + i, _p(out[i]), _p(inv[i:i + 1]))
        assert rc == 0
    return out, inv


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


# ---- the reference's own GGUF reader (oracle/_ref/libns_ref_gguf.so) -------------

_ref_gguf = None


def ref_gguf_available():
    return os.path.exists(REF_GGUF_PATH)


def ref_gguf():
    global _ref_gguf
    if _ref_gguf is None:
        R = ctypes.CDLL(REF_GGUF_PATH)
        vp, u32, u64, cp = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_char_p
        R.nsref_gguf_open.restype = vp
        R.nsref_gguf_open.argtypes = [cp, vp, u64]
        R.nsref_gguf_close.argtypes = [vp]
        for n in ("nsref_gguf_data_offset", "nsref_gguf_file_size"):
            getattr(R, n).restype = u64
            getattr(R, n).argtypes = [vp]
        R.nsref_gguf_tensor_count.restype = u32
        R.nsref_gguf_tensor_count.argtypes = [vp]
        R.nsref_gguf_tensor.argtypes = [vp, u32, vp, u64, vp, vp, vp, vp, vp]
        R.nsref_gguf_find.argtypes = [vp, cp, vp, u64]
        R.nsref_gguf_meta_u64.argtypes = [vp, cp, vp, vp, u64]
        R.nsref_gguf_meta_number.argtypes = [vp, cp, vp, vp, u64]
        R.nsref_gguf_meta_string.argtypes = [vp, cp, vp, u64]
        R.nsref_gguf_meta_array.argtypes = [vp, cp, ctypes.c_int, vp, u64, vp]
        _ref_gguf = R
    return _ref_gguf


class RefGguf:
    """The reference's GGUF class on a file: .error is its exception message when the
    constructor threw, else the parsed fields are available."""

    def __init__(self, path):
        err = ctypes.create_string_buffer(512)
        self.h = ref_gguf().nsref_gguf_open(str(path).encode(), err, 512)
        self.error = None if self.h else err.value.decode()

    def close(self):
        if self.h:
            ref_gguf().nsref_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def data_offset(self):
        return ref_gguf().nsref_gguf_data_offset(self.h)

    def file_size(self):
        return ref_gguf().nsref_gguf_file_size(self.h)

    def tensors(self):
        out = []
        for i in range(ref_gguf().nsref_gguf_tensor_count(self.h)):
            name = ctypes.create_string_buffer(1024)
            t, nd, off, nb = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
            shape = (ctypes.c_uint64 * 4)()
            ref_gguf().nsref_gguf_tensor(self.h, i, name, 1024, ctypes.byref(t), ctypes.byref(nd), shape,
                                         ctypes.byref(off), ctypes.byref(nb))
            out.append((name.value.decode(), t.value, tuple(shape[:nd.value]), off.value, nb.value))
        return out

    def find(self, name):
        err = ctypes.create_string_buffer(512)
        rc = ref_gguf().nsref_gguf_find(self.h, name.encode(), err, 512)
        return None if rc == 0 else err.value.decode()

    def meta_u64(self, key):
        v, err = ctypes.c_uint64(), ctypes.create_string_buffer(512)
        rc = ref_gguf().nsref_gguf_meta_u64(self.h, key.encode(), ctypes.byref(v), err, 512)
        return (v.value, None) if rc == 0 else (None, err.value.decode())

    def meta_number(self, key):
        v, err = ctypes.c_double(), ctypes.create_string_buffer(512)
        rc = ref_gguf().nsref_gguf_meta_number(self.h, key.encode(), ctypes.byref(v), err, 512)
        return (v.value, None) if rc == 0 else (None, err.value.decode())

    def meta_string(self, key):
        out = ctypes.create_string_buffer(1 << 16)
        rc = ref_gguf().nsref_gguf_meta_string(self.h, key.encode(), out, 1 << 16)
        return (out.value.decode(), None) if rc == 0 else (None, out.value.decode())

    def meta_array(self, key, elem, dtype):
        cap = 1 << 20
        buf = ctypes.create_string_buffer(cap)
        n = ctypes.c_uint64()
        rc = ref_gguf().nsref_gguf_meta_array(self.h, key.encode(), elem, buf, cap, ctypes.byref(n))
        if rc:
            return None
        return np.frombuffer(buf.raw[:n.value * np.dtype(dtype).itemsize], dtype=dtype)
