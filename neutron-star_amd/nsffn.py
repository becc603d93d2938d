"""ctypes binding of libnsffn.so (include/ns_ffn.h) for tests, smoke and bench.

Device buffers are torch tensors (PyTorch is only used for device memory and
streams); host utilities take numpy arrays.  Loading fails loudly when the
library has not been built: there is no fallback path.
"""
import ctypes
import os
import re

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "libnsffn.so")
HEADER = os.path.join(ROOT, "include", "ns_ffn.h")

Q4_K, Q6_K = 12, 14
ROW_MAJOR, NSMFFN, CDNA4 = 0, 1, 2
FFN_GATE, FFN_UP, FFN_DOWN, FFN_NONE = 0, 1, 2, 0xFFFFFFFF
ACC_FP32, ACC_FP16 = 0, 1
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210}

_lib = None


class NsError(RuntimeError):
    """A non-zero status from the C ABI, with ns_last_error()'s message."""

    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def header_functions():
    """Names of the functions declared in include/ns_ffn.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ns_[a-z0-9_]+)\s*\(", text)))


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        vp, u32, u64, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int
        L.ns_last_error.restype = ctypes.c_char_p
        L.ns_layer_seed.restype = u64
        L.ns_layer_seed.argtypes = [u64, u32]
        L.ns_nsmffn_fingerprint.restype = u64
        L.ns_nsmffn_fingerprint.argtypes = [vp, u64, u64]
        L.ns_nsmffn_data.restype = vp
        L.ns_nsmffn_data.argtypes = [vp]
        L.ns_nsmffn_size.restype = u64
        L.ns_nsmffn_size.argtypes = [vp]
        for name, rt in (("ns_gguf_data_offset", u64), ("ns_gguf_file_size", u64), ("ns_gguf_mapped_data", vp),
                         ("ns_gguf_tensor_count", u32)):
            getattr(L, name).restype = rt
            getattr(L, name).argtypes = [vp]
        sigs = {
            "ns_abi_version": [],
            "ns_ctx_create": [i32, ctypes.POINTER(vp)],
            "ns_ctx_destroy": [vp],
            "ns_ctx_workspace_bytes": [vp, ctypes.POINTER(u64)],
            "ns_ctx_set_tuning": [vp, ctypes.c_char_p, i32],
            "ns_ctx_status": [vp, vp],
            "ns_ctx_set_wait_free": [vp, i32],
            "ns_matmul": [vp, vp, i32, i32, u32, u32, u32, vp, i32, vp, vp],
            "ns_matmul_noalloc": [vp, i32, i32, u32, u32, u32, vp, i32, vp, vp],
            "ns_noalloc_status": [vp],
            "ns_gate_up_geglu_decode": [vp, vp, vp, i32, u32, u32, vp, vp, vp],
            "ns_gate_up_geglu_rm32": [vp, vp, vp, i32, u32, u32, u32, vp, vp, i32, vp],
            "ns_gate_up_geglu": [vp, vp, vp, i32, u32, u32, u32, vp, vp, vp],
            "ns_ffn_down": [vp, vp, i32, i32, u32, u32, u32, vp, i32, i32, vp, vp],
            "ns_dequant": [vp, vp, i32, i32, u32, u32, u32, u32, vp, vp, vp],
            "ns_rmsnorm": [vp, vp, vp, u32, u32, ctypes.c_float, vp, i32, vp],
            "ns_rmsnorm_add": [vp, vp, vp, vp, vp, u32, u32, ctypes.c_float, vp, vp],
            "ns_rmsnorm_add_then": [vp, vp, vp, vp, vp, vp, u32, u32, ctypes.c_float, vp, vp, i32, vp],
            "ns_rms_gate_up_geglu_decode": [vp, vp, vp, i32, u32, u32, vp, vp, ctypes.c_float, vp, vp],
            "ns_geglu": [vp, vp, vp, u64, vp, i32, vp],
            "ns_ffn_block_decode": [vp, vp, vp, vp, i32, i32, u32, u32, vp, vp, ctypes.c_float, vp, vp, vp],
            "ns_ffn_stack_decode": [vp, u32, vp, vp, vp, vp, i32, u32, u32, vp, vp, ctypes.c_float, vp, vp, vp],
            "ns_retile": [vp, vp, i32, u32, u32, i32, i32],
            "ns_retile_device": [vp, vp, i32, u32, u32, i32, i32, vp],
            "ns_synth_blocks": [i32, u64, u64, u64, vp, i32],
            "ns_synth_normal_f32": [u64, u64, u64, vp, i32],
            "ns_synth_normal_f16": [u64, u64, u64, vp, i32],
            "ns_nsmffn_convert": [ctypes.c_char_p, vp, u64, u64, vp, u32],
            "ns_nsmffn_convert_in_place": [ctypes.c_char_p, ctypes.c_char_p, u64, vp, u32],
            "ns_nsmffn_open": [ctypes.c_char_p, u64, u64, vp, u32, ctypes.POINTER(vp)],
            "ns_nsmffn_close": [vp],
            "ns_nsmffn_lookup": [vp, u64, ctypes.POINTER(u64), ctypes.POINTER(i32)],
            "ns_embedding": [vp, vp, i32, i32, u32, u32, vp, u32, ctypes.c_float, vp, vp],
            "ns_qkv": [vp, vp, vp, vp, i32, i32, u32, u32, u32, u32, vp, vp, vp, vp, vp],
            "ns_gguf_open": [ctypes.c_char_p, i32, ctypes.POINTER(vp)],
            "ns_gguf_close": [vp],
            "ns_gguf_tensor": [vp, u32, ctypes.POINTER(GgufTensorInfo)],
            "ns_gguf_find_tensor": [vp, ctypes.c_char_p, ctypes.POINTER(u32)],
            "ns_gguf_has_meta": [vp, ctypes.c_char_p],
            "ns_gguf_meta_u64": [vp, ctypes.c_char_p, ctypes.POINTER(u64)],
            "ns_gguf_meta_number": [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)],
            "ns_gguf_meta_string": [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)],
            "ns_gguf_meta_array": [vp, ctypes.c_char_p, ctypes.POINTER(u32), ctypes.POINTER(u64),
                                   ctypes.POINTER(vp)],
            "ns_gguf_ffn_table": [vp, vp, u32, ctypes.POINTER(u32)],
        }
        for name, args in sigs.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = ctypes.c_int
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise NsError(rc, lib().ns_last_error().decode())
    return rc


def _ptr(a):
    """Device pointer of a torch CUDA tensor (None passes through).  Host arrays are
    refused: a host pointer handed to a kernel faults the GPU."""
    if a is None:
        return None
    if isinstance(a, np.ndarray) or not getattr(a, "is_cuda", False):
        raise TypeError("device entry points take torch CUDA tensors, got " + type(a).__name__)
    return a.data_ptr()


def _hptr(a):
    """Host pointer of a numpy array for the host-side utilities."""
    if not isinstance(a, np.ndarray):
        raise TypeError("host utilities take numpy arrays, got " + type(a).__name__)
    return a.ctypes.data


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return stream


def default_threads():
    return max(1, min(16, os.cpu_count() or 1))


# ---- host utilities --------------------------------------------------------

def synth_blocks(qtype, seed, nblocks, first=0, nthreads=None):
    out = np.empty(nblocks * BLOCK_BYTES[qtype], dtype=np.uint8)
    check(lib().ns_synth_blocks(qtype, seed, first, nblocks, _hptr(out), nthreads or default_threads()))
    return out


def synth_weights(qtype, seed, rows, cols, nthreads=None):
    """ROW_MAJOR bytes of a seeded [rows][cols] tensor (block i = row*nb + kb)."""
    return synth_blocks(qtype, seed, rows * (cols // 256), nthreads=nthreads)


def synth_normal_f32(seed, n, first=0, nthreads=None):
    out = np.empty(n, dtype=np.float32)
    check(lib().ns_synth_normal_f32(seed, first, n, _hptr(out), nthreads or default_threads()))
    return out


def synth_normal_f16(seed, n, first=0, nthreads=None):
    out = np.empty(n, dtype=np.uint16)
    check(lib().ns_synth_normal_f16(seed, first, n, _hptr(out), nthreads or default_threads()))
    return out


def layer_seed(seed, layer):
    return lib().ns_layer_seed(seed, layer)


def retile(src, qtype, cols, rows, from_layout, to_layout):
    src = np.ascontiguousarray(src, dtype=np.uint8)
    dst = np.empty_like(src)
    check(lib().ns_retile(_hptr(src), _hptr(dst), qtype, cols, rows, from_layout, to_layout))
    return dst


# ---- .nsmffn v3 files ---------------------------------------------------------

TENSOR_DESC = np.dtype([("source_offset", "<u8"), ("bytes", "<u8"), ("type", "<u4"), ("cols", "<u4"),
                        ("rows", "<u4"), ("layer", "<u4"), ("kind", "<u4"), ("reserved", "<u4")])
assert TENSOR_DESC.itemsize == 40


def tensor_table(rows):
    """ns_tensor_desc array from (source_offset, bytes, type, cols, rows, layer, kind) tuples."""
    return np.array([tuple(r) + (0,) for r in rows], dtype=TENSOR_DESC)


def nsmffn_fingerprint(head, gguf_size):
    head = np.ascontiguousarray(head, dtype=np.uint8)
    return lib().ns_nsmffn_fingerprint(_hptr(head), head.size, gguf_size)


def nsmffn_convert(path, gguf, data_offset, table):
    gguf = np.ascontiguousarray(gguf, dtype=np.uint8)
    check(lib().ns_nsmffn_convert(str(path).encode(), _hptr(gguf), gguf.size, data_offset, _hptr(table), len(table)))


def nsmffn_convert_in_place(model_path, metadata_path, data_offset, table):
    check(lib().ns_nsmffn_convert_in_place(str(model_path).encode(), str(metadata_path).encode(), data_offset,
                                           _hptr(table), len(table)))


class NsmffnFile:
    """MetalFfnFile (src/native/metal_ffn.cpp:253-311): a validated read-only mapping."""

    handle = None

    def __init__(self, path, gguf_size, fingerprint, table):
        h = ctypes.c_void_p()
        check(lib().ns_nsmffn_open(str(path).encode(), gguf_size, fingerprint, _hptr(table), len(table),
                                   ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            lib().ns_nsmffn_close(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def size(self):
        return lib().ns_nsmffn_size(self.handle)

    def lookup(self, source_offset):
        off, re = ctypes.c_uint64(), ctypes.c_int()
        check(lib().ns_nsmffn_lookup(self.handle, source_offset, ctypes.byref(off), ctypes.byref(re)))
        return off.value, bool(re.value)

    def view(self, offset, nbytes):
        """Bytes [offset, offset + nbytes) of the mapping (a copy)."""
        base = lib().ns_nsmffn_data(self.handle)
        return np.frombuffer((ctypes.c_uint8 * nbytes).from_address(base + offset), dtype=np.uint8).copy()


# ---- GGUF v3 reader -----------------------------------------------------------

class GgufTensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_uint32), ("n_dims", ctypes.c_uint32),
                ("shape", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64)]


# numpy element type of each GGUF array value type
GGUF_ARRAY_DTYPES = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32,
                     6: np.float32, 7: np.uint8, 10: np.uint64, 11: np.int64, 12: np.float64}


class GgufFile:
    """GGUF (src/native/gguf.cpp:71-129): a validated read-only mapping of a GGUF v3 file."""

    handle = None

    def __init__(self, path, prefetch=False):
        h = ctypes.c_void_p()
        check(lib().ns_gguf_open(str(path).encode(), int(prefetch), ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            lib().ns_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def data_offset(self):
        return lib().ns_gguf_data_offset(self.handle)

    def file_size(self):
        return lib().ns_gguf_file_size(self.handle)

    def tensors(self):
        """[(name, type, shape, offset, bytes)] in GGUF order."""
        out = []
        for i in range(lib().ns_gguf_tensor_count(self.handle)):
            t = GgufTensorInfo()
            check(lib().ns_gguf_tensor(self.handle, i, ctypes.byref(t)))
            out.append((t.name.decode(), t.type, tuple(t.shape[:t.n_dims]), t.offset, t.bytes))
        return out

    def find(self, name):
        idx = ctypes.c_uint32()
        check(lib().ns_gguf_find_tensor(self.handle, name.encode(), ctypes.byref(idx)))
        return idx.value

    def has(self, key):
        return bool(lib().ns_gguf_has_meta(self.handle, key.encode()))

    def meta_u64(self, key):
        v = ctypes.c_uint64()
        check(lib().ns_gguf_meta_u64(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def meta_number(self, key):
        v = ctypes.c_double()
        check(lib().ns_gguf_meta_number(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def meta_string(self, key):
        v = ctypes.c_char_p()
        check(lib().ns_gguf_meta_string(self.handle, key.encode(), ctypes.byref(v)))
        return v.value.decode()

    def meta_array(self, key):
        """(element type, numpy array or None for string arrays, count)."""
        et, n, p = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_void_p()
        check(lib().ns_gguf_meta_array(self.handle, key.encode(), ctypes.byref(et), ctypes.byref(n),
                                       ctypes.byref(p)))
        if et.value == 8:
            return et.value, None, n.value
        dt = np.dtype(GGUF_ARRAY_DTYPES[et.value])
        raw = (ctypes.c_uint8 * (n.value * dt.itemsize)).from_address(p.value) if n.value else b""
        return et.value, np.frombuffer(bytes(raw), dtype=dt), n.value

    def ffn_table(self):
        """The ns_tensor_desc table for the .nsmffn functions (ffn_tensors, metal_ffn.cpp:63-71)."""
        n = ctypes.c_uint32()
        check(lib().ns_gguf_ffn_table(self.handle, None, 0, ctypes.byref(n)))
        table = np.zeros(n.value, dtype=TENSOR_DESC)
        check(lib().ns_gguf_ffn_table(self.handle, _hptr(table), n.value, ctypes.byref(n)))
        return table

    def bytes_at(self, offset, nbytes):
        base = lib().ns_gguf_mapped_data(self.handle)
        return np.frombuffer((ctypes.c_uint8 * nbytes).from_address(base + offset), dtype=np.uint8).copy()


# ---- device entry points (torch tensors) ------------------------------------

class Context:
    def __init__(self, device=0):
        h = ctypes.c_void_p()
        check(lib().ns_ctx_create(device, ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            lib().ns_ctx_destroy(self.handle)
            self.handle = None

    def set_tuning(self, key, value):
        """Test hook: override one kernel-selection choice of this context
        (ns_ctx_set_tuning; keys gemv_pf, gemv_waves, gemv_whole, gemv_qslab,
        gemm_kparts, gemm_q4_reg, mt_mfma, mt_parts, mt_slabs, mt_spw, block_fused, block_spin, gemm_rs)."""
        check(lib().ns_ctx_set_tuning(self.handle, key.encode(), int(value)))

    def workspace_bytes(self):
        n = ctypes.c_uint64()
        check(lib().ns_ctx_workspace_bytes(self.handle, ctypes.byref(n)))
        return n.value

    def status(self, stream=None):
        """ns_ctx_status (finish_command, mm:231-243): waits for the stream, raises NsError
        (NS_ERR_TIMEOUT) when a bounded cross-workgroup wait of this context ran out."""
        check(lib().ns_ctx_status(self.handle, _stream(stream)))

    def set_wait_free(self, on=True):
        """ns_ctx_set_wait_free: launches in which no workgroup waits for another."""
        check(lib().ns_ctx_set_wait_free(self.handle, int(bool(on))))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def matmul(self, w, qtype, layout, cols, rows, batch, inp, out, half_input=False, stream=None):
        check(lib().ns_matmul(self.handle, _ptr(w), qtype, layout, cols, rows, batch, _ptr(inp),
                              int(half_input), _ptr(out), _stream(stream)))

    def gate_up_geglu_decode(self, wg, wu, layout, cols, rows, x, h, stream=None):
        check(lib().ns_gate_up_geglu_decode(self.handle, _ptr(wg), _ptr(wu), layout, cols, rows,
                                            _ptr(x), _ptr(h), _stream(stream)))

    def gate_up_geglu(self, wg, wu, layout, cols, rows, batch, x, h, stream=None):
        """gate_up_geglu (mm:281): fp16 x and h; batch <= 4 streams the weights once."""
        check(lib().ns_gate_up_geglu(self.handle, _ptr(wg), _ptr(wu), layout, cols, rows, batch,
                                     _ptr(x), _ptr(h), _stream(stream)))

    def gate_up_geglu_rm32(self, wg, wu, layout, cols, rows, batch, x, h, fast_swa, stream=None):
        check(lib().ns_gate_up_geglu_rm32(self.handle, _ptr(wg), _ptr(wu), layout, cols, rows, batch,
                                          _ptr(x), _ptr(h), int(fast_swa), _stream(stream)))

    def ffn_down(self, w, qtype, layout, cols, rows, batch, inp, out, half_input, fast_swa, stream=None):
        check(lib().ns_ffn_down(self.handle, _ptr(w), qtype, layout, cols, rows, batch, _ptr(inp),
                                int(half_input), int(fast_swa), _ptr(out), _stream(stream)))

    def ffn_block(self, gate, up, down, down_type, layout, cols, ffn, batch, inp, mid, out, prefill, swa,
                  exact_ffn=False, stream=None):
        """The FFN part of the engine's per-layer loop (metal_engine.mm:564-573): gate/up +
        GeGLU into `mid`, then down into `out`, in the mode fast_swa_ffn = prefill && swa &&
        !exact_ffn (mm:565).  Prefill: inp/mid fp16 bits; decode: fp32."""
        fast = bool(prefill and swa and not exact_ffn)
        if prefill and batch > 4:
            self.gate_up_geglu_rm32(gate, up, layout, cols, ffn, batch, inp, mid, fast, stream)
        elif prefill:  # mm:569: 2-4 tokens take gate_up_geglu (small-batch kernel, FP32)
            self.gate_up_geglu(gate, up, layout, cols, ffn, batch, inp, mid, stream)
        elif batch == 1:  # mm:571-573 in one launch (or the same two launches)
            self.ffn_block_decode(gate, up, down, down_type, layout, cols, ffn, inp, mid, out, stream=stream)
            return
        else:  # mm:570: matmul(gate), matmul(up) (small-batch kernels), then gemma_geglu
            import torch
            g = torch.empty(batch * ffn, dtype=torch.float32, device=mid.device)
            u = torch.empty(batch * ffn, dtype=torch.float32, device=mid.device)
            self.matmul(gate, Q4_K, layout, cols, ffn, batch, inp, g, stream=stream)
            self.matmul(up, Q4_K, layout, cols, ffn, batch, inp, u, stream=stream)
            self.geglu(g, u, batch * ffn, mid, stream=stream)
        self.ffn_down(down, down_type, layout, ffn, cols, batch, mid, out, prefill, fast, stream)

    def geglu(self, gate, up, count, out, half_out=False, stream=None):
        """gemma_geglu[_f16] (metal:530-531): out = gelu_tanh(gate) * up, elementwise."""
        check(lib().ns_geglu(self.handle, _ptr(gate), _ptr(up), count, _ptr(out), int(half_out), _stream(stream)))

    def rmsnorm(self, x, weight, rows, width, eps, y, half_out=False, stream=None):
        """rms / rms_half (mm:291-292): y = (x * r) * weight per row."""
        check(lib().ns_rmsnorm(self.handle, _ptr(x), _ptr(weight), rows, width, eps, _ptr(y), int(half_out),
                               _stream(stream)))

    def rmsnorm_add(self, x, weight, residual, scale, rows, width, eps, y, stream=None):
        """rms_add (mm:295): y = residual + (x * r) * weight [* scale]."""
        check(lib().ns_rmsnorm_add(self.handle, _ptr(x), _ptr(weight), _ptr(residual), _ptr(scale), rows, width,
                                   eps, _ptr(y), _stream(stream)))

    def rmsnorm_add_then(self, x, weight, residual, scale, next_weight, rows, width, eps, y, nxt, half_next,
                         stream=None):
        """rms_add_then_half (mm:296) or, with half_next False, rms_add followed by rms."""
        check(lib().ns_rmsnorm_add_then(self.handle, _ptr(x), _ptr(weight), _ptr(residual), _ptr(scale),
                                        _ptr(next_weight), rows, width, eps, _ptr(y), _ptr(nxt), int(half_next),
                                        _stream(stream)))

    def rms_gate_up_geglu_decode(self, wg, wu, layout, cols, rows, x, norm_weight, eps, h, stream=None):
        """rms (mm:563) then gate_up_geglu_decode (mm:571), one launch."""
        check(lib().ns_rms_gate_up_geglu_decode(self.handle, _ptr(wg), _ptr(wu), layout, cols, rows, _ptr(x),
                                                _ptr(norm_weight), eps, _ptr(h), _stream(stream)))

    def ffn_block_decode(self, wg, wu, wd, down_type, layout, cols, ffn, x, h, y, norm_weight=None, eps=1e-6,
                         stream=None):
        """The decode FFN block (mm:571-573) in one launch where the shapes allow it:
        h = GeGLU(Wg.n, Wu.n), y = Wd.h, n = x or its RMSNorm with norm_weight."""
        check(lib().ns_ffn_block_decode(self.handle, _ptr(wg), _ptr(wu), _ptr(wd), down_type, layout, cols, ffn,
                                        _ptr(x), None if norm_weight is None else _ptr(norm_weight), eps, _ptr(h),
                                        _ptr(y), _stream(stream)))

    def ffn_stack_decode(self, wg, wu, wd, down_types, layout, cols, ffn, x, h, y, norm_weights=None, eps=1e-6,
                         stream=None):
        """The decode FFN blocks of len(wg) consecutive layers (mm:563-573 repeated) in one
        launch: x_{l+1} = Wd[l].(gelu(Wg[l].n_l) * (Wu[l].n_l)), n_l = x_l or its RMSNorm with
        norm_weights[l]; y = the last layer's output, h its h."""
        n = len(wg)
        assert len(wu) == n and len(wd) == n and len(down_types) == n
        P = ctypes.c_void_p * n
        tw, tu, td = P(*[_ptr(t) for t in wg]), P(*[_ptr(t) for t in wu]), P(*[_ptr(t) for t in wd])
        types = (ctypes.c_int * n)(*[int(t) for t in down_types])
        nws = None if norm_weights is None else P(*[_ptr(t) for t in norm_weights])
        check(lib().ns_ffn_stack_decode(self.handle, n, tw, tu, td, types, layout, cols, ffn, _ptr(x), nws, eps,
                                        _ptr(h), _ptr(y), _stream(stream)))

    def embedding(self, w, qtype, layout, cols, rows, ids, batch, scale, out, stream=None):
        """gemma_q6k_embedding (metal:503): out[t] = scale * W[ids[t]]."""
        check(lib().ns_embedding(self.handle, _ptr(w), qtype, layout, cols, rows, _ptr(ids), batch, scale, _ptr(out),
                                 _stream(stream)))

    def qkv(self, wq, wk, wv, v_type, layout, cols, q_rows, kv_rows, batch, x, q, k, v, stream=None):
        """qkv (mm:311): Q, K, V projections of fp16 x; wv None for tied V."""
        check(lib().ns_qkv(self.handle, _ptr(wq), _ptr(wk), _ptr(wv), v_type, layout, cols, q_rows, kv_rows, batch,
                           _ptr(x), _ptr(q), _ptr(k), _ptr(v), _stream(stream)))

    def dequant(self, w, qtype, layout, cols, rows, row0, nrows, out_f32=None, out_f16=None, stream=None):
        check(lib().ns_dequant(self.handle, _ptr(w), qtype, layout, cols, rows, row0, nrows,
                               _ptr(out_f32), _ptr(out_f16), _stream(stream)))


def matmul_noalloc(w, qtype, layout, cols, rows, batch, inp, out, half_input=False, stream=None):
    """ns_matmul_noalloc: ns_matmul on the library's static device scratch (no context)."""
    check(lib().ns_matmul_noalloc(_ptr(w), qtype, layout, cols, rows, batch, _ptr(inp), int(half_input), _ptr(out),
                                  _stream(stream)))


def noalloc_status(stream=None):
    """ns_noalloc_status: waits for the stream, raises NsError on a timed-out wait recorded
    in the static scratch."""
    check(lib().ns_noalloc_status(_stream(stream)))


def retile_device(src, dst, qtype, cols, rows, from_layout, to_layout, stream=None):
    check(lib().ns_retile_device(_ptr(src), _ptr(dst), qtype, cols, rows, from_layout, to_layout,
                                 _stream(stream)))
