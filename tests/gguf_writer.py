"""A GGUF v3 writer for the tests (the published GGUF v3 layout, little endian):
magic "GGUF", u32 version, u64 tensor count, u64 metadata count; metadata entries
(string key, u32 value type, value; arrays: u32 element type, u64 length, elements);
tensor entries (string name, u32 rank, u64 dims, u32 type, u64 offset in the data
section); the data section at the next multiple of the alignment.  Strings are a u64
length and that many bytes.  Knobs let tests write malformed files."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64: "<d"}
TYPE_BYTES = {0: (4, 1), 1: (2, 1), 12: (144, 256), 14: (210, 256)}  # type: (bytes per block, values per block)


def _s(x):
    b = x.encode() if isinstance(x, str) else x
    return struct.pack("<Q", len(b)) + b


def _value(vtype, value):
    if vtype == STRING:
        return _s(value)
    if vtype == ARRAY:
        et, items = value
        out = struct.pack("<IQ", et, len(items))
        if et == STRING:
            return out + b"".join(_s(i) for i in items)
        return out + b"".join(struct.pack(_SCALAR[et], i) for i in items)
    return struct.pack(_SCALAR[vtype], value)


def tensor_nbytes(ttype, shape):
    bb, per = TYPE_BYTES[ttype]
    return int(np.prod(shape)) // per * bb


def build(meta, tensors, alignment=32, version=3, magic=b"GGUF", counts=None):
    """meta: [(key, type, value)]; tensors: [(name, shape, type, bytes or None)] with data
    placed in order at aligned offsets (random bytes when None).  Returns (file bytes,
    data_offset, [offsets])."""
    head = magic + struct.pack("<I", version)
    nt, nm = counts if counts else (len(tensors), len(meta))
    head += struct.pack("<QQ", nt, nm)
    for k, t, v in meta:
        head += _s(k) + struct.pack("<I", t) + _value(t, v)
    offsets, pos, datas = [], 0, []
    rng = np.random.default_rng(7)
    for name, shape, ttype, data in tensors:
        nb = tensor_nbytes(ttype, shape) if ttype in TYPE_BYTES else 64
        if data is None:
            data = rng.integers(0, 256, nb, dtype=np.uint8).tobytes()
        offsets.append(pos)
        datas.append((pos, data))
        pos = (pos + len(data) + alignment - 1) // alignment * alignment
    for (name, shape, ttype, _), off in zip(tensors, offsets):
        head += _s(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        head += struct.pack("<IQ", ttype, off)
    data_offset = (len(head) + alignment - 1) // alignment * alignment
    buf = bytearray(head + b"\0" * (data_offset - len(head)) + b"\0" * pos)
    for off, data in datas:
        buf[data_offset + off:data_offset + off + len(data)] = data
    return bytes(buf), data_offset, offsets


def write(path, meta, tensors, **kw):
    data, data_offset, offsets = build(meta, tensors, **kw)
    with open(path, "wb") as f:
        f.write(data)
    return data, data_offset, offsets
