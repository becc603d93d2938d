"""CPU tests of the .nsmffn v3 file support (include/ns_ffn.h, csrc/ns_nsmffn.cpp).

The format is the reference's (include/neutron/native/metal_ffn.hpp:13-40,
src/native/metal_ffn.cpp).  The reference's own tests never exercise it, and its
converter only accepts a full 48-layer Gemma 4 12B GGUF, so it is pinned here by:
  * the published FNV-1a 64 test vectors (the fingerprint's hash);
  * an independent numpy parse of the header and entries (metal_ffn.hpp:16-40);
  * the slab reorder, checked against ns_retile (itself pinned against the
    reorder formula of metal_ffn.cpp:145-146 in test_host.py) and by round trip;
  * rejection of every field the reader validates (metal_ffn.cpp:264-287).
"""
import struct

import numpy as np
import pytest

import nsffn as N

HEADER = np.dtype([("magic", "S8"), ("version", "<u4"), ("row_tile", "<u4"), ("entry_count", "<u4"),
                   ("header_bytes", "<u4"), ("model_size", "<u8"), ("model_fingerprint", "<u8"),
                   ("file_size", "<u8"), ("reserved", "<u8", (3,))])
ENTRY = np.dtype([("layer", "<u4"), ("kind", "<u4"), ("type", "<u4"), ("cols", "<u4"), ("rows", "<u4"),
                  ("reserved", "<u4"), ("source_offset", "<u8"), ("offset", "<u8"), ("bytes", "<u8")])
PAGE = 65536
NONE = N.FFN_NONE


def fnv1a64(data, h=0xcbf29ce484222325):
    for b in bytes(data):
        h = ((h ^ b) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return h


def test_fnv1a_published_vectors():
    # test vectors of the FNV reference (Fowler/Noll/Vo), FNV-1a 64-bit
    assert fnv1a64(b"") == 0xcbf29ce484222325
    assert fnv1a64(b"a") == 0xaf63dc4c8601ec8c
    assert fnv1a64(b"foobar") == 0x85944171f73967e8
    assert HEADER.itemsize == 72 and ENTRY.itemsize == 48


def make_gguf(data_offset=PAGE + 4096, seed=5):
    """A GGUF-shaped image: random metadata bytes, then a data section holding two
    layers' FFN tensors plus non-FFN tensors (F32 vector, Q4_K attention matrix),
    32-byte aligned with gaps.  Returns (image, tensor table)."""
    rng = np.random.default_rng(seed)
    D, F = 512, 256
    specs = [  # (type, cols, rows, layer, kind)
        (0, D, 1, NONE, NONE),
        (N.Q4_K, D, 128, NONE, NONE),
    ]
    for layer in range(2):
        specs += [(N.Q4_K, D, F, layer, N.FFN_GATE), (N.Q4_K, D, F, layer, N.FFN_UP),
                  (N.Q6_K if layer == 0 else N.Q4_K, F, D, layer, N.FFN_DOWN)]
    rows, blobs, off = [], [], 0
    for i, (t, cols, r, layer, kind) in enumerate(specs):
        if t == 0:
            blob = rng.standard_normal(cols).astype(np.float32).view(np.uint8)
        else:
            blob = N.synth_weights(t, 100 + i, r, cols)
        off = (off + 31) // 32 * 32 + 32 * i  # aligned, with gaps
        rows.append((off, blob.size, t, cols, r, layer, kind))
        blobs.append((off, blob))
        off += blob.size
    size = data_offset + off + 96
    img = np.zeros(size, dtype=np.uint8)
    img[:data_offset] = rng.integers(0, 256, data_offset, dtype=np.uint8)
    for o, b in blobs:
        img[data_offset + o:data_offset + o + b.size] = b
    return img, N.tensor_table(rows)


def convert(tmp_path, img, data_offset, table, name="m.nsmffn"):
    path = tmp_path / name
    N.nsmffn_convert(path, img, data_offset, table)
    return path, np.fromfile(path, dtype=np.uint8)


# The reference starts its hash at 1469598103934665603 (metal_ffn.cpp:82): one
# digit short of the standard FNV-1a offset basis 14695981039346656037.  Files
# are only interchangeable if this build starts from the same value.
REF_BASIS = 1469598103934665603


def test_fingerprint_definition():
    img, _ = make_gguf()
    do = PAGE + 4096
    want = fnv1a64(struct.pack("<I", 3) + struct.pack("<Q", img.size) + img[:do].tobytes(), REF_BASIS)
    assert N.nsmffn_fingerprint(img[:do], img.size) == want
    # only the first 16 MiB of the metadata area count (metal_ffn.cpp:88)
    big = np.random.default_rng(1).integers(0, 256, (16 << 20) + 64, dtype=np.uint8)
    f0 = N.nsmffn_fingerprint(big, 1 << 30)
    big2 = big.copy()
    big2[-1] ^= 1
    assert N.nsmffn_fingerprint(big2, 1 << 30) == f0
    big2[(16 << 20) - 1] ^= 1
    assert N.nsmffn_fingerprint(big2, 1 << 30) != f0
    assert N.nsmffn_fingerprint(big, (1 << 30) + 1) != f0  # the GGUF size is hashed


def test_convert_layout(tmp_path):
    do = PAGE + 4096
    img, table = make_gguf(do)
    _, out = convert(tmp_path, img, do, table)
    assert out.size == img.size
    h = out[:HEADER.itemsize].view(HEADER)[0]
    assert h["magic"] == b"NSMFFN03" and h["version"] == 3 and h["row_tile"] == 64
    assert h["entry_count"] == len(table) and h["header_bytes"] == PAGE
    assert h["model_size"] == img.size and h["file_size"] == img.size
    assert h["model_fingerprint"] == N.nsmffn_fingerprint(img[:do], img.size)
    assert not h["reserved"].any()
    ents = out[72:72 + 48 * len(table)].view(ENTRY)
    assert not out[72 + 48 * len(table):PAGE].any()  # rest of the header page is zero
    assert not out[PAGE:do].any()                     # the copy converter writes only page + tensors
    for e, t in zip(ents, table):
        assert (e["type"], e["cols"], e["rows"], e["source_offset"], e["bytes"]) == \
               (t["type"], t["cols"], t["rows"], t["source_offset"], t["bytes"])
        assert e["offset"] == do + t["source_offset"] and e["reserved"] == 0
        assert (e["layer"], e["kind"]) == (t["layer"], t["kind"])
        src = img[do + t["source_offset"]:do + t["source_offset"] + t["bytes"]]
        got = out[e["offset"]:e["offset"] + e["bytes"]]
        if t["kind"] == NONE:
            assert np.array_equal(got, src)
        else:
            want = N.retile(src, int(t["type"]), int(t["cols"]), int(t["rows"]), N.ROW_MAJOR, N.NSMFFN)
            assert np.array_equal(got, want)
            back = N.retile(got, int(t["type"]), int(t["cols"]), int(t["rows"]), N.NSMFFN, N.ROW_MAJOR)
            assert np.array_equal(back, src)


def test_reader_accepts_and_looks_up(tmp_path):
    do = PAGE + 4096
    img, table = make_gguf(do)
    path, _ = convert(tmp_path, img, do, table)
    fp = N.nsmffn_fingerprint(img[:do], img.size)
    f = N.NsmffnFile(path, img.size, fp, table)
    assert f.size() == img.size
    for t in table:
        off, re = f.lookup(int(t["source_offset"]))
        assert off == do + t["source_offset"] and re == (t["kind"] != NONE)
        if t["kind"] == NONE:
            assert np.array_equal(f.view(off, int(t["bytes"])), img[off:off + int(t["bytes"])])
    with pytest.raises(N.NsError, match="missing"):
        f.lookup(123456789)
    f.close()


def _expect_reject(path, size, fp, table, match):
    with pytest.raises(N.NsError, match=match) as e:
        N.NsmffnFile(path, size, fp, table)
    return e.value.code


HEADER_FIELDS = [  # (byte offset, new value packer) of each validated header field
    (0, b"NSMFFN02"), (8, struct.pack("<I", 2)), (12, struct.pack("<I", 32)), (16, struct.pack("<I", 6)),
    (20, struct.pack("<I", 4096)), (24, struct.pack("<Q", 1)), (32, struct.pack("<Q", 7)), (40, struct.pack("<Q", 9)),
]


@pytest.mark.parametrize("field", range(len(HEADER_FIELDS)))
def test_reader_rejects_header_mismatch(tmp_path, field):
    do = PAGE + 4096
    img, table = make_gguf(do)
    path, out = convert(tmp_path, img, do, table)
    fp = N.nsmffn_fingerprint(img[:do], img.size)
    pos, val = HEADER_FIELDS[field]
    out[pos:pos + len(val)] = np.frombuffer(val, dtype=np.uint8)
    out.tofile(path)
    assert _expect_reject(path, img.size, fp, table, "does not match this GGUF") == 6


ENTRY_FIELDS = ["layer", "kind", "type", "cols", "rows", "source_offset", "bytes", "offset"]


@pytest.mark.parametrize("field", ENTRY_FIELDS)
def test_reader_rejects_entry_mismatch(tmp_path, field):
    do = PAGE + 4096
    img, table = make_gguf(do)
    path, out = convert(tmp_path, img, do, table)
    fp = N.nsmffn_fingerprint(img[:do], img.size)
    ents = out[72:72 + 48 * len(table)].view(ENTRY)
    i = 3  # a gate tensor of layer 0... every field, including the offset running past the file
    ents[i][field] = img.size if field == "offset" else ents[i][field] + 1
    out.tofile(path)
    _expect_reject(path, img.size, fp, table, f"invalid Metal FFN tensor entry {i}")


def test_reader_rejects_wrong_gguf_truncation_and_duplicates(tmp_path):
    do = PAGE + 4096
    img, table = make_gguf(do)
    path, out = convert(tmp_path, img, do, table)
    fp = N.nsmffn_fingerprint(img[:do], img.size)
    _expect_reject(path, img.size + 1, fp, table, "does not match")          # another GGUF size
    _expect_reject(path, img.size, fp ^ 1, table, "does not match")          # another GGUF
    _expect_reject(path, img.size, fp, table[:-1], "does not match")         # entry count
    np.concatenate([out, np.zeros(8, np.uint8)]).tofile(tmp_path / "long")
    _expect_reject(tmp_path / "long", img.size, fp, table, "does not match")  # file size
    out[:1000].tofile(tmp_path / "short")
    _expect_reject(tmp_path / "short", img.size, fp, table, "invalid Metal FFN file")
    _expect_reject(tmp_path / "absent", img.size, fp, table, "cannot open")
    # two tensors claiming the same GGUF offset
    dup = table.copy()
    dup[1] = dup[0]
    p2, _ = convert(tmp_path, img, do, dup, name="dup.nsmffn")
    _expect_reject(p2, img.size, fp, dup, "duplicate")


def test_converter_rejects_bad_ffn_tensors(tmp_path):
    do = PAGE + 4096
    img, table = make_gguf(do)
    bad = table.copy()
    bad[2]["rows"] = 100  # not a whole number of 64-row slabs
    with pytest.raises(N.NsError, match="unsupported shape"):
        N.nsmffn_convert(tmp_path / "x", img, do, bad)
    bad = table.copy()
    bad[2]["type"] = 1  # F16 FFN tensor
    with pytest.raises(N.NsError, match="unsupported type"):
        N.nsmffn_convert(tmp_path / "x", img, do, bad)
    assert not (tmp_path / "x").exists() and not (tmp_path / "x.tmp").exists()


def test_convert_in_place(tmp_path):
    do = PAGE + 4096
    img, table = make_gguf(do)
    _, copy = convert(tmp_path, img, do, table)
    model = tmp_path / "model.gguf"
    img.tofile(model)
    meta = tmp_path / "meta.gguf"
    N.nsmffn_convert_in_place(model, meta, do, table)
    got = np.fromfile(model, dtype=np.uint8)
    assert np.array_equal(got[:PAGE], copy[:PAGE])          # same header page as the copy converter
    assert np.array_equal(got[PAGE:do], img[PAGE:do])       # rest of the metadata area untouched
    for t in table:
        a = do + int(t["source_offset"])
        assert np.array_equal(got[a:a + int(t["bytes"])], copy[a:a + int(t["bytes"])])
    m = np.fromfile(meta, dtype=np.uint8)
    assert m.size == img.size and np.array_equal(m[:do], img[:do]) and not m[do:].any()
    fp = N.nsmffn_fingerprint(img[:do], img.size)
    N.NsmffnFile(model, img.size, fp, table).close()
    with pytest.raises(N.NsError, match="too small"):
        N.nsmffn_convert_in_place(model, meta, PAGE - 32, table)
