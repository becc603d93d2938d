"""The GGUF v3 reader (ns_gguf_*, the engine's GGUF class, src/native/gguf.cpp:71-129) and the
FFN tensor table it feeds to the .nsmffn converter (ffn_tensors, metal_ffn.cpp:63-71): CPU tests.

Files are written by tests/gguf_writer.py.  Where oracle/_ref holds the reference's own
reader (built from src/native/gguf.cpp by oracle/Makefile), every parse result and every
error message is compared with it; without it the checks against the written values stay.
"""
import struct

import numpy as np
import pytest

import gguf_writer as W
import ns_oracle as O
import nsffn as N

REF = O.ref_gguf_available()

META = [
    ("general.architecture", W.STRING, "gemma4"),
    ("general.alignment", W.U32, 32),
    ("gemma4.block_count", W.U32, 11),
    ("gemma4.embedding_length", W.U64, 3840),
    ("gemma4.attention.layer_norm_rms_epsilon", W.F32, 1e-6),
    ("gemma4.rope.freq_base", W.F64, 1e6),
    ("gemma4.attention.sliding_window_pattern", W.ARRAY, (W.BOOL, [1, 1, 1, 1, 1, 0])),
    ("x.u8", W.U8, 200), ("x.i8", W.I8, -5), ("x.u16", W.U16, 65535), ("x.i16", W.I16, -300),
    ("x.i32", W.I32, -70000), ("x.i64", W.I64, -(1 << 40)), ("x.u64", W.U64, (1 << 63) + 5),
    ("x.bool", W.BOOL, 1),
    ("x.arr_u32", W.ARRAY, (W.U32, [1, 2, 3])), ("x.arr_i32", W.ARRAY, (W.I32, [-1, 7])),
    ("x.arr_f32", W.ARRAY, (W.F32, [0.5, -2.0])), ("x.arr_f64", W.ARRAY, (W.F64, [1e300])),
    ("x.arr_u64", W.ARRAY, (W.U64, [])), ("x.arr_str", W.ARRAY, (W.STRING, ["a", "bc", ""])),
]

TENSORS = [
    ("token_embd.weight", (256, 64), 14, None),
    ("output_norm.weight", (256,), 0, None),
    ("blk.0.ffn_gate.weight", (512, 64), 12, None),
    ("blk.0.ffn_up.weight", (512, 64), 12, None),
    ("blk.0.ffn_down.weight", (256, 128), 14, None),
    ("blk.0.ffn_norm.weight", (512,), 0, None),
    ("blk.10.ffn_gate.weight", (256, 64), 12, None),
    ("blk.10.ffn_down.weight", (256, 128), 12, None),
    ("blk.x.ffn_up.weight", (256, 64), 12, None),
    ("blk.1.ffn_up.weight.extra", (256, 64), 12, None),
    ("half.vector", (64,), 1, None),
    ("rank3", (4, 4, 16), 0, None),
]


@pytest.fixture(scope="module")
def written(tmp_path_factory):
    path = tmp_path_factory.mktemp("gguf") / "model.gguf"
    data, data_offset, offsets = W.write(path, META, TENSORS)
    return path, data, data_offset, offsets


def test_reads_what_was_written(written):
    path, data, data_offset, offsets = written
    g = N.GgufFile(path)
    assert g.data_offset() == data_offset and g.data_offset() % 32 == 0
    assert g.file_size() == len(data)
    want = [(n, t, tuple(s), off, W.tensor_nbytes(t, s)) for (n, s, t, _), off in zip(TENSORS, offsets)]
    assert g.tensors() == want
    for i, (n, t, s, off, nb) in enumerate(want):
        assert g.find(n) == i
        np.testing.assert_array_equal(g.bytes_at(data_offset + off, nb),
                                      np.frombuffer(data[data_offset + off:data_offset + off + nb], np.uint8))
    assert g.meta_string("general.architecture") == "gemma4"
    assert g.meta_u64("gemma4.block_count") == 11 and g.meta_u64("x.u64") == (1 << 63) + 5
    assert g.meta_u64("x.i8") == (1 << 64) - 5  # signed integers read as their u64 pattern
    assert g.meta_number("gemma4.rope.freq_base") == 1e6
    assert g.meta_number("gemma4.attention.layer_norm_rms_epsilon") == float(np.float32(1e-6))
    et, arr, n = g.meta_array("gemma4.attention.sliding_window_pattern")
    assert et == W.BOOL and list(arr) == [1, 1, 1, 1, 1, 0]
    assert list(g.meta_array("x.arr_i32")[1]) == [-1, 7]
    assert g.meta_array("x.arr_str")[0] == W.STRING and g.meta_array("x.arr_str")[2] == 3
    assert g.meta_array("x.arr_u64")[2] == 0
    assert g.has("x.bool") and not g.has("x.nope")
    with pytest.raises(N.NsError, match="missing tensor: nope"):
        g.find("nope")
    with pytest.raises(N.NsError, match="metadata is not integer: general.architecture"):
        g.meta_u64("general.architecture")
    with pytest.raises(N.NsError, match="missing GGUF metadata: x.nope"):
        g.meta_string("x.nope")


@pytest.mark.skipif(not REF, reason="oracle/_ref/libns_ref_gguf.so not built (no reference checkout)")
def test_matches_reference_reader(written):
    path = written[0]
    g, r = N.GgufFile(path), O.RefGguf(path)
    assert r.error is None
    assert (g.data_offset(), g.file_size()) == (r.data_offset(), r.file_size())
    assert g.tensors() == r.tensors()
    assert g.find("blk.0.ffn_up.weight") == 3 and r.find("blk.0.ffn_up.weight") is None
    assert r.find("nope") == "missing tensor: nope"
    for key, t, _ in META:
        if t in (W.STRING,):
            assert r.meta_string(key) == (g.meta_string(key), None)
        elif t == W.ARRAY:
            et, arr, n = g.meta_array(key)
            if et != W.STRING:
                np.testing.assert_array_equal(r.meta_array(key, et, N.GGUF_ARRAY_DTYPES[et]), arr)
        elif t == W.BOOL:  # neither reader reads a scalar bool as an integer
            assert r.meta_u64(key)[1] == f"metadata is not integer: {key}"
            with pytest.raises(N.NsError, match=f"metadata is not integer: {key}"):
                g.meta_u64(key)
        else:
            if t not in (W.F32, W.F64):
                assert r.meta_u64(key) == (g.meta_u64(key), None), key
            assert r.meta_number(key) == (g.meta_number(key), None), key
    assert r.meta_u64("general.architecture")[1] == "metadata is not integer: general.architecture"
    assert r.meta_string("x.nope")[1] == "missing GGUF metadata: x.nope"


@pytest.mark.parametrize("alignment", [1, 64, 4096])
def test_alignment(tmp_path, alignment):
    path = tmp_path / "a.gguf"
    meta = [("general.alignment", W.U32, alignment)]
    _, data_offset, offsets = W.write(path, meta, TENSORS[:3], alignment=alignment)
    g = N.GgufFile(path)
    assert g.data_offset() == data_offset and data_offset % alignment == 0
    assert [t[3] for t in g.tensors()] == offsets
    if REF:
        r = O.RefGguf(path)
        assert (r.data_offset(), r.tensors()) == (g.data_offset(), g.tensors())


def _malformed():
    base, _, _ = W.build(META[:3], TENSORS[:3])
    big = TENSORS[:2] + [("blk.0.ffn_gate.weight", (512, 64), 12, None)]
    cases = {
        "bad_magic": W.build(META, TENSORS, magic=b"GGML")[0],
        "version_2": W.build(META, TENSORS, version=2)[0],
        "too_many_tensors": W.build(META, TENSORS, counts=(100001, len(META)))[0],
        "too_many_keys": W.build(META, TENSORS, counts=(len(TENSORS), 100001))[0],
        "truncated_header": base[:30],  # inside the first key's length
        "truncated_in_tensor_table": base[:base.index(b"blk.0.ffn_gate.weight") + 23],  # inside the rank
        "rank_0": W.build([], [("t", (), 0, b"\0" * 4)])[0],
        "rank_5": W.build([], [("t", (1, 1, 1, 1, 4), 0, b"\0" * 16)])[0],
        "q4k_not_256": W.build([], [("blk.0.ffn_gate.weight", (100, 3), 12, b"\0" * 64)])[0],
        "unsupported_type": W.build([], [("q8", (256, 64), 8, b"\0" * 64)])[0],
        "outside_mapping": W.build([], big)[0][:-100],
        "string_too_long": W.build([("k", W.STRING, "v" * 8)], [])[0].replace(
            b"\x08\0\0\0\0\0\0\0vvvvvvvv", b"\xff\xff\0\0\0\0\0\0vvvvvvvv"),
        "array_too_long": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k"
                          + struct.pack("<IIQ", W.ARRAY, W.U8, (1 << 31) + 1) + b"\0" * 16,
        "nested_array": W.build([("k", W.ARRAY, (W.ARRAY, []))], [])[0],
    }
    return cases


EXPECTED = {
    "bad_magic": "bad GGUF magic", "version_2": "only GGUF v3 is supported",
    "too_many_tensors": "invalid GGUF counts", "too_many_keys": "invalid GGUF counts",
    "truncated_header": "truncated GGUF header", "truncated_in_tensor_table": "truncated GGUF header",
    "rank_0": "invalid tensor rank", "rank_5": "invalid tensor rank",
    "q4k_not_256": "invalid quantized tensor shape: blk.0.ffn_gate.weight",
    "unsupported_type": "unsupported tensor type 8: q8",
    "outside_mapping": "tensor outside GGUF mapping: blk.0.ffn_gate.weight",
    "string_too_long": "invalid GGUF string length", "array_too_long": "unreasonable GGUF array length",
    "nested_array": "nested/invalid GGUF array type",
}


@pytest.mark.parametrize("case", sorted(EXPECTED))
def test_malformed_files_fail_like_the_reference(tmp_path, case):
    path = tmp_path / f"{case}.gguf"
    data = _malformed()[case]
    path.write_bytes(data)
    with pytest.raises(N.NsError) as e:
        N.GgufFile(path)
    assert EXPECTED[case] in str(e.value), str(e.value)
    if REF:
        assert O.RefGguf(path).error == EXPECTED[case]


def test_ffn_table(written):
    """blk.<i>.ffn_{gate,up,down}.weight get (layer, kind); everything else NS_FFN_NONE."""
    path, _, _, offsets = written
    t = N.GgufFile(path).ffn_table()
    none = 0xFFFFFFFF
    want = {"blk.0.ffn_gate.weight": (0, 0), "blk.0.ffn_up.weight": (0, 1), "blk.0.ffn_down.weight": (0, 2),
            "blk.10.ffn_gate.weight": (10, 0), "blk.10.ffn_down.weight": (10, 2)}
    for row, (name, shape, ttype, _), off in zip(t, TENSORS, offsets):
        assert (int(row["layer"]), int(row["kind"])) == want.get(name, (none, none)), name
        assert (int(row["source_offset"]), int(row["type"]), int(row["cols"])) == (off, ttype, shape[0])
        assert int(row["bytes"]) == W.tensor_nbytes(ttype, shape)


def test_gguf_to_nsmffn_chain(tmp_path):
    """A GGUF file through the reader, the table and the .nsmffn converter: FFN matrices come
    back re-laid in 64-row slabs (equal to ns_retile ROW_MAJOR -> NSMFFN of their GGUF bytes),
    other tensors unchanged, and MetalFfnFile validates the result."""
    q4 = N.synth_blocks(N.Q4_K, 5, 2 * 64)     # 512 x 64 Q4_K
    q6 = N.synth_blocks(N.Q6_K, 6, 1 * 128)    # 256 x 128 Q6_K
    tensors = [("token_embd.weight", (256, 64), 14, None), ("blk.0.ffn_gate.weight", (512, 64), 12, q4.tobytes()),
               ("blk.0.ffn_down.weight", (256, 128), 14, q6.tobytes()), ("blk.0.ffn_norm.weight", (512,), 0, None)]
    gpath = tmp_path / "m.gguf"
    # a vocabulary puts the data section past the .nsmffn header page, as in any real model file
    vocab = [("tokenizer.ggml.tokens", W.ARRAY, (W.STRING, [f"tok{i:06d}" for i in range(8192)]))]
    data, data_offset, offsets = W.write(gpath, META[:2] + vocab, tensors)
    assert data_offset > 65536
    g = N.GgufFile(gpath)
    table = g.ffn_table()
    out = tmp_path / "m.nsmffn"
    image = np.frombuffer(data, dtype=np.uint8)
    N.nsmffn_convert(out, image, g.data_offset(), table)
    fp = N.nsmffn_fingerprint(image[:g.data_offset()], g.file_size())
    f = N.NsmffnFile(out, g.file_size(), fp, table)
    for (name, shape, ttype, raw), off in zip(tensors, offsets):
        pos, reordered = f.lookup(off)
        nb = W.tensor_nbytes(ttype, shape)
        got = f.view(pos, nb)
        src = np.frombuffer(data[data_offset + off:data_offset + off + nb], np.uint8)
        if name.startswith("blk.0.ffn_gate") or name.startswith("blk.0.ffn_down"):
            assert reordered
            np.testing.assert_array_equal(got, N.retile(src, ttype, shape[0], shape[1], N.ROW_MAJOR, N.NSMFFN))
        else:
            assert not reordered
            np.testing.assert_array_equal(got, src)
