"""CPU tests of the GGUF reader (include/rrr_gguf.h), the writer and the
model configuration read from metadata.

The reader is checked against a hand-assembled image (every field written out
by hand from the specification's layout), against the restatement of the
reference's reader (oracle/gguf_ref.py) on every file the reference reads
correctly, and against the writer over every value type, ggml type and
alignment.  Malformed files -- each truncation of a valid file, mutants, and
one case per validation rule -- must be rejected with an error code, never
read out of bounds (a sanitizer build runs the mutants).
"""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import rrr_hip
from oracle import gguf_ref as R
from rrr_hip import decode
from rrr_hip import gguf as G
from rrr_hip.engine import (ERR_BAD_SHAPE, ERR_BAD_TYPE, ERR_FORMAT, ERR_INVALID_ARG, ERR_IO, ERR_NO_DEVICE,
                            ERR_NOT_FOUND, ERR_STALE, ERR_STATE)

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)


def le(v, n):
    return int(v).to_bytes(n, "little", signed=v < 0)


# Block sizes of the ggml types as the sums of their block structs' fields
# (ggml-common.h: d/dmin halves, scale bytes, quant bytes): independent of the
# reader's table.
BLOCK = {
    0: (1, 4), 1: (1, 2), 2: (32, 2 + 16), 3: (32, 2 + 2 + 16), 6: (32, 2 + 4 + 16), 7: (32, 2 + 2 + 4 + 16),
    8: (32, 2 + 32), 9: (32, 2 + 2 + 32), 10: (256, 16 + 64 + 2 + 2), 11: (256, 32 + 64 + 12 + 2),
    12: (256, 2 + 2 + 12 + 128), 13: (256, 2 + 2 + 12 + 32 + 128), 14: (256, 128 + 64 + 16 + 2),
    15: (256, 4 + 256 + 32), 16: (256, 2 + 64), 17: (256, 2 + 64 + 8), 18: (256, 2 + 96), 19: (256, 2 + 32 + 16),
    20: (32, 2 + 16), 21: (256, 2 + 64 + 8 + 32 + 4), 22: (256, 2 + 64 + 8 + 8), 23: (256, 2 + 2 + 4 + 128),
    24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8), 29: (256, 32 + 16 + 8), 30: (1, 2),
    34: (256, 48 + 4 + 2), 35: (256, 64 + 2), 39: (32, 1 + 16),
}


def kat_image():
    """Hand-assembled GGUF v3: 2 metadata pairs (a UINT8 and a STRING), one
    256 x 1 Q4_K tensor.  Offsets by hand: header 24 bytes; pair 1 = 8 + 4
    (key) + 4 (type) + 1 (value) -> byte 41; pair 2 = 8 + 4 + 4 + 8 + 2 ->
    byte 67; tensor record = 8 + 1 + 4 + 2 * 8 + 4 + 8 -> byte 108; data at
    the next multiple of 32, byte 128; one 144-byte block -> 272 bytes."""
    img = (b"GGUF" + le(3, 4) + le(1, 8) + le(2, 8)
           + le(4, 8) + b"a.u8" + le(0, 4) + b"\x07"
           + le(4, 8) + b"b.st" + le(8, 4) + le(2, 8) + b"hi"
           + le(1, 8) + b"w" + le(2, 4) + le(256, 8) + le(1, 8) + le(12, 4) + le(0, 8))
    assert len(img) == 108
    img += b"\0" * 20 + bytes(range(144))
    assert len(img) == 272
    return img


def test_known_answer_image():
    img = kat_image()
    m = G.GGUFModel(data=img)
    assert (m.version, m.n_tensors, m.n_kv, m.alignment, m.data_offset) == (3, 1, 2, 32, 128)
    assert m.metadata == {"a.u8": 7, "b.st": "hi"}
    assert m.metadata_types == {"a.u8": (G.UINT8, G.UINT8), "b.st": (G.STRING, G.STRING)}
    assert m.tensor_infos == [G.TensorInfo("w", (256, 1), 12, 0, 256, 144)]
    assert m.tensor_bytes("w").tobytes() == bytes(range(144))
    assert m.get_u64("a.u8") == 7 and m.get_str("b.st") == "hi"


def test_writer_reproduces_known_answer_image(tmp_path):
    p = tmp_path / "kat.gguf"
    off = G.write_gguf(p, [("a.u8", G.UINT8, 7), ("b.st", G.STRING, "hi")],
                       [("w", 12, (256, 1), np.arange(144, dtype=np.uint8))])
    assert off == 128
    assert p.read_bytes() == kat_image()


def test_reference_misreads_uint8():
    """gguf.rs:100 reads a UINT8 value as 4 bytes: in the image above it takes
    07 04 00 00 (the value and the low bytes of the next key's length), 0x407
    = 1031, then reads the next key's length from the wrong bytes and panics
    on the slice; the product reader returns 7 and the rest of the file."""
    img = kat_image()
    r = R.Reader(img)
    r.pos = 24 + 8 + 4 + 4
    assert r.value(0) == ("U32", 1031)
    with pytest.raises(R.RefPanic):
        R.RefModel(img)
    assert G.GGUFModel(data=img).metadata["b.st"] == "hi"


def all_types_metadata(with_narrow):
    """Every value type (UINT8/INT8 only if with_narrow: the reference
    misreads them), arrays of each, strings, nested arrays, bool."""
    md = [("general.architecture", G.STRING, "phi3"),
          ("u16", G.UINT16, 65535), ("i16", G.INT16, -32768), ("u32", G.UINT32, 4000000000),
          ("i32", G.INT32, -2000000000), ("f32", G.FLOAT32, 1.5), ("bool", G.BOOL, True), ("boolf", G.BOOL, False),
          ("str", G.STRING, "héllo ☃"), ("empty", G.STRING, ""), ("u64", G.UINT64, 2 ** 64 - 1),
          ("i64", G.INT64, -2 ** 63), ("f64", G.FLOAT64, -2.25e300),
          ("a.i32", G.ARRAY, (G.INT32, np.array([1, -2, 3], np.int32))),
          ("a.f32", G.ARRAY, (G.FLOAT32, np.array([0.5, -1e30], np.float32))),
          ("a.str", G.ARRAY, (G.STRING, ["a", "", "üñî"])),
          ("a.empty", G.ARRAY, (G.UINT64, np.zeros(0, np.uint64))),
          ("a.bool", G.ARRAY, (G.BOOL, [True, False, True])),
          ("a.nest", G.ARRAY, (G.ARRAY, [(G.UINT32, [1, 2]), (G.STRING, ["x", "yz"]), (G.ARRAY, [(G.INT16, [-1])])]))]
    if with_narrow:
        md += [("u8", G.UINT8, 255), ("i8", G.INT8, -128),
               ("a.u8", G.ARRAY, (G.UINT8, np.arange(7, dtype=np.uint8))),
               ("a.i8", G.ARRAY, (G.INT8, np.array([-1, 2], np.int8))), ("after", G.UINT32, 12345)]
    return md


def expected_value(vtype, value):
    if vtype == G.ARRAY:
        et, items = value
        if et in (G.STRING, G.ARRAY):
            return [expected_value(et, it) for it in items]
        return list(np.asarray(items).tolist())
    if vtype == G.FLOAT32:
        return float(np.float32(value))
    return value


def normalize(v):
    if isinstance(v, np.ndarray):
        return v.tolist()
    if isinstance(v, list):
        return [normalize(x) for x in v]
    return v


def random_tensors(rng, types):
    out = []
    for i, t in enumerate(types):
        be, bb = BLOCK[t]
        ne0 = be * int(rng.integers(1, 4))
        shape = (ne0,) if i % 3 == 0 else (ne0, int(rng.integers(1, 4))) if i % 3 == 1 else (ne0, 2, 3)
        n = int(np.prod(shape))
        out.append((f"t{i}.{t}", t, shape, rng.integers(0, 256, n // be * bb, dtype=np.uint8)))
    return out


@pytest.mark.parametrize("alignment", [1, 8, 32, 64, 4096])
def test_roundtrip_every_value_and_ggml_type(tmp_path, alignment):
    rng = np.random.default_rng(alignment)
    md = all_types_metadata(with_narrow=True)
    tensors = random_tensors(rng, sorted(BLOCK))
    p = tmp_path / "all.gguf"
    off = G.write_gguf(p, md, tensors, alignment=alignment)
    with G.GGUFModel.load(p) as m:
        assert m.version == 3 and m.alignment == alignment and m.data_offset == off
        assert off % alignment == 0
        exp = {k: expected_value(t, v) for k, t, v in md}
        if alignment != 32:
            exp["general.alignment"] = alignment
        assert {k: normalize(v) for k, v in m.metadata.items()} == exp
        assert m.get_u64("u8") == 255 and m.get_u64("after") == 12345 and m.get_u64("u64") == 2 ** 64 - 1
        assert m.get_f64("f64") == -2.25e300 and m.get_f64("f32") == 1.5
        for code, key in ((ERR_INVALID_ARG, "i8"), (ERR_INVALID_ARG, "i64"), (ERR_BAD_TYPE, "str"),
                          (ERR_BAD_TYPE, "bool"), (ERR_NOT_FOUND, "missing")):
            with pytest.raises(rrr_hip.RrrError) as e:
                m.get_u64(key)
            assert e.value.code == code
        with pytest.raises(rrr_hip.RrrError) as e:
            m.get_f64("u32")
        assert e.value.code == ERR_BAD_TYPE
        assert len(m.tensor_infos) == len(tensors)
        for info, (name, t, shape, raw) in zip(m.tensor_infos, tensors):
            be, bb = BLOCK[t]
            assert (info.name, info.shape, info.typ) == (name, shape, t)
            assert info.offset % alignment == 0
            assert info.nbytes == raw.nbytes == int(np.prod(shape)) // be * bb
            assert np.array_equal(m.tensor_bytes(name), raw)


def test_type_table_matches_block_structs_and_reference():
    for t in range(64):
        if t in BLOCK:
            assert G.type_size(t) == BLOCK[t]
        else:
            with pytest.raises(rrr_hip.RrrError) as e:
                G.type_size(t)
            assert e.value.code == ERR_BAD_TYPE
    for t, size in R.RefModel.SIZES.items():   # the reference's 11 types (gguf.rs:179-189)
        assert BLOCK[t] == size


def test_agrees_with_reference_where_it_reads_correctly(tmp_path):
    """On files without UINT8/INT8 values and with the reference's 11 tensor
    types, both readers give the same metadata, tensor records, data offset
    and tensor bytes."""
    rng = np.random.default_rng(7)
    md = all_types_metadata(with_narrow=False)
    tensors = random_tensors(rng, sorted(R.RefModel.SIZES) * 2)
    for alignment in (32, 64):
        p = tmp_path / f"ref{alignment}.gguf"
        G.write_gguf(p, md, tensors, alignment=alignment)
        ref = R.RefModel(p.read_bytes())
        with G.GGUFModel.load(p) as m:
            assert ref.data_offset == m.data_offset and ref.version == m.version
            assert [(n, tuple(s), t, o) for n, s, t, o in ref.tensor_infos] == \
                [(i.name, i.shape, i.typ, i.offset) for i in m.tensor_infos]

            def untag(v):
                tag, x = v
                return [untag(e) for e in x] if tag == "Array" else x

            assert {k: untag(v) for k, v in ref.metadata.items()} == {k: normalize(v) for k, v in m.metadata.items()}
            for i in m.tensor_infos:
                assert ref.tensor_bytes(i.name) == m.tensor_bytes(i.name).tobytes()


def test_reference_desynchronises_on_uint8_array(tmp_path):
    """A UINT8 array (e.g. tokenizer.ggml.precompiled_charsmap of SentencePiece
    GGUFs) before other keys: the reference reads each element as 4 bytes and
    loses the file; the product reader keeps every key and tensor."""
    p = tmp_path / "charsmap.gguf"
    md = [("tokenizer.ggml.precompiled_charsmap", G.ARRAY, (G.UINT8, np.arange(40, dtype=np.uint8))),
          ("phi3.block_count", G.UINT32, 32)]
    G.write_gguf(p, md, [("w", 0, (4,), np.ones(4, np.float32))])
    with G.GGUFModel.load(p) as m:
        assert m.get_u64("phi3.block_count") == 32
        assert np.array_equal(m.metadata["tokenizer.ggml.precompiled_charsmap"], np.arange(40))
    try:
        ref = R.RefModel(p.read_bytes())
    except R.RefPanic:
        return
    assert R.as_u64(ref.metadata.get("phi3.block_count", ("Bool", 0))) != 32


def test_every_truncation_is_rejected(tmp_path):
    rng = np.random.default_rng(1)
    p = tmp_path / "t.gguf"
    G.write_gguf(p, all_types_metadata(True)[:12], random_tensors(rng, [12, 0, 14]))
    img = p.read_bytes()
    G.GGUFModel(data=img).close()
    for n in range(len(img)):
        with pytest.raises(rrr_hip.RrrError) as e:
            G.GGUFModel(data=img[:n] if n else b"\0")
        assert e.value.code == ERR_FORMAT, (n, e.value)


def test_mutants_are_parsed_or_rejected():
    """Random overwrites, truncations and extreme counts: each mutant is
    either rejected with an error code or parsed with every tensor inside the
    image."""
    rng = np.random.default_rng(2)
    tensors = random_tensors(rng, [12, 13, 14, 0])
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "m.gguf")
        G.write_gguf(p, all_types_metadata(True), tensors)
        img = bytearray(open(p, "rb").read())
    accepted = 0
    for it in range(1500):
        m = bytearray(img)
        for _ in range(int(rng.integers(1, 6))):
            at = int(rng.integers(0, min(len(m), 700)))
            m[at] = int(rng.integers(0, 256))
        try:
            g = G.GGUFModel(data=bytes(m))
        except rrr_hip.RrrError as e:
            assert e.code < 0
            continue
        accepted += 1
        for i in g.tensor_infos:
            assert g.data_offset + i.offset + i.nbytes <= len(m)
        g.close()
    assert 0 < accepted < 1500


def expect_format(img, fragment):
    with pytest.raises(rrr_hip.RrrError) as e:
        G.GGUFModel(data=img)
    assert e.value.code == ERR_FORMAT and fragment in e.value.msg, e.value.msg


def header(n_tensors, n_kv, version=3):
    return b"GGUF" + le(version, 4) + le(n_tensors, 8) + le(n_kv, 8)


def kv(key, vtype, payload):
    return le(len(key), 8) + key.encode() + le(vtype, 4) + payload


def tensor(name, dims, typ, offset):
    return le(len(name), 8) + name.encode() + le(len(dims), 4) + b"".join(le(d, 8) for d in dims) + le(typ, 4) + \
        le(offset, 8)


def test_rejections():
    pad = b"\0" * 64
    expect_format(b"GGUX" + b"\0" * 20, "not a GGUF file")
    expect_format(header(0, 0, version=1), "version 1")
    expect_format(header(0, 0, version=0x03000000), "big-endian")
    expect_format(header(0, 0, version=4), "unsupported GGUF version 4")
    expect_format(header(0, 1) + kv("k", 13, b"\0" * 8), "unknown value type 13")
    expect_format(header(0, 1) + kv("k", G.ARRAY, le(13, 4) + le(1, 8) + b"\0" * 8), "unknown array element type")
    expect_format(header(0, 1 << 60), "metadata pairs cannot fit")
    expect_format(header(0, 1) + kv("k", G.ARRAY, le(G.UINT32, 4) + le(1 << 62, 8)), "run past the end")
    expect_format(header(0, 1) + kv("k", G.ARRAY, le(G.STRING, 4) + le(1 << 40, 8)), "cannot fit")
    expect_format(header(0, 1) + kv("k", G.STRING, le(1 << 63, 8) + b"ab"), "runs past the end")
    nest = le(G.UINT32, 4) + le(0, 8)
    for _ in range(5):
        nest = le(G.ARRAY, 4) + le(1, 8) + nest
    expect_format(header(0, 1) + kv("k", G.ARRAY, nest), "nested deeper")
    expect_format(header(0, 2) + kv("k", G.UINT32, le(1, 4)) + kv("k", G.UINT32, le(2, 4)), "duplicate metadata key")
    expect_format(header(0, 1) + le(2, 8) + b"\xff\xfe" + le(G.UINT32, 4) + le(1, 4), "not UTF-8")
    expect_format(header(0, 1) + le(2, 8) + b"a\0" + le(G.UINT32, 4) + le(1, 4), "NUL")
    expect_format(header(1 << 59, 0), "tensor records cannot fit")
    expect_format(header(1, 0) + tensor("w", [1, 1, 1, 1, 1], 0, 0) + pad, "at most 4")
    expect_format(header(1, 0) + tensor("w", [256], 4, 0) + pad, "unknown ggml type 4")
    expect_format(header(1, 0) + tensor("w", [256], 99, 0) + pad, "unknown ggml type 99")
    expect_format(header(1, 0) + tensor("w", [100, 2], 12, 0) + pad, "not a multiple of the 256-element Q4_K")
    expect_format(header(1, 0) + tensor("w", [1 << 40, 1 << 40], 0, 0) + pad, "overflows")
    expect_format(header(1, 0) + tensor("w", [1 << 62, 8], 0, 0) + pad, "overflows")
    expect_format(header(2, 0) + tensor("w", [4], 0, 0) + tensor("w", [4], 0, 32) + pad, "duplicate tensor name")
    expect_format(header(1, 0) + tensor("w", [4], 0, 16) + pad, "not a multiple of the alignment 32")
    expect_format(header(1, 0) + tensor("w", [64], 0, 0) + pad, "past the end of the file")
    expect_format(header(1, 0) + tensor("w", [4], 0, 1 << 63) + pad, "past the end of the file")
    for a, vt in ((0, G.UINT32), (3, G.UINT32), (1 << 31, G.UINT64), (-32, G.INT32)):
        payload = struct.pack(G._SCALAR[vt][0], a)
        expect_format(header(0, 1) + kv("general.alignment", vt, payload), "general.alignment")
    expect_format(header(0, 1) + kv("general.alignment", G.STRING, le(2, 8) + b"32"), "not an integer")


def test_accepts_edge_files():
    # no metadata, no tensors: the header alone (data offset rounded past the end)
    with G.GGUFModel(data=header(0, 0)) as m:
        assert (m.n_kv, m.n_tensors, m.data_offset) == (0, 0, 32)
    # version 2, alignment from an INT64 key, a zero-element tensor at the end
    body = header(1, 1, version=2) + kv("general.alignment", G.INT64, le(8, 8)) + tensor("z", [0, 3], 12, 0)
    with G.GGUFModel(data=body) as m:
        assert m.version == 2 and m.alignment == 8 and m.tensor_infos[0].nbytes == 0
        assert m.tensor_bytes("z").size == 0


def test_handles_and_errors(tmp_path):
    lib = rrr_hip._lib.hip()
    import ctypes
    h = ctypes.c_void_p()
    assert lib.rrr_gguf_open(str(tmp_path / "missing.gguf").encode(), ctypes.byref(h)) == ERR_IO
    assert h.value is None
    assert lib.rrr_gguf_open(str(tmp_path).encode(), ctypes.byref(h)) == ERR_IO
    (tmp_path / "empty.gguf").write_bytes(b"")
    assert lib.rrr_gguf_open(str(tmp_path / "empty.gguf").encode(), ctypes.byref(h)) == ERR_FORMAT
    assert lib.rrr_gguf_close(None) == 0
    m = G.GGUFModel(data=kat_image())
    raw = m._handle
    view = m.tensor_bytes("w")
    with pytest.raises(rrr_hip.RrrError) as e:
        m.close()
    assert e.value.code == ERR_STATE
    del view
    m.close()
    assert lib.rrr_gguf_close(raw) == ERR_STALE
    t = rrr_hip._lib.GgufTensor()
    assert lib.rrr_gguf_find_tensor(raw, b"w", ctypes.byref(t)) == ERR_STALE
    with pytest.raises(rrr_hip.RrrError):
        m.tensor_bytes("w")


def test_string_array_ranges():
    md = [("toks", G.ARRAY, (G.STRING, [f"tok{i}" for i in range(1000)])), ("one", G.STRING, "solo")]
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "s.gguf")
        G.write_gguf(p, md, [])
        with G.GGUFModel.load(p) as m:
            assert m.metadata["toks"][999] == "tok999" and m.metadata["one"] == "solo"
            lib, import_ct = rrr_hip._lib.hip(), __import__("ctypes")
            ptrs, lens = (import_ct.c_void_p * 3)(), (import_ct.c_uint64 * 3)()
            assert lib.rrr_gguf_kv_strings(m._h, 0, 998, 3, ptrs, lens) == ERR_INVALID_ARG
            assert lib.rrr_gguf_kv_strings(m._h, 0, 997, 3, ptrs, lens) == 0
            assert import_ct.string_at(ptrs[2], lens[2]) == b"tok999"
            assert lib.rrr_gguf_kv_strings(m._h, 1, 0, 1, ptrs, lens) == 0
            assert import_ct.string_at(ptrs[0], lens[0]) == b"solo"
            assert lib.rrr_gguf_kv_strings(m._h, 1, 1, 1, ptrs, lens) == ERR_INVALID_ARG
            assert lib.rrr_gguf_kv_strings(m._h, 1, 1, 2 ** 64 - 1, ptrs, lens) == ERR_INVALID_ARG   # no wrap
            assert lib.rrr_gguf_kv_strings(m._h, 0, 1, 2 ** 64 - 1, ptrs, lens) == ERR_INVALID_ARG


def test_upload_validation_without_device(tmp_path):
    p = tmp_path / "u.gguf"
    G.write_gguf(p, [], [("q8", 8, (256, 2), np.zeros(2 * 8 * 34, np.uint8)),
                         ("f", 0, (100,), np.zeros(100, np.float32)),
                         ("q4", 12, (512, 3), np.zeros(3 * 2 * 144, np.uint8))])
    with G.GGUFModel.load(p) as m, rrr_hip.Context(rrr_hip.DEVICE_NONE) as ctx:
        for name, code in (("q8", ERR_BAD_TYPE), ("f", ERR_BAD_SHAPE), ("nope", ERR_NOT_FOUND),
                           ("q4", ERR_NO_DEVICE)):
            with pytest.raises(rrr_hip.RrrError) as e:
                m.upload(ctx, name)
            assert e.value.code == code, (name, e.value)
            if code != ERR_NOT_FOUND:
                assert f"'{name}'" in e.value.msg


PHI4_MINI_MD = [
    ("general.architecture", G.STRING, "phi3"), ("general.name", G.STRING, "Phi 4 Mini"),
    ("phi3.context_length", G.UINT32, 131072), ("phi3.rope.scaling.original_context_length", G.UINT32, 4096),
    ("phi3.embedding_length", G.UINT32, 3072), ("phi3.feed_forward_length", G.UINT32, 8192),
    ("phi3.block_count", G.UINT32, 32), ("phi3.attention.head_count", G.UINT32, 24),
    ("phi3.attention.head_count_kv", G.UINT32, 8), ("phi3.attention.layer_norm_rms_epsilon", G.FLOAT32, 1e-5),
    ("phi3.rope.dimension_count", G.UINT32, 96), ("phi3.rope.freq_base", G.FLOAT32, 10000.0),
    ("phi3.rope.scaling.attn_factor", G.FLOAT32, 1.190238), ("general.file_type", G.UINT32, 15),
    ("tokenizer.ggml.model", G.STRING, "gpt2"), ("tokenizer.ggml.add_bos_token", G.BOOL, False),
    ("general.quantization_version", G.UINT32, 2),
]


def test_model_config_from_phi4_mini_metadata(tmp_path):
    """ModelConfig::from_gguf (phi4.rs:31-101) on the Phi-4-mini key set: the
    decode shape is the 3072 / 24 / 8 / 8192 / 32-layer model (a 512-entry
    token_embd stands in for the 200064-entry one)."""
    p = tmp_path / "phi4.gguf"
    d = 3072
    tensors = [("token_embd.weight", 14, (d, 512), np.zeros(512 * 12 * 210, np.uint8)),
               ("rope_factors_short.weight", 0, (48,), np.ones(48, np.float32)),
               ("blk.0.attn_qkv.weight", 13, (d, 5120), np.zeros(5120 * 12 * 176, np.uint8)),
               ("blk.0.ffn_up.weight", 12, (d, 16384), np.zeros(16384 * 12 * 144, np.uint8))]
    G.write_gguf(p, PHI4_MINI_MD, tensors)
    with G.GGUFModel.load(p) as m:
        cfg = G.ModelConfig.from_gguf(m)
    assert (cfg.arch, cfg.d_model, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn_dim, cfg.n_layers,
            cfg.vocab_size, cfg.rope_dim) == ("phi3", 3072, 24, 8, 128, 8192, 32, 512, 96)
    assert cfg.rms_eps == float(np.float32(1e-5)) and cfg.rope_theta == 10000.0
    assert cfg.rope_attn_factor == float(np.float32(1.190238))
    assert cfg.has_rope_factors and not (cfg.separate_qkv or cfg.separate_gate_up or cfg.has_qkv_bias)
    assert not cfg.has_output_weight and cfg.qkv_dim == 5120 and cfg.gate_up_dim == 16384
    s = decode.shape_from_config(cfg)
    ref = decode.Phi4Shape()
    assert (s.d_model, s.n_layers, s.n_heads, s.n_kv_heads, s.head_dim, s.ffn_dim, s.rope_dim, s.qkv_dim) == \
        (ref.d_model, ref.n_layers, ref.n_heads, ref.n_kv_heads, ref.head_dim, ref.ffn_dim, ref.rope_dim, ref.qkv_dim)
    assert np.float32(s.eps) == np.float32(ref.eps) and np.float32(s.rope_attn_factor) == np.float32(
        ref.rope_attn_factor)


def test_model_config_defaults():
    """Missing keys take the reference's defaults: arch "llama", head_dim
    128, eps 1e-5, full-width rotation, theta 10000, attention factor 1."""
    with G.GGUFModel(data=header(0, 0)) as m:
        cfg = G.ModelConfig.from_gguf(m)
    assert (cfg.arch, cfg.d_model, cfg.head_dim, cfg.rms_eps, cfg.rope_dim, cfg.rope_theta, cfg.rope_attn_factor,
            cfg.vocab_size) == ("llama", 0, 128, 1e-5, 128, 10000.0, 1.0, 0)
    body = header(0, 3) + kv("general.architecture", G.STRING, le(5, 8) + b"qwen2") + \
        kv("qwen2.embedding_length", G.UINT16, le(896, 2)) + kv("qwen2.attention.head_count", G.UINT8, le(14, 1))
    with G.GGUFModel(data=body) as m:
        cfg = G.ModelConfig.from_gguf(m)
    assert (cfg.arch, cfg.d_model, cfg.n_heads, cfg.head_dim) == ("qwen2", 896, 14, 64)


def test_synthetic_export_matches_the_synthetic_tensors(tmp_path):
    """write_synthetic_gguf holds the same bytes as the seeded tensors the
    synthetic sweep uploads, under the names the GGUF loader reads."""
    import dataclasses
    s = dataclasses.replace(decode.Phi4Shape(), n_layers=2, vocab=512, d_model=512, ffn_dim=1024, n_heads=4,
                            n_kv_heads=2)
    p = tmp_path / "syn.gguf"
    decode.write_synthetic_gguf(p, s, seed=5, alignment=64)
    with G.GGUFModel.load(p) as m:
        cfg = G.ModelConfig.from_gguf(m)
        assert decode.shape_from_config(cfg).qkv_dim == s.qkv_dim and cfg.n_layers == 2
        for i in range(2):
            h = decode.layer_host(5, s, i)
            for name, qt, K, N in s.layer_tensors(i):
                info = m.tensor_info(f"blk.{i}.{name}.weight")
                assert (info.typ, info.shape) == (qt, (K, N))
                assert np.array_equal(m.tensor_bytes(info.name), h[name].view(np.uint8))
            assert np.array_equal(m.tensor_f32(f"blk.{i}.ffn_norm.weight"), h["ffn_norm"])
        assert np.array_equal(m.tensor_bytes("token_embd.weight"), decode.embedding_q6k_host(5, s).view(np.uint8))
        assert np.array_equal(m.tensor_f32("rope_factors_short.weight"), decode.rope_factors_host(5, s))
        ref = R.RefModel(p.read_bytes())
        assert ref.data_offset == m.data_offset
        assert ref.tensor_bytes("blk.1.ffn_down.weight") == m.tensor_bytes("blk.1.ffn_down.weight").tobytes()


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_sanitized_mutation_run(tmp_path):
    """gguf.cpp built with AddressSanitizer and UBSan (host code only) parses
    6000 mutants of a file and reads every range it returns."""
    exe = tmp_path / "fuzz"
    src = os.path.join(REPO, "recursive-routing-racer-rs_amd", "csrc", "gguf.cpp")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", os.path.join(REPO, "include"), src, os.path.join(HERE, "gguf_fuzz_driver.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=240)
    rng = np.random.default_rng(3)
    img = tmp_path / "seed.gguf"
    G.write_gguf(img, all_types_metadata(True), random_tensors(rng, [12, 14, 0, 8]))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe), str(img), "6000", "11"], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "mutants 6000" in r.stdout
