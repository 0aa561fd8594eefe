"""Safetensors and GGUF tensor tables (qnn_tensor_files_*, qnn_gguf_*), host only.

The library's readers are checked against three independent sources:
  * the `safetensors` package (Hugging Face's own reader and writer) for what
    a safetensors file holds;
  * files built byte by byte from the GGUF specification (tests/gguf_writer.py),
    whose expected tables follow from construction (shape reversed from ne[],
    byte size = elements / block * block bytes);
  * oracle/formats.py, the pure-Python restatement of SafeTensors.pas:522-690
    and GGUF.pas:206-337, on every file, malformed ones included.
"""
import json
import os
import struct

import numpy as np
import pytest

from oracle import formats as of
from tests.gguf_writer import ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64, gguf_bytes

ck = pytest.importorskip("quicknn_amd.checkpoint")
from quicknn_amd import hip  # noqa: E402


def st_bytes(header, data: bytes = b"", raw_header: bytes | None = None, pad: bool = True) -> bytes:
    h = raw_header if raw_header is not None else json.dumps(header, separators=(",", ":")).encode()
    if pad:
        h += b" " * ((-len(h)) % 8)
    return struct.pack("<Q", len(h)) + h + data


def write(tmp_path, name: str, blob: bytes) -> str:
    p = os.path.join(tmp_path, name)
    with open(p, "wb") as f:
        f.write(blob)
    return p


# ---------------------------------------------------------------------------
# safetensors
# ---------------------------------------------------------------------------
def test_reads_what_the_safetensors_package_writes(tmp_path):
    import safetensors.numpy as sn

    rng = np.random.default_rng(0)
    tensors = {
        "model.embed_tokens.weight": rng.standard_normal((17, 24)).astype(np.float32),
        "model.layers.0.self_attn.q_proj.weight": rng.standard_normal((8, 24)).astype(np.float16),
        "ids": np.arange(7, dtype=np.int64),
        "bytes": rng.integers(0, 255, (3, 5), dtype=np.uint8),
        "i32": rng.integers(-9, 9, (2, 2, 3), dtype=np.int32),
        "f64": rng.standard_normal(3),
        "empty": np.zeros((0, 4), np.float32),
    }
    p = os.path.join(tmp_path, "model.safetensors")
    sn.save_file(tensors, p, metadata={"format": "pt", "note": "x"})
    ora = of.parse_safetensors(p)
    with ck.SafeTensorFiles.Open(p) as f:
        (info,) = f.files
        assert not info.is_gguf and info.file_size == os.path.getsize(p)
        assert info.header_json == ora["header"] and info.offset == ora["offset"] == 8 + info.header_size
        got = f.Tensors()
        assert [(t.name, t.st_dtype, t.shape, t.data_offset, t.data_size) for t in got] == ora["tensors"]
        assert len({t.identity for t in got}) == len(got) and all(t.identity >> 63 for t in got)
        for name, v in tensors.items():
            a = f.array(name)
            assert a.dtype == v.dtype and a.shape == v.shape and np.array_equal(a, v), name
        assert f.GetTensor("absent") is None


def test_bf16_linear_weights_are_mapped_views(tmp_path):
    torch = pytest.importorskip("torch")
    import safetensors.torch as stt

    w = torch.randn(6, 40, dtype=torch.float32).to(torch.bfloat16)
    h = torch.randn(3, 8, dtype=torch.float16)
    v = torch.randn(5)
    p = os.path.join(tmp_path, "m.safetensors")
    stt.save_file({"w": w, "h": h, "v": v}, p)
    with ck.SafeTensorFiles.Open(p) as f:
        t = f.GetTensor("w")
        assert t.st_dtype == ck.ST_BF16 and t.dtype == hip.DT_BF16
        blk = f.GetLinearWeight("w")
        assert (blk.dtype, blk.shape, blk.size, blk.identity) == (hip.DT_BF16, (6, 40), 240, t.identity)
        assert blk.data.ctypes.data == t.data  # a view of the mapping, not a copy
        assert np.array_equal(blk.data.view(np.uint16).reshape(6, 40), w.view(torch.int16).numpy().view(np.uint16))
        # F16 -> an F32 copy (AsSingle), exactly the half values widened.
        hb = f.GetLinearWeight("h")
        assert hb.dtype == hip.DT_F32 and hb.shape == (3, 8)
        assert np.array_equal(hb.data.view(np.float32).reshape(3, 8), h.float().numpy())
        assert f.GetLinearWeight("h").data.ctypes.data == hb.data.ctypes.data  # converted once, kept
        vb = f.GetLinearWeight("v")
        assert vb.dtype == hip.DT_F32 and vb.shape == (5, 1)
        with pytest.raises(hip.ESafeTensorError):
            f.GetLinearWeight("missing")


def test_descriptor_order_zero_sizes_and_subbyte_types(tmp_path):
    # Descriptors out of offset order, a zero-size tensor and F4 / I4 packed
    # types: accepted because the data buffer is tiled exactly.
    hdr = {"b": {"dtype": "F4", "shape": [2, 3], "data_offsets": [4, 7]},
           "z": {"dtype": "F32", "shape": [0], "data_offsets": [7, 7]},
           "a": {"dtype": "I4", "shape": [8], "data_offsets": [0, 4]},
           "__metadata__": {"k": "v"}}
    p = write(tmp_path, "x.safetensors", st_bytes(hdr, bytes(range(7))))
    ora = of.parse_safetensors(p)
    with ck.SafeTensorFiles.Open(p) as f:
        got = [(t.name, t.st_dtype, t.shape, t.data_offset, t.data_size) for t in f.Tensors()]
    assert got == ora["tensors"] and [g[0] for g in got] == ["b", "z", "a"]


BAD_HEADERS = [
    ("not json", None, b"{oops", b""),
    ("array header", None, b"[1,2]", b""),
    ("metadata not object", {"__metadata__": [1]}, None, b""),
    ("metadata value not string", {"__metadata__": {"a": 1}}, None, b""),
    ("descriptor not object", {"t": [1]}, None, b""),
    ("missing offsets", {"t": {"dtype": "F32", "shape": [1]}}, None, b"\0" * 4),
    ("offsets not array", {"t": {"dtype": "F32", "shape": [1], "data_offsets": {"a": 0}}}, None, b"\0" * 4),
    ("three offsets", {"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4, 4]}}, None, b"\0" * 4),
    ("dtype not string", {"t": {"dtype": 3, "shape": [1], "data_offsets": [0, 4]}}, None, b"\0" * 4),
    ("unknown dtype", {"t": {"dtype": "F12", "shape": [1], "data_offsets": [0, 4]}}, None, b"\0" * 4),
    ("UNKNOWN dtype", {"t": {"dtype": "UNKNOWN", "shape": [1], "data_offsets": [0, 4]}}, None, b"\0" * 4),
    ("fractional offset", None, b'{"t":{"dtype":"F32","shape":[1],"data_offsets":[0,4.0]}}', b"\0" * 4),
    ("exponent offset", None, b'{"t":{"dtype":"F32","shape":[1],"data_offsets":[0,4e0]}}', b"\0" * 4),
    ("string offset", {"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, "4"]}}, None, b"\0" * 4),
    ("int64 overflow", None, b'{"t":{"dtype":"F32","shape":[9223372036854775808],"data_offsets":[0,4]}}', b"\0" * 4),
    ("negative offset", {"t": {"dtype": "U8", "shape": [1], "data_offsets": [-1, 0]}}, None, b"\0"),
    ("end before start", {"t": {"dtype": "U8", "shape": [0], "data_offsets": [1, 0]}}, None, b"\0"),
    ("past the data", {"t": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]}}, None, b"\0"),
    ("negative dimension", {"t": {"dtype": "U8", "shape": [-1], "data_offsets": [0, 0]}}, None, b""),
    ("size mismatch", {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}, None, b"\0" * 4),
    ("odd nibbles", {"t": {"dtype": "I4", "shape": [3], "data_offsets": [0, 2]}}, None, b"\0" * 2),
    ("gap", {"t": {"dtype": "U8", "shape": [1], "data_offsets": [1, 2]}}, None, b"\0" * 2),
    ("overlap", {"a": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]},
                 "b": {"dtype": "U8", "shape": [2], "data_offsets": [1, 3]}}, None, b"\0" * 3),
    ("trailing bytes", {"t": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}, None, b"\0" * 2),
    ("duplicate names", None, b'{"t":{"dtype":"U8","shape":[1],"data_offsets":[0,1]},'
                              b'"t":{"dtype":"U8","shape":[1],"data_offsets":[1,2]}}', b"\0" * 2),
    ("invalid UTF-8", None, b'{"\xff":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}', b"\0"),
    ("NaN literal", None, b'{"t":NaN}', b""),
]


@pytest.mark.parametrize("case", BAD_HEADERS, ids=[c[0] for c in BAD_HEADERS])
def test_malformed_safetensors_are_rejected(tmp_path, case):
    _, hdr, raw, data = case
    p = write(tmp_path, "bad.safetensors", st_bytes(hdr, data, raw_header=raw))
    with pytest.raises(of.FormatError):
        of.parse_safetensors(p)
    with pytest.raises(hip.ESafeTensorError):
        ck.SafeTensorFiles.Open(p)


def test_header_length_and_missing_files(tmp_path):
    for blob in (b"\1\0\0\0\0\0\0\0{", struct.pack("<Q", 100) + b"{}", b"\0" * 5,
                 struct.pack("<Q", 100_000_001) + b"{}"):
        p = write(tmp_path, "h.safetensors", blob)
        with pytest.raises(hip.ESafeTensorError):
            ck.SafeTensorFiles.Open(p)
    with pytest.raises(hip.EInOutError):
        ck.SafeTensorFiles.Open(os.path.join(tmp_path, "nope.safetensors"))


def test_shard_index_opens_files_in_first_appearance_order(tmp_path):
    import safetensors.numpy as sn

    sn.save_file({"a": np.ones(3, np.float32), "shared": np.zeros(2, np.float32)},
                 os.path.join(tmp_path, "m-2.safetensors"))
    sn.save_file({"b": np.full(4, 2, np.float32), "shared": np.ones(2, np.float32)},
                 os.path.join(tmp_path, "m-1.safetensors"))
    index = {"metadata": {"total_size": 0}, "weight_map": {"b": "m-1.safetensors", "a": "m-2.safetensors",
                                                           "shared": "m-1.safetensors"}}
    with open(os.path.join(tmp_path, "model.safetensors.index.json"), "w") as f:
        json.dump(index, f)
    with ck.LoadSafeTensorShards(str(tmp_path), "model.safetensors.index.json", "model.safetensors") as f:
        assert [os.path.basename(x.path) for x in f.files] == ["m-1.safetensors", "m-2.safetensors"]
        # GetTensor searches the files in order: "shared" comes from m-1.
        assert f.GetTensor("shared").file == 0 and np.array_equal(f.array("shared"), np.ones(2, np.float32))
        assert f.GetTensor("a").file == 1
    # No index: the single file.
    os.remove(os.path.join(tmp_path, "model.safetensors.index.json"))
    with ck.LoadSafeTensorShards(str(tmp_path), "model.safetensors.index.json", "m-2.safetensors") as f:
        assert len(f.files) == 1 and f.GetTensor("a") is not None
    for bad in ([], {"weight_map": []}, {"weight_map": {}}, {"weight_map": {"a": ""}}, {"weight_map": {"a": 3}}):
        with open(os.path.join(tmp_path, "bad.index.json"), "w") as f:
            json.dump(bad, f)
        with pytest.raises(hip.ESafeTensorError):
            ck.LoadSafeTensorShards(str(tmp_path), "bad.index.json", "")


# ---------------------------------------------------------------------------
# GGUF
# ---------------------------------------------------------------------------
def q_data(st: int, ne) -> bytes:
    enc, be, bb = of.GGUF_QUANT[st]
    return bytes((i * 7 + 3) & 255 for i in range(int(np.prod(ne)) // be * bb))


def sample_gguf(alignment: int = 32) -> tuple[bytes, list]:
    meta = [("general.architecture", STRING, "gemma2"),
            ("general.alignment", U32, alignment),
            ("gemma2.block_count", U32, 42),
            ("gemma2.rope.freq_base", F32, 10000.0),
            ("gemma2.attention.layer_norm_rms_epsilon", F64, 1e-6),
            ("flag", BOOL, 1), ("i8", I8, -5), ("u8", U8, 250), ("i16", I16, -300), ("u16", U16, 60000),
            ("i32", I32, -70000), ("i64", I64, -(1 << 40)), ("u64", U64, 1 << 63),
            ("tokenizer.ggml.tokens", ARRAY, (STRING, ["<s>", "a", "b", "c"])),
            ("tokenizer.ggml.merges", ARRAY, (STRING, ["a b"])),
            ("tokenizer.ggml.scores", ARRAY, (F32, [0.5, 0.25, 0.0, 1.0])),
            ("tokenizer.ggml.token_type", ARRAY, (I32, [1, 1, 1, 3]))]
    tensors = [("token_embd.weight", [512, 3], 12, q_data(12, [512, 3]), None),
               ("blk.0.attn_q.weight", [256, 2], 14, q_data(14, [256, 2]), None),
               ("blk.0.ffn_down.weight", [64, 5], 8, q_data(8, [64, 5]), None),
               ("blk.0.attn_norm.weight", [24], 0, struct.pack("<24f", *range(24)), None),
               ("blk.0.x.weight", [8, 2], 1, bytes(32), None),
               ("blk.0.y.weight", [8, 2], 30, bytes(32), None),
               ("blk.0.q2k.weight", [256], 10, q_data(10, [256]), None),
               ("blk.0.q3k.weight", [256], 11, q_data(11, [256]), None),
               ("blk.0.iq4nl.weight", [64], 20, q_data(20, [64]), None)]
    return gguf_bytes(meta, tensors, alignment=alignment), tensors


@pytest.mark.parametrize("alignment", [32, 64])
def test_gguf_table_matches_construction(tmp_path, alignment):
    blob, tensors = sample_gguf(alignment)
    p = write(tmp_path, "m.gguf", blob)
    h = ck.GGUFHeader.ReadFile(p, metadata=False, include_vocabulary=False)
    ora = of.parse_gguf(p, False, False)
    assert (h.version, h.alignment, h.architecture, h.vocabulary_size) == (3, alignment, "gemma2", 4)
    assert h.data_offset == ora["data_offset"] and h.data_offset % alignment == 0 and h.metadata is None
    assert len(h.tensors) == len(tensors)
    for t, (name, ne, st, data, _), o in zip(h.tensors, tensors, ora["tensors"]):
        assert t.name == name and t.shape == tuple(reversed(ne)) and t.storage_type == st
        assert t.byte_size == len(data) and t.offset % alignment == 0
        assert (t.name, t.shape, t.storage_type, t.encoding, t.offset, t.byte_size) == (
            o["name"], o["shape"], o["storage_type"], o["encoding"], o["offset"], o["byte_size"])
    # Closed forms: Q4_K [3, 512] = 6 blocks of 144 B; Q6_K [2, 256] = 2 x 210 B; Q8_0 [5, 64] = 10 x 34 B.
    assert [t.byte_size for t in h.tensors[:3]] == [6 * 144, 2 * 210, 10 * 34]
    assert [t.encoding for t in h.tensors] == [hip.WE_Q4_K, hip.WE_Q6_K, hip.WE_Q8_0, 0, 0, 0, hip.WE_Q2_K,
                                                hip.WE_Q3_K, 6]


def test_gguf_metadata_values(tmp_path):
    blob, _ = sample_gguf()
    p = write(tmp_path, "m.gguf", blob)
    h = ck.GGUFHeader.ReadFile(p, metadata=True, include_vocabulary=True)
    m = h.metadata
    assert m == of.parse_gguf(p, True, True)["metadata"]
    assert "general.alignment" not in m and m["general.architecture"] == "gemma2"
    assert m["gemma2.block_count"] == 42 and m["flag"] is True and m["u64"] == 1 << 63 and m["i64"] == -(1 << 40)
    assert np.float32(m["gemma2.rope.freq_base"]) == np.float32(10000.0)
    assert m["gemma2.attention.layer_norm_rms_epsilon"] == 1e-6
    assert m["tokenizer.ggml.tokens"] == ["<s>", "a", "b", "c"] and h.vocabulary_size == 4
    # Without the vocabulary: tokens counted and skipped; merges, scores and token types dropped.
    h2 = ck.GGUFHeader.ReadFile(p, metadata=True, include_vocabulary=False)
    assert h2.vocabulary_size == 4
    assert not any(k.startswith("tokenizer.") for k in h2.metadata)
    assert h2.metadata == of.parse_gguf(p, True, False)["metadata"]


def test_gguf_through_tensor_files(tmp_path):
    blob, tensors = sample_gguf()
    p = write(tmp_path, "m.gguf", blob)
    hdr = ck.GGUFHeader.ReadFile(p)
    with ck.SafeTensorFiles.Open(p) as f:
        (info,) = f.files
        assert info.is_gguf and info.architecture == "gemma2" and info.offset == hdr.data_offset
        assert info.header_json == b"" and info.data_size == info.file_size - info.offset
        st = {12: ck.ST_U8, 14: ck.ST_U8, 8: ck.ST_U8, 0: ck.ST_F32, 1: ck.ST_F16, 30: ck.ST_BF16}
        for t, g in zip(f.Tensors(), hdr.tensors):
            assert t.data_offset == hdr.data_offset + g.offset and t.data_size == g.byte_size
            if g.storage_type in st:
                assert t.st_dtype == st[g.storage_type]
        q4 = f.GetLinearWeight("token_embd.weight")
        assert (q4.dtype, q4.encoding, q4.shape, q4.size) == (hip.DT_U8, hip.WE_Q4_K, (3, 512), 1536)
        assert bytes(q4.data[:6 * 144]) == tensors[0][3]
        norm = f.GetLinearWeight("blk.0.attn_norm.weight")
        assert norm.dtype == hip.DT_F32 and np.array_equal(norm.data.view(np.float32), np.arange(24, dtype=np.float32))


def _meta(*extra):
    return [("general.architecture", STRING, "llama"), *extra]


BAD_GGUF = [
    ("magic", dict(magic=0x46554746)),
    ("version 1", dict(version=1)),
    ("version 4", dict(version=4)),
    ("too many tensors", dict(tensor_count=1_000_001)),
    ("truncated metadata", dict(metadata_count=5)),
    ("empty key", dict(metadata=[("", U32, 1)])),
    ("duplicate key", dict(metadata=[("a", U32, 1), ("a", U32, 2)])),
    ("architecture kind", dict(metadata=[("general.architecture", U32, 1)])),
    ("alignment kind", dict(metadata=[("general.alignment", U64, 32)])),
    ("alignment zero", dict(metadata=[("general.alignment", U32, 0)])),
    ("alignment not power of two", dict(metadata=[("general.alignment", U32, 48)])),
    ("alignment too large", dict(metadata=[("general.alignment", U32, 131072)])),
    ("unknown kind", dict(metadata=[("x", 13, 0)])),
    ("vocabulary not strings", dict(metadata=[("tokenizer.ggml.tokens", ARRAY, (U32, [1]))])),
    ("invalid UTF-8 string", dict(metadata=[("x", STRING, b"\xc3\x28")])),
    ("rank 0", dict(tensors=[("t", [], 0, b"", 0)])),
    ("rank 5", dict(tensors=[("t", [1, 1, 1, 1, 1], 0, b"\0" * 4, 0)])),
    ("zero dimension", dict(tensors=[("t", [0], 0, b"", 0)])),
    ("unsupported type Q4_0", dict(tensors=[("t", [32], 2, b"\0" * 18, 0)])),
    ("incomplete Q4_K row", dict(tensors=[("t", [128, 2], 12, b"\0" * 144, 0)])),
    ("unaligned offset", dict(tensors=[("t", [4], 0, b"\0" * 16, 8)])),
    ("overlap", dict(tensors=[("a", [8], 0, b"\0" * 32, 0), ("b", [8], 0, b"\0" * 32, 0)])),
    ("duplicate tensor", dict(tensors=[("a", [8], 0, b"\0" * 32, 0), ("a", [8], 0, b"\0" * 32, 32)])),
]


@pytest.mark.parametrize("case", BAD_GGUF, ids=[c[0] for c in BAD_GGUF])
def test_malformed_gguf_is_rejected(tmp_path, case):
    kw = dict(case[1])
    kw.setdefault("metadata", _meta())
    p = write(tmp_path, "bad.gguf", gguf_bytes(**kw))
    # The reading mode of OpenGGUF (SafeTensors.pas:483): no metadata, vocabulary skipped.
    with pytest.raises(of.FormatError):
        of.parse_gguf(p, False, False)
    with pytest.raises(hip.ESafeTensorError):
        ck.GGUFHeader.ReadFile(p, include_vocabulary=False)
    with pytest.raises(hip.ESafeTensorError):
        ck.SafeTensorFiles.Open(p)


def test_gguf_truncated_payload_and_metadata_modes(tmp_path):
    blob = gguf_bytes(_meta(), [("t", [64], 0, b"\0" * 256, None)])
    p = write(tmp_path, "t.gguf", blob[:-1])
    for fn in (lambda: ck.GGUFHeader.ReadFile(p), lambda: ck.SafeTensorFiles.Open(p)):
        with pytest.raises(hip.ESafeTensorError):
            fn()
    # Nested arrays are skipped when metadata is not collected but refused when it is;
    # a Boolean byte of 2 only matters when it is read.
    nested = _meta(("n", ARRAY, (ARRAY, [(U8, [1, 2])])), ("b", BOOL, 2))
    p = write(tmp_path, "n.gguf", gguf_bytes(nested, [("t", [8], 0, b"\0" * 32, None)]))
    assert ck.GGUFHeader.ReadFile(p).tensors[0].name == "t"
    assert of.parse_gguf(p)["tensors"][0]["name"] == "t"
    with pytest.raises(hip.ESafeTensorError):
        ck.GGUFHeader.ReadFile(p, metadata=True)
    with pytest.raises(of.FormatError):
        of.parse_gguf(p, True)
    # 17 levels of nested arrays exceed the nesting limit even when skipped.
    deep = (U8, [1])
    for _ in range(17):
        deep = (ARRAY, [deep])
    p = write(tmp_path, "d.gguf", gguf_bytes(_meta(("deep", ARRAY, deep))))
    with pytest.raises(hip.ESafeTensorError):
        ck.GGUFHeader.ReadFile(p)
    with pytest.raises(of.FormatError):
        of.parse_gguf(p)
    # Padding between tensors is allowed.
    p = write(tmp_path, "gap.gguf", gguf_bytes(_meta(), [("a", [8], 0, b"\0" * 32, 0), ("b", [8], 0, b"\1" * 32, 96)]))
    h = ck.GGUFHeader.ReadFile(p)
    assert [t.offset for t in h.tensors] == [0, 96]
