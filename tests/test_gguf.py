"""GGUF reader: the directory the HBM loader uploads from.

Cases follow the reference's reader tests (tests/test_gguf.py:28-87,
tests/test_gguf_errors.py:150-300): a valid file parses with the expected
header, directory and absolute offsets; every malformed field is refused with
a GGUFError naming it.  Files are written byte by byte by tests/gguf_writer.py.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

from pyrite_amd.gguf import GGUFError, GGUFReader
from tests import gguf_writer as gw


def parse(tmp_path, data: bytes, name: str = "candidate.gguf") -> GGUFReader:
    path = tmp_path / name
    path.write_bytes(data)
    r = GGUFReader(path)
    r.header(), r.metadata(), r.tensor_index()
    return r


def good() -> gw.Writer:
    w = gw.Writer()
    w.kv("qwen3.embedding_length", gw.U32, 8)
    w.tensor("blk.0.attn_norm.weight", (8,), 0, struct.pack("<8f", *range(8)))
    return w


def test_valid_file_header_and_directory(tmp_path):
    r = parse(tmp_path, good().bytes())
    h = r.header()
    assert (h.version, h.tensor_count, h.metadata_count, h.alignment) == (3, 1, 3, 32)
    assert h.data_offset % 32 == 0 and h.data_offset == r.tensor_data_offset
    t = r.tensor("blk.0.attn_norm.weight")
    assert (t.dims, t.ggml_type, t.offset, t.size, t.element_count) == ((8,), 0, h.data_offset, 32, 8)
    assert r.read_tensor(t) == struct.pack("<8f", *range(8))
    assert r.get("general.architecture") == "qwen3" and r.get("qwen3.embedding_length") == 8
    assert r.tensor_names() == ("blk.0.attn_norm.weight",) and r.has_tensor("blk.0.attn_norm.weight")
    assert r.size_bytes == (tmp_path / "candidate.gguf").stat().st_size
    with pytest.raises(KeyError, match="no tensor named"):
        r.tensor("nope")


def test_tiny_file_known_layout(tmp_path):
    """The reference's hand-built file (tests/test_gguf.py:10-34): 24 + 33 header bytes, data at byte 64."""
    desc = struct.pack("<Q", 1) + b"x" + struct.pack("<I", 1) + struct.pack("<Q", 2) + struct.pack("<IQ", 0, 0)
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 0)
    pad = bytes((32 - (len(head) + len(desc)) % 32) % 32)
    r = parse(tmp_path, head + desc + pad + struct.pack("<2f", 1.0, 2.0))
    (t,) = r.tensor_index()
    assert (t.name, t.dims, t.size, t.offset) == ("x", (2,), 8, 64)
    assert struct.unpack("<2f", r.read_tensor(t)) == (1.0, 2.0)


def test_metadata_value_types_and_arrays(tmp_path):
    w = gw.Writer()
    vals = {"u8": (gw.U8, 250), "i8": (gw.I8, -5), "u16": (gw.U16, 65000), "i16": (gw.I16, -30000),
            "u32": (gw.U32, 4_000_000_000), "i32": (gw.I32, -2_000_000_000), "f32": (gw.F32, 1.5),
            "bool": (gw.BOOL, 1), "u64": (gw.U64, 1 << 60), "i64": (gw.I64, -(1 << 60)), "f64": (gw.F64, 0.1),
            "str": (gw.STRING, "héllo")}
    for k, (t, v) in vals.items():
        w.kv(k, t, v)
    scores = np.arange(151936, dtype=np.float32) * np.float32(-0.5)
    w.kv("tokenizer.ggml.scores", gw.ARRAY, scores.tolist(), gw.F32)
    w.kv("tokenizer.ggml.tokens", gw.ARRAY, ["a", "bb", ""], gw.STRING)
    w.kv("flags", gw.ARRAY, [1, 0, 1], gw.BOOL)
    w.kv("nested", gw.ARRAY, [], gw.U32)
    md = parse(tmp_path, w.bytes()).metadata()
    for k, (t, v) in vals.items():
        assert md[k] == (bool(v) if t == gw.BOOL else v), k
    assert isinstance(md["bool"], bool) and md["f64"] == 0.1
    assert np.array_equal(np.asarray(md["tokenizer.ggml.scores"], dtype=np.float32), scores)
    assert md["tokenizer.ggml.tokens"] == ("a", "bb", "")
    assert md["flags"] == (True, False, True) and md["nested"] == ()


def test_quantized_size_is_validated_per_row(tmp_path):
    # the total is one Q4_K block, but each of the two 128-element rows is invalid
    w = gw.Writer()
    w.tensor("bad", (128, 2), 12, bytes(144))
    with pytest.raises(ValueError, match="row requires element count"):
        parse(tmp_path, w.bytes())
    w = gw.Writer()
    w.tensor("good", (256, 2), 12, bytes(288))
    assert parse(tmp_path, w.bytes(), "ok.gguf").tensor("good").size == 288


def test_sizes_of_stacked_expert_tensors(tmp_path):
    """(2048, 768, 128) Q4_K and (768, 2048, 128) Q6_K stacks (pyrite/qwen3_moe.py:432-443), at 2 experts."""
    w = gw.Writer()
    w.tensor("blk.0.ffn_gate_exps.weight", (2048, 768, 2), 12, bytes(2 * 884_736))
    w.tensor("blk.0.ffn_down_exps.weight", (768, 2048, 2), 14, bytes(2 * 1_290_240))
    r = parse(tmp_path, w.bytes())
    assert r.tensor("blk.0.ffn_gate_exps.weight").size == 2 * 884_736
    assert r.tensor("blk.0.ffn_down_exps.weight").size == 2 * 1_290_240


def test_nonmonotonic_offsets_are_accepted(tmp_path):
    w = gw.Writer()
    w.tensor("first", (1,), 0, struct.pack("<f", 1.0), offset=32)
    w.tensor("second", (1,), 0, struct.pack("<f", 2.0), offset=0)
    r = parse(tmp_path, w.bytes())
    d = r.header().data_offset
    assert [t.offset for t in r.tensor_index()] == [d + 32, d]
    assert struct.unpack("<f", r.read_tensor(r.tensor("first"))) == (1.0,)


def test_overlapping_payloads_are_rejected(tmp_path):
    w = gw.Writer()
    w.tensor("a", (16,), 0, bytes(64), offset=0)
    w.tensor("b", (16,), 0, bytes(64), offset=32)
    with pytest.raises(GGUFError, match="'a' and 'b' overlap"):
        parse(tmp_path, w.bytes())


def test_zero_dimension_tensor_is_a_scalar(tmp_path):
    w = gw.Writer()
    w.tensor("output_norm.weight", (), 0, struct.pack("<f", 1.5))
    r = parse(tmp_path, w.bytes())
    t = r.tensor_index()[0]
    assert t.dims == () and t.element_count == 1 and r.read_tensor(t) == struct.pack("<f", 1.5)


def test_alignment_metadata_is_honoured(tmp_path):
    w = gw.Writer(alignment=64)
    w.tensor("a", (8,), 0, bytes(32))
    w.tensor("b", (8,), 0, bytes(32))
    r = parse(tmp_path, w.bytes())
    assert r.header().alignment == 64 and r.header().data_offset % 64 == 0
    assert r.tensor("b").offset - r.tensor("a").offset == 64


def test_version_two_is_accepted(tmp_path):
    assert parse(tmp_path, good().bytes(version=2)).header().version == 2


@pytest.mark.parametrize("case, match", [
    ("magic", "magic"), ("empty", "too short"), ("short", "file ends at"), ("v1", "version 1 "),
    ("v4", "version 4 "), ("neg_count", "safety limits"), ("many_tensors", "safety limits"),
    ("many_meta", "safety limits"), ("truncated", "past the end of the file"), ("huge_string", r"declares \d+ bytes; only \d+ are left"),
    ("string_past_end", r"declares 1099511627776 bytes; only"), ("long_name", "GGML_MAX_NAME"), ("dup_key", "twice in the metadata"),
    ("dup_tensor", "twice in the directory"), ("dims", "at most 4"), ("zero_dim", "empty dimension"),
    ("type", "unsupported GGML tensor type"), ("offset", "past the end of the data section"),
    ("unaligned", "not a multiple"), ("alignment", "power of two"), ("bool", "neither 0 nor 1"),
    ("array_count", "bytes are left"), ("value_type", "does not define"),
])
def test_malformed_files_are_rejected(tmp_path, case, match):
    w = good()
    kw = {}
    data = None
    if case == "magic":
        kw = {"magic": b"GGML"}
    elif case == "empty":
        data = b""
    elif case == "short":
        data = good().bytes()[:12]
    elif case == "v1":
        kw = {"version": 1}
    elif case == "v4":
        kw = {"version": 4}
    elif case == "neg_count":
        kw = {"n_tensors": -1}
    elif case == "many_tensors":
        kw = {"n_tensors": GGUFReader.MAX_TENSORS + 1}
    elif case == "many_meta":
        kw = {"n_meta": GGUFReader.MAX_METADATA + 1}
    elif case == "truncated":
        kw = {"truncate": 16}
    elif case == "huge_string":
        w.raw_kv("general.name", gw.STRING, struct.pack("<Q", GGUFReader.MAX_STRING_BYTES + 1) + b"x")
    elif case == "string_past_end":
        w.raw_kv("general.name", gw.STRING, struct.pack("<Q", 1 << 40))
    elif case == "long_name":
        w = gw.Writer()
        w.tensor("t", (8,), 0, bytes(32), name_len=GGUFReader.MAX_NAME + 1)
        w.kv("pad", gw.STRING, "p" * 200)  # enough bytes after the name for the long read
    elif case == "dup_key":
        w.kv("general.alignment", gw.U32, 64)
    elif case == "dup_tensor":
        w.tensor("blk.0.attn_norm.weight", (8,), 0, bytes(32))
    elif case == "dims":
        w = gw.Writer()
        w.tensor("t", (8,), 0, bytes(32), n_dims=GGUFReader.MAX_DIMS + 1)
    elif case == "zero_dim":
        w = gw.Writer()
        w.tensor("t", (8, 0), 0, b"")
    elif case == "type":
        w = gw.Writer()
        w.tensor("t", (8,), 4242, bytes(32))
    elif case == "offset":
        w = gw.Writer()
        w.tensor("t", (8,), 0, b"", offset=1 << 40)
        w.payloads = [(0, bytes(32))]
    elif case == "unaligned":
        w = gw.Writer()
        w.tensor("t", (1,), 0, bytes(4), offset=4)
    elif case == "alignment":
        w = gw.Writer(alignment=None)
        w.kv("general.alignment", gw.U32, 48)
        w.tensor("t", (8,), 0, bytes(32))
    elif case == "bool":
        w.raw_kv("flag", gw.BOOL, b"\x02")
    elif case == "array_count":
        w.raw_kv("arr", gw.ARRAY, struct.pack("<IQ", gw.U8, 1 << 20))  # under the count limit, past the end
    elif case == "value_type":
        w.raw_kv("weird", 13, b"\x00" * 8)
    if data is None:
        data = w.bytes(**kw)
    with pytest.raises(GGUFError, match=match):
        parse(tmp_path, data)


def test_reader_is_lazy_and_checks_missing_files(tmp_path):
    r = GGUFReader(tmp_path / "absent.gguf")  # nothing read yet
    with pytest.raises(FileNotFoundError):
        r.header()


def test_resident_tensors_need_a_gpu_device(tmp_path):
    """The HBM loader refuses a host device before reading anything (no CPU fallback)."""
    from pyrite_amd.resident import ResidentTensors
    r = parse(tmp_path, good().bytes())
    with pytest.raises(ValueError, match="CUDA"):
        ResidentTensors(r, device="cpu")


def test_string_cap_is_enforced(tmp_path):
    """A string longer than MAX_STRING_BYTES is refused even when the file holds it."""
    w = good()
    n = GGUFReader.MAX_STRING_BYTES + 1
    w.raw_kv("general.name", gw.STRING, struct.pack("<Q", n) + b"x" * n)
    with pytest.raises(GGUFError, match="cap on strings"):
        parse(tmp_path, w.bytes())
