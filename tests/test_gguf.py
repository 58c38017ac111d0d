"""GGUF reader (nemo_amd/gguf.py) against the GGUF layout the reference reads
(src/gguf/reader.ts:42-161): typed metadata, tensor table, data alignment,
the reference's error messages, and model dims from mistral3 metadata."""
import math
import struct

import numpy as np
import pytest

import synth
from gguf_writer import (ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64, nemotron_metadata,
                         write_gguf)
from nemo_amd import gguf


def _sample(alignment=None):
    md = [("a.u8", U8, 200), ("a.i8", I8, -5), ("a.u16", U16, 65000), ("a.i16", I16, -300), ("a.u32", U32, 4000000000),
          ("a.i32", I32, -7), ("a.f32", F32, 1.5), ("a.bool", BOOL, True), ("a.str", STRING, "héllo"),
          ("a.arr", ARRAY, (U32, [1, 2, 3])), ("a.strs", ARRAY, (STRING, ["x", "yz"])), ("a.u64", U64, 2 ** 40),
          ("a.i64", I64, -2 ** 40), ("a.f64", F64, 0.25), ("a.nested", ARRAY, (ARRAY, [(I8, [1, -1]), (I8, [])]))]
    if alignment:
        md.append(("general.alignment", U32, alignment))
    q4k = synth.random_q4k(1, 2).tobytes()
    tensors = [("w.q4k", [256, 2], 12, q4k), ("w.f32", [3], 0, np.arange(3, dtype=np.float32).tobytes()),
               ("w.q6k", [256, 1], 14, synth.random_q6k(2, 1).tobytes()),
               ("w.q40", [64, 1], 2, synth.random_q40(3, 2).tobytes()), ("w.f16", [5], 1, bytes(10))]
    return md, tensors


@pytest.mark.parametrize("alignment", [None, 64, 256])
def test_round_trip_metadata_tensors_and_alignment(alignment):
    md, tensors = _sample(alignment)
    data = write_gguf(md, tensors, alignment=alignment or 32)
    m = gguf.GGUFReader(data).parse()
    assert m.version == 3 and m.alignment == (alignment or 32)
    assert m.dataOffset % (alignment or 32) == 0
    for key, type_, value in md:
        got = m.metadata[key]
        if type_ == F32:
            assert got == pytest.approx(value)
        elif type_ == ARRAY:
            elem, items = value
            assert got == ([list(v[1]) for v in items] if elem == ARRAY else list(items))
        else:
            assert got == value
    for name, dims, type_, raw in tensors:
        t = m.tensors[name]
        assert t["dimensions"] == dims and t["type"] == type_ and t["elementCount"] == math.prod(dims)
        assert t["byteLength"] == len(raw)
        assert data[t["byteOffset"]:t["byteOffset"] + t["byteLength"]] == raw


def test_metadata_filter_keeps_offsets():
    md, tensors = _sample()
    data = write_gguf(md, tensors)
    m = gguf.GGUFReader(data).parse(metadata_keys={"a.str", "a.f64"})
    assert set(m.metadata) == {"a.str", "a.f64"}
    assert m.tensors["w.f32"]["byteOffset"] == gguf.GGUFReader(data).parse().tensors["w.f32"]["byteOffset"]


def test_header_layout_by_hand():
    """A file assembled field by field: magic, version 2, counts, one u32
    alignment key of 64, one F32 tensor of 4 values at offset 0."""
    key = b"general.alignment"
    head = struct.pack("<IIQQ", 0x46554747, 2, 1, 1) + struct.pack("<Q", len(key)) + key + struct.pack("<II", 4, 64)
    head += struct.pack("<Q", 1) + b"t" + struct.pack("<IQ", 1, 4) + struct.pack("<IQ", 0, 0)
    data_offset = (len(head) + 63) // 64 * 64
    blob = head + bytes(data_offset - len(head)) + struct.pack("<4f", 1, 2, 3, 4)
    m = gguf.GGUFReader(blob).parse()
    assert (m.version, m.alignment, m.dataOffset) == (2, 64, data_offset)
    assert m.tensors["t"]["byteOffset"] == data_offset and m.tensors["t"]["byteLength"] == 16


def test_u64_alignment_is_not_a_number():
    """The reference only honours a general.alignment that JavaScript reads as
    a number; a 64-bit value is a BigInt there, so the default 32 applies."""
    md = [("general.alignment", U64, 64)]
    data = write_gguf(md, [("t", [8], 0, bytes(32))], alignment=32)
    assert gguf.GGUFReader(data).parse().alignment == 32


@pytest.mark.parametrize("mutate,message", [
    (lambda b: b"XXXX" + b[4:], "not a GGUF file"),
    (lambda b: b[:4] + struct.pack("<I", 1) + b[8:], "unsupported GGUF version 1"),
    (lambda b: b[:4] + struct.pack("<I", 4) + b[8:], "unsupported GGUF version 4"),
    (lambda b: b[:-1], "w.f16 extends past end of GGUF file"),
])
def test_errors_match_reference(mutate, message):
    md, tensors = _sample()
    tensors = tensors[:-1] + [("w.f16", [5], 1, bytes(10))]
    data = write_gguf(md, tensors)
    with pytest.raises(ValueError, match=message):
        gguf.GGUFReader(mutate(data)).parse()


def test_tensor_byte_length_rules():
    # src/gguf/reader.ts:19-35
    assert gguf.tensor_byte_length(12, 512) == 288 and gguf.tensor_byte_length(14, 256) == 210
    assert gguf.tensor_byte_length(2, 64) == 36 and gguf.tensor_byte_length(1, 3) == 6
    with pytest.raises(ValueError, match="Q4_K tensor has 300 elements, not divisible by 256"):
        gguf.tensor_byte_length(12, 300)
    with pytest.raises(ValueError, match="Q4_0 tensor has 33 elements, not divisible by 32"):
        gguf.tensor_byte_length(2, 33)
    with pytest.raises(ValueError, match="unsupported GGML tensor type 8"):
        gguf.tensor_byte_length(8, 32)


def test_unsupported_metadata_type():
    blob = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13)
    with pytest.raises(ValueError, match="unsupported GGUF metadata value type 13"):
        gguf.GGUFReader(blob).parse()


def test_dims_from_metadata():
    from nemo_amd import runtime as rt
    d = rt.make_dims(hidden=512, q_heads=8, kv_heads=2, head_dim=64, intermediate=1024, layers=3, vocab=77)
    data = write_gguf(nemotron_metadata(d), [("token_embd.weight", [512, 77], 1, bytes(512 * 77 * 2))])
    got = gguf.dims_from_metadata(gguf.GGUFReader(data).parse(gguf.NEMOTRON3_METADATA_KEYS))
    assert (got.hidden, got.q_heads, got.kv_heads, got.head_dim, got.intermediate, got.layers, got.vocab) == (
        512, 8, 2, 64, 1024, 3, 77)
    assert got.rms_epsilon == pytest.approx(1e-5) and got.rope_theta == 1e6
    bad = write_gguf([("general.architecture", STRING, "llama")], [])
    with pytest.raises(ValueError, match="expected a mistral3 GGUF"):
        gguf.dims_from_metadata(gguf.GGUFReader(bad).parse())
