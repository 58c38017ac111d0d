"""Writes GGUF v2/v3 files for the tests (test input generation, not a
checker): header, typed metadata, tensor infos, tensor data at the
alignment boundary, each tensor padded to the alignment."""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", U64: "<Q", I64: "<q", F64: "<d"}


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(type_: int, value) -> bytes:
    if type_ in _FMT:
        return struct.pack(_FMT[type_], value)
    if type_ == BOOL:
        return struct.pack("<B", 1 if value else 0)
    if type_ == STRING:
        return _string(value)
    if type_ == ARRAY:
        elem, items = value
        return struct.pack("<IQ", elem, len(items)) + b"".join(_value(elem, v) for v in items)
    raise ValueError(type_)


def write_gguf(metadata, tensors, alignment: int = 32, version: int = 3) -> bytes:
    """metadata: [(key, value_type, value)] (ARRAY values are (elem_type,
    items)); tensors: [(name, dims, ggml_type, bytes)] with dims ne0 first.
    `alignment` must match any general.alignment in `metadata` (32 when
    absent); the last tensor is not padded."""
    out = bytearray(struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(metadata)))
    for key, type_, value in metadata:
        out += _string(key) + struct.pack("<I", type_) + _value(type_, value)
    offset = 0
    offsets = []
    for name, dims, type_, data in tensors:
        offsets.append(offset)
        out += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", type_, offset)
        offset += (len(data) + alignment - 1) // alignment * alignment
    out += bytes((-len(out)) % alignment)
    for i, (name, dims, type_, data) in enumerate(tensors):
        out += data
        if i + 1 < len(tensors):
            out += bytes((-len(data)) % alignment)
    return bytes(out)


def nemotron_metadata(dims, alignment=None):
    """The mistral3.* keys of a Nemotron-3-Embed GGUF for a model of `dims`."""
    md = [("general.architecture", STRING, "mistral3"), ("general.name", STRING, "synthetic"),
          ("mistral3.block_count", U32, dims.layers), ("mistral3.embedding_length", U32, dims.hidden),
          ("mistral3.feed_forward_length", U32, dims.intermediate),
          ("mistral3.attention.head_count", U32, dims.q_heads),
          ("mistral3.attention.head_count_kv", U32, dims.kv_heads),
          ("mistral3.attention.key_length", U32, dims.head_dim), ("mistral3.attention.value_length", U32, dims.head_dim),
          ("mistral3.attention.layer_norm_rms_epsilon", F32, 1e-5), ("mistral3.rope.freq_base", F32, 1e6),
          ("mistral3.attention.causal", BOOL, False), ("tokenizer.ggml.bos_token_id", U32, 1)]
    if alignment is not None:
        md.append(("general.alignment", U32, alignment))
    return md
