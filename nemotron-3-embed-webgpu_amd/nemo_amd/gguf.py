"""GGUF v2/v3 reader (src/gguf/reader.ts:42-161, src/gguf/types.ts).

Same contract as the reference's ``GGUFReader.parse``: little-endian header
(magic "GGUF", version 2 or 3, u64 tensor and metadata counts), typed
metadata values (arrays nest), tensor infos (name, u32 dimension count, u64
dimensions, u32 GGML type, u64 offset), and tensor data at
``ceil(header end / general.alignment)`` (default 32). Only the metadata keys
in ``metadata_keys`` are kept when it is given; every value is still walked so
offsets stay right. Errors carry the reference's messages.

``dims_from_metadata`` maps the ``mistral3.*`` keys of a Nemotron-3-Embed GGUF
to the model shape the runtime takes.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field

GGUF_MAGIC = 0x46554747
F32, F16, Q4_0, Q4_K, Q6_K = 0, 1, 2, 12, 14

# GGUFValueType (src/gguf/types.ts:1-15)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}

# src/gguf/reader.ts:180-210
NEMOTRON3_METADATA_KEYS = frozenset([
    "general.architecture", "general.name", "general.alignment", "general.license", "general.license.name",
    "general.license.link", "mistral3.block_count", "mistral3.context_length", "mistral3.embedding_length",
    "mistral3.feed_forward_length", "mistral3.attention.head_count", "mistral3.attention.head_count_kv",
    "mistral3.attention.causal", "mistral3.attention.key_length", "mistral3.attention.value_length",
    "mistral3.attention.layer_norm_rms_epsilon", "mistral3.attention.temperature_scale", "mistral3.rope.freq_base",
    "mistral3.rope.dimension_count", "mistral3.rope.scaling.type", "mistral3.rope.scaling.factor",
    "mistral3.rope.scaling.original_context_length", "mistral3.rope.scaling.yarn_beta_fast",
    "mistral3.rope.scaling.yarn_beta_slow", "mistral3.rope.scaling.yarn_log_multiplier", "mistral3.pooling_type",
    "tokenizer.ggml.bos_token_id", "tokenizer.ggml.eos_token_id", "tokenizer.ggml.padding_token_id",
])


def tensor_byte_length(type_: int, elements: int) -> int:
    """src/gguf/reader.ts:19-35."""
    if type_ == F32:
        return elements * 4
    if type_ == F16:
        return elements * 2
    if type_ == Q4_0:
        if elements % 32:
            raise ValueError(f"Q4_0 tensor has {elements} elements, not divisible by 32")
        return elements // 32 * 18
    if type_ in (Q4_K, Q6_K):
        name = "Q4_K" if type_ == Q4_K else "Q6_K"
        if elements % 256:
            raise ValueError(f"{name} tensor has {elements} elements, not divisible by 256")
        return elements // 256 * (144 if type_ == Q4_K else 210)
    raise ValueError(f"unsupported GGML tensor type {type_}")


@dataclass
class GGUFModel:
    version: int
    alignment: int
    metadata: dict
    tensors: dict          # name -> {name, dimensions, type, offset, byteOffset, byteLength, elementCount}
    dataOffset: int        # noqa: N815 (reference field name)
    buffer: bytes = field(repr=False)


class GGUFReader:
    """GGUFReader(buffer).parse(metadata_keys=None) -> GGUFModel."""

    def __init__(self, buffer):
        self.buffer = bytes(buffer) if not isinstance(buffer, (bytes, memoryview)) else buffer
        self._view = memoryview(self.buffer)
        self._offset = 0

    def parse(self, metadata_keys=None) -> GGUFModel:
        if self._u32() != GGUF_MAGIC:
            raise ValueError("not a GGUF file")
        version = self._u32()
        if version < 2 or version > 3:
            raise ValueError(f"unsupported GGUF version {version}")
        tensor_count = self._u64("tensor count")
        metadata_count = self._u64("metadata count")
        metadata = {}
        alignment_is_number = True
        for _ in range(metadata_count):
            key = self._string()
            type_ = self._u32()
            retain = metadata_keys is None or key in metadata_keys
            value = self._value(type_, retain)
            if retain:
                metadata[key] = value
                if key == "general.alignment":
                    # 64-bit integers are BigInt in the reference, not numbers
                    alignment_is_number = type_ not in (UINT64, INT64, STRING, ARRAY, BOOL)
        headers = []
        for _ in range(tensor_count):
            name = self._string()
            ndim = self._u32()
            dims = [self._u64("tensor dimension") for _ in range(ndim)]
            type_ = self._u32()
            offset = self._u64("tensor offset")
            headers.append({"name": name, "dimensions": dims, "type": type_, "offset": offset,
                            "elementCount": math.prod(dims)})
        alignment = metadata.get("general.alignment")
        alignment = alignment if alignment is not None and alignment_is_number else 32
        data_offset = int(math.ceil(self._offset / alignment) * alignment)
        tensors = {}
        for t in headers:
            byte_length = tensor_byte_length(t["type"], t["elementCount"])
            byte_offset = data_offset + t["offset"]
            if byte_offset + byte_length > len(self.buffer):
                raise ValueError(f"{t['name']} extends past end of GGUF file")
            tensors[t["name"]] = dict(t, byteOffset=byte_offset, byteLength=byte_length)
        return GGUFModel(version, alignment, metadata, tensors, data_offset, self.buffer)

    # -- primitives ---------------------------------------------------------
    def _take(self, n: int) -> memoryview:
        if self._offset + n > len(self._view):
            raise ValueError("GGUF header extends past end of file")
        v = self._view[self._offset:self._offset + n]
        self._offset += n
        return v

    def _u32(self) -> int:
        return struct.unpack("<I", self._take(4))[0]

    def _u64(self, label: str) -> int:
        v = struct.unpack("<Q", self._take(8))[0]
        if v > 2 ** 53 - 1:
            raise ValueError(f"{label} exceeds JavaScript's safe integer range")
        return v

    def _string(self) -> str:
        n = self._u64("string length")
        return bytes(self._take(n)).decode("utf-8", errors="replace")

    def _value(self, type_: int, retain: bool):
        if type_ in _SCALAR:
            fmt = _SCALAR[type_]
            v = struct.unpack(fmt, self._take(struct.calcsize(fmt)))[0]
            return v if retain else None
        if type_ == BOOL:
            v = self._take(1)[0] != 0
            return v if retain else None
        if type_ == STRING:
            v = self._string()
            return v if retain else None
        if type_ == ARRAY:
            elem = self._u32()
            n = self._u64("metadata array length")
            items = [self._value(elem, retain) for _ in range(n)]
            return items if retain else None
        raise ValueError(f"unsupported GGUF metadata value type {type_}")


def dims_from_metadata(model: GGUFModel):
    """Model shape from the mistral3.* metadata and the token table's size
    (the reference hard-codes the same values, src/webgpu/model.ts:19-28)."""
    from .runtime import reference_dims
    md = model.metadata
    arch = md.get("general.architecture")
    if arch != "mistral3":
        raise ValueError("expected a mistral3 GGUF")
    d = reference_dims()

    def get(key, default):
        v = md.get(f"mistral3.{key}", default)
        return v

    d.hidden = int(get("embedding_length", d.hidden))
    d.layers = int(get("block_count", d.layers))
    d.q_heads = int(get("attention.head_count", d.q_heads))
    d.kv_heads = int(get("attention.head_count_kv", d.kv_heads))
    d.head_dim = int(get("attention.key_length", d.hidden // d.q_heads))
    d.intermediate = int(get("feed_forward_length", d.intermediate))
    d.rms_epsilon = float(get("attention.layer_norm_rms_epsilon", d.rms_epsilon))
    d.rope_theta = float(get("rope.freq_base", d.rope_theta))
    # the merge point is the reference's constant (model.ts:26), not metadata
    d.merge_after_layer = min(d.merge_after_layer, d.layers)
    emb = model.tensors.get("token_embd.weight")
    if emb is not None:
        d.vocab = int(emb["dimensions"][1])
    return d


__all__ = ["GGUFReader", "GGUFModel", "tensor_byte_length", "dims_from_metadata", "NEMOTRON3_METADATA_KEYS"]
