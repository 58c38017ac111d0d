"""The self-contained model pack (src/prepacked/format.ts).

File layout, as the reference writes it: 8-byte magic ``WGPACK02``, u32
little-endian JSON header length, the JSON header, then tensor payloads, each
at a 256-byte aligned offset from the 256-byte aligned data start. Tensors
are stored ``raw`` (GGUF bytes) or ``q4_0-tile32-compact`` (20-byte records
``[f16 d][2 zero bytes][16 nibble bytes]`` ordered tile -> kBlock -> row32).
"""
from __future__ import annotations

import json
import math
import struct
from dataclasses import dataclass
from decimal import Decimal

MAGIC = b"WGPACK02"
PRELUDE_BYTES = 12
DATA_ALIGNMENT = 256
PREPACKED_LAYOUT = "q4_0-tile32-compact-v2"
PREPACKED_TILE_ROWS = 32
PREPACKED_BLOCK_VALUES = 32
PREPACKED_BLOCK_BYTES = 20
PREPACKED_STORAGE_COMPACT = "q4_0-tile32-compact"
PREPACKED_STORAGE_RAW = "raw"
GGML_Q4_0 = 2


def _align(value: int, alignment: int) -> int:
    return math.ceil(value / alignment) * alignment


@dataclass
class PackedTensorBytes:
    name: str
    dimensions: list
    type: int
    storage: str
    bytes: bytes


@dataclass
class PrepackedModel:
    header: dict
    tensors: dict   # name -> header entry plus "byteOffset"
    buffer: bytes
    dataOffset: int  # noqa: N815 (reference field name)


def _js_number_text(x: float) -> str:
    """Number::toString (ECMA-262 6.1.6.1.20) of a double: the shortest
    round-trip digits, fixed notation for 1e-7 <= |x| < 1e21, else
    exponential with an explicit exponent sign."""
    if x != x or x in (float("inf"), float("-inf")):
        return "null"  # JSON.stringify writes non-finite numbers as null
    if x == 0:
        return "0"
    sign = "-" if x < 0 else ""
    digits_tuple = Decimal(repr(abs(x))).normalize().as_tuple()
    digits = "".join(str(d) for d in digits_tuple.digits)
    k = len(digits)
    n = digits_tuple.exponent + k
    if k <= n <= 21:
        text = digits + "0" * (n - k)
    elif 0 < n <= 21:
        text = digits[:n] + "." + digits[n:]
    elif -6 < n <= 0:
        text = "0." + "0" * (-n) + digits
    else:
        e = n - 1
        mant = digits if k == 1 else digits[0] + "." + digits[1:]
        text = f"{mant}e{'+' if e >= 0 else '-'}{abs(e)}"
    return sign + text


def js_json(value) -> str:
    """JSON.stringify(value): compact, UTF-8 text (control characters
    escaped), numbers as JavaScript writes them."""
    if isinstance(value, bool) or value is None:
        return json.dumps(value)
    if isinstance(value, int):
        return str(value)
    if isinstance(value, float):
        return _js_number_text(value)
    if isinstance(value, str):
        return json.dumps(value, ensure_ascii=False)
    if isinstance(value, dict):
        return "{" + ",".join(json.dumps(str(k), ensure_ascii=False) + ":" + js_json(v) for k, v in value.items()) + "}"
    if isinstance(value, (list, tuple)):
        return "[" + ",".join(js_json(v) for v in value) + "]"
    raise TypeError(f"cannot serialize {type(value).__name__}")


def pack_q40_tile32(name: str, parts: list[dict]) -> PackedTensorBytes:
    """src/prepacked/format.ts:65-99. parts: dicts with name, k, n, bytes
    (row-major Q4_0 blocks of 18 bytes)."""
    if not parts:
        raise ValueError(f"cannot pack {name} without tensor parts")
    k = parts[0]["k"]
    if k % PREPACKED_BLOCK_VALUES:
        raise ValueError(f"{name} K={k} is not divisible by 32")
    for part in parts:
        if part["k"] != k:
            raise ValueError(f"{name} has mismatched K dimensions")
        expected = part["n"] * (k // 32) * 18
        if len(part["bytes"]) != expected:
            raise ValueError(f"{part['name']} has {len(part['bytes'])} bytes; expected {expected}")
    n = sum(p["n"] for p in parts)
    k_blocks = k // PREPACKED_BLOCK_VALUES
    n_tiles = math.ceil(n / PREPACKED_TILE_ROWS)
    out = bytearray(n_tiles * k_blocks * PREPACKED_TILE_ROWS * PREPACKED_BLOCK_BYTES)
    row_parts = [(p, r) for p in parts for r in range(p["n"])]
    for tile in range(n_tiles):
        for kb in range(k_blocks):
            for local in range(PREPACKED_TILE_ROWS):
                row = tile * PREPACKED_TILE_ROWS + local
                if row >= n:
                    continue
                part, prow = row_parts[row]
                src = (prow * k_blocks + kb) * 18
                dst = ((tile * k_blocks + kb) * PREPACKED_TILE_ROWS + local) * PREPACKED_BLOCK_BYTES
                b = part["bytes"]
                out[dst] = b[src]
                out[dst + 1] = b[src + 1]
                out[dst + 4:dst + 20] = b[src + 2:src + 18]
    return PackedTensorBytes(name, [k, n], GGML_Q4_0, PREPACKED_STORAGE_COMPACT, bytes(out))


def raw_tensor(name: str, dimensions, type_: int, data: bytes) -> PackedTensorBytes:
    """src/prepacked/format.ts:101-103."""
    return PackedTensorBytes(name, list(dimensions), type_, PREPACKED_STORAGE_RAW, bytes(data))


def build_prepacked_file(source_sha256: str, source_bytes: int, metadata: dict,
                         tensors: list[PackedTensorBytes]) -> bytes:
    """src/prepacked/format.ts:105-144."""
    relative = 0
    entries = []
    for t in tensors:
        relative = _align(relative, DATA_ALIGNMENT)
        entries.append({"name": t.name, "dimensions": list(t.dimensions), "type": t.type, "storage": t.storage,
                        "offset": relative, "byteLength": len(t.bytes)})
        relative += len(t.bytes)
    header = {"version": 2, "sourceSha256": source_sha256, "sourceBytes": source_bytes, "layout": PREPACKED_LAYOUT,
              "tileRows": PREPACKED_TILE_ROWS, "blockValues": PREPACKED_BLOCK_VALUES,
              "blockBytes": PREPACKED_BLOCK_BYTES, "metadata": metadata, "tensors": entries}
    header_bytes = js_json(header).encode()
    data_offset = _align(PRELUDE_BYTES + len(header_bytes), DATA_ALIGNMENT)
    out = bytearray(data_offset + relative)
    out[0:8] = MAGIC
    out[8:12] = struct.pack("<I", len(header_bytes))
    out[PRELUDE_BYTES:PRELUDE_BYTES + len(header_bytes)] = header_bytes
    for t, e in zip(tensors, entries):
        out[data_offset + e["offset"]:data_offset + e["offset"] + len(t.bytes)] = t.bytes
    return bytes(out)


def parse_prepacked_model(buffer: bytes) -> PrepackedModel:
    """src/prepacked/format.ts:146-169 (same checks and messages)."""
    buffer = bytes(buffer)
    if len(buffer) < PRELUDE_BYTES:
        raise ValueError("prepacked model is shorter than its prelude")
    magic = buffer[:8]
    if magic != MAGIC:
        raise ValueError(f"invalid prepacked model magic {json.dumps(magic.decode('latin-1'))}")
    (header_length,) = struct.unpack_from("<I", buffer, 8)
    if PRELUDE_BYTES + header_length > len(buffer):
        raise ValueError("prepacked model header extends past end of file")
    header = json.loads(buffer[PRELUDE_BYTES:PRELUDE_BYTES + header_length].decode())
    if (header.get("version") != 2 or header.get("layout") != PREPACKED_LAYOUT or header.get("tileRows") != 32
            or header.get("blockValues") != 32 or header.get("blockBytes") != 20):
        raise ValueError(f"unsupported prepacked layout {header.get('layout')}")
    data_offset = _align(PRELUDE_BYTES + header_length, DATA_ALIGNMENT)
    tensors: dict = {}
    for t in header["tensors"]:
        byte_offset = data_offset + t["offset"]
        if byte_offset + t["byteLength"] > len(buffer):
            raise ValueError(f"{t['name']} extends past end of prepacked file")
        if t["name"] in tensors:
            raise ValueError(f"duplicate prepacked tensor {t['name']}")
        if t["storage"] == PREPACKED_STORAGE_COMPACT and (t["type"] != GGML_Q4_0 or len(t["dimensions"]) != 2):
            raise ValueError(f"{t['name']} has invalid compact Q4_0 metadata")
        if t["storage"] not in (PREPACKED_STORAGE_COMPACT, PREPACKED_STORAGE_RAW):
            raise ValueError(f"{t['name']} has unsupported storage {t['storage']}")
        tensors[t["name"]] = dict(t, byteOffset=byte_offset)
    return PrepackedModel(header, tensors, buffer, data_offset)
