"""Offline prepack: a Nemotron-3-Embed GGUF -> a self-contained .wgpack whose
projections are Q4_0 in the tile32-compact layout (scripts/prepack-model.ts).

    python -m nemo_amd.prepack model.gguf model.wgpack

Same steps and checks as the reference's script: the GGUF must be mistral3;
per layer attn_q/attn_k/attn_v are requantized to Q4_0 and packed as
attn_qkv, attn_output alone, ffn_gate/ffn_up as ffn_gate_up, ffn_down alone
(:39-45); any other matrix except token_embd.weight is an error (:47-48);
every remaining tensor is stored raw (:50-57); the header records the source's
SHA-256 and size and the NEMOTRON3 metadata (:58-59). The requantization
(requantizeMatrixToQ40, src/gguf/quantization.ts:101-131) runs on the GPU
through libnemo (nemo_requantize_q40), bit-exact with the JavaScript. The
layer count comes from mistral3.block_count (the reference's model has 16).
"""
from __future__ import annotations

import hashlib
import json
import sys

from . import gguf
from .prepacked import build_prepacked_file, pack_q40_tile32, raw_tensor

_QUANTIZED = (gguf.Q4_0, gguf.Q4_K, gguf.Q6_K)


def _metadata_value(value):
    """scripts/prepack-model.ts:19-27: integers must be safe in JavaScript."""
    def convert(item):
        if isinstance(item, int) and not isinstance(item, bool) and abs(item) > 2 ** 53 - 1:
            raise ValueError(f"metadata bigint {item} is not safely representable")
        return item
    return [convert(v) for v in value] if isinstance(value, list) else convert(value)


def prepack_gguf(source: bytes, requantize=None) -> bytes:
    """GGUF bytes -> .wgpack bytes. `requantize(type, bytes, k, n)` defaults to
    the GPU requantization of libnemo."""
    if requantize is None:
        from .runtime import requantize_q40 as requantize
    model = gguf.GGUFReader(source).parse(gguf.NEMOTRON3_METADATA_KEYS)
    if model.metadata.get("general.architecture") != "mistral3":
        raise ValueError("expected a mistral3 GGUF")
    sha = hashlib.sha256(source).hexdigest()
    consumed: set[str] = set()
    view = memoryview(source)

    def part(name: str) -> dict:
        t = model.tensors.get(name)
        if t is None or t["type"] not in _QUANTIZED or len(t["dimensions"]) != 2:
            raise ValueError(f"{name} is not a supported quantized matrix")
        consumed.add(name)
        k, n = t["dimensions"]
        data = view[t["byteOffset"]:t["byteOffset"] + t["byteLength"]]
        return {"name": name, "k": k, "n": n, "bytes": requantize(t["type"], data, k, n)}

    layers = int(model.metadata.get("mistral3.block_count", 16))
    packed = []
    for layer in range(layers):
        p = f"blk.{layer}"
        packed.append(pack_q40_tile32(f"{p}.attn_qkv.weight",
                                      [part(f"{p}.attn_q.weight"), part(f"{p}.attn_k.weight"), part(f"{p}.attn_v.weight")]))
        packed.append(pack_q40_tile32(f"{p}.attn_output.weight", [part(f"{p}.attn_output.weight")]))
        packed.append(pack_q40_tile32(f"{p}.ffn_gate_up.weight", [part(f"{p}.ffn_gate.weight"), part(f"{p}.ffn_up.weight")]))
        packed.append(pack_q40_tile32(f"{p}.ffn_down.weight", [part(f"{p}.ffn_down.weight")]))
    unexpected = [t["name"] for t in model.tensors.values()
                  if len(t["dimensions"]) == 2 and t["name"] != "token_embd.weight" and t["name"] not in consumed]
    if unexpected:
        raise ValueError(f"unpacked matrices: {', '.join(unexpected)}")
    raw = [raw_tensor(t["name"], t["dimensions"], t["type"], view[t["byteOffset"]:t["byteOffset"] + t["byteLength"]])
           for t in model.tensors.values() if t["name"] not in consumed]
    metadata = {key: _metadata_value(value) for key, value in model.metadata.items()}
    return build_prepacked_file(sha, len(source), metadata, raw + packed)


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    source_path = argv[0] if argv else "models/nemotron-3-embed-1b-q4_k_m.gguf"
    output_path = argv[1] if len(argv) > 1 else "models/nemotron-3-embed-1b-q4-webgpu.wgpack"
    with open(source_path, "rb") as f:
        source = f.read()
    out = prepack_gguf(source)
    with open(output_path, "wb") as f:
        f.write(out)
    from .prepacked import parse_prepacked_model
    pack = parse_prepacked_model(out)
    n_raw = sum(1 for t in pack.tensors.values() if t["storage"] == "raw")
    print(json.dumps({"sourcePath": source_path, "outputPath": output_path,
                      "sourceSha256": pack.header["sourceSha256"], "rawTensors": n_raw,
                      "packedTensors": len(pack.tensors) - n_raw, "tensors": len(pack.tensors), "bytes": len(out)},
                     indent=2))
    return 0


if __name__ == "__main__":
    sys.exit(main())
