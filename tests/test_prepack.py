"""The prepack tool (nemo_amd/prepack.py, scripts/prepack-model.ts) on the
CPU with the oracle's requantizeMatrixToQ40 standing in for the GPU one:
tensor set, fusion order, raw tensors, header fields and the reference's
errors. The GPU requantization itself is compared with the oracle in
tests/test_gpu_requant.py."""
import hashlib

import numpy as np
import pytest

import oracle
import synth
from gguf_writer import STRING, U32, nemotron_metadata, write_gguf
from nemo_amd import prepack, prepacked
from nemo_amd import runtime as rt


def _requant(type_, data, k, n):
    return oracle.requantize_to_q40(bytes(data), type_, k, n)


def _model_gguf(dims, seed=3):
    t = synth.model_tensors(dims, seed=seed, embedding_type=14, fused=False)
    return t, write_gguf(nemotron_metadata(dims), [(n, d, ty, b) for n, (ty, d, b) in t.items()])


def _dims():
    return rt.make_dims(hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=256, layers=2, vocab=64,
                        merge_after_layer=2)


def test_prepack_layout_and_header():
    dims = _dims()
    tensors, blob = _model_gguf(dims)
    pack = prepacked.parse_prepacked_model(prepack.prepack_gguf(blob, requantize=_requant))
    assert pack.header["sourceSha256"] == hashlib.sha256(blob).hexdigest()
    assert pack.header["sourceBytes"] == len(blob)
    assert pack.header["metadata"]["general.architecture"] == "mistral3"
    assert pack.header["metadata"]["mistral3.block_count"] == 2
    compact = [t["name"] for t in pack.tensors.values() if t["storage"] == "q4_0-tile32-compact"]
    assert compact == [f"blk.{l}.{n}.weight" for l in range(2)
                       for n in ("attn_qkv", "attn_output", "ffn_gate_up", "ffn_down")]
    raw = {t["name"] for t in pack.tensors.values() if t["storage"] == "raw"}
    assert raw == {"token_embd.weight", "output_norm.weight"} | {f"blk.{l}.{n}.weight" for l in range(2)
                                                                  for n in ("attn_norm", "ffn_norm")}
    # attn_qkv = rows [q; k; v] requantized to Q4_0, then tile32-packed
    l0 = "blk.0."
    parts = [tensors[l0 + n] for n in ("attn_q.weight", "attn_k.weight", "attn_v.weight")]
    q40 = b"".join(_requant(t, b, d[0], d[1]) for t, d, b in parts)
    n_rows = sum(d[1] for _, d, _ in parts)
    entry = pack.tensors[l0 + "attn_qkv.weight"]
    assert entry["dimensions"] == [256, n_rows]
    got = pack.buffer[entry["byteOffset"]:entry["byteOffset"] + entry["byteLength"]]
    assert got == oracle.pack_q40_tile32(q40, 256, n_rows)
    emb = pack.tensors["token_embd.weight"]
    assert pack.buffer[emb["byteOffset"]:emb["byteOffset"] + emb["byteLength"]] == tensors["token_embd.weight"][2]


def test_prepack_errors_match_reference():
    dims = _dims()
    tensors, blob = _model_gguf(dims)
    bad = write_gguf([("general.architecture", STRING, "llama")], [])
    with pytest.raises(ValueError, match="expected a mistral3 GGUF"):
        prepack.prepack_gguf(bad, requantize=_requant)
    extra = dict(tensors)
    extra["blk.0.extra.weight"] = (12, [256, 8], synth.random_q4k(9, 8).tobytes())
    blob2 = write_gguf(nemotron_metadata(dims), [(n, d, ty, b) for n, (ty, d, b) in extra.items()])
    with pytest.raises(ValueError, match="unpacked matrices: blk.0.extra.weight"):
        prepack.prepack_gguf(blob2, requantize=_requant)
    f32 = dict(tensors)
    f32["blk.1.attn_q.weight"] = (0, [256, 256], bytes(256 * 256 * 4))
    blob3 = write_gguf(nemotron_metadata(dims), [(n, d, ty, b) for n, (ty, d, b) in f32.items()])
    with pytest.raises(ValueError, match="blk.1.attn_q.weight is not a supported quantized matrix"):
        prepack.prepack_gguf(blob3, requantize=_requant)
