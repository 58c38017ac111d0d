"""A Q4_K_M-style GGUF through GGUFReader -> NemotronHipModel (dims from the
mistral3 metadata; src/gguf/reader.ts, src/webgpu/model.ts:281-304): attn_q
and attn_k Q4_K with attn_v Q6_K (kept as separate projections), ffn_down
Q6_K, token table Q6_K. Embeddings within cosine 0.9999 of the oracle."""
import numpy as np
import pytest

import oracle
import synth
from gguf_writer import nemotron_metadata, write_gguf
from nemo_amd import gguf
from nemo_amd import runtime as rt

pytestmark = pytest.mark.gpu


def _q4km_tensors(dims, seed):
    t = synth.model_tensors(dims, seed=seed, embedding_type=14, fused=False)
    KW = dims.kv_heads * dims.head_dim
    for l in range(dims.layers):
        w = 0.02 * synth.normal(seed + 1000 + l, KW * dims.hidden).reshape(KW, dims.hidden)
        t[f"blk.{l}.attn_v.weight"] = (14, [dims.hidden, KW], synth.quantize_q6k(w).tobytes())
    return t


def test_q4km_gguf_matches_oracle(torch_cuda):
    # two layers: the reference's merge after layer 4 clamps to the last layer
    dims = rt.make_dims(hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, layers=2, vocab=320,
                        merge_after_layer=2)
    tensors = _q4km_tensors(dims, 4242)
    blob = write_gguf(nemotron_metadata(dims, alignment=64),
                      [(name, d, typ, data) for name, (typ, d, data) in tensors.items()], alignment=64)
    model_file = gguf.GGUFReader(blob).parse(gguf.NEMOTRON3_METADATA_KEYS)
    model = rt.NemotronHipModel(model_file)
    assert (model.dims.hidden, model.dims.layers, model.dims.vocab, model.dims.merge_after_layer) == (256, 2, 320, 2)
    om = synth.oracle_model(dims, tensors)
    seqs = [[1] + list(synth.randint(300 + i, n - 1, 2, 320)) for i, n in enumerate([30, 12, 45])]
    S = max(len(s) for s in seqs)
    ids = np.full(len(seqs) * S, 11, dtype=np.uint32)
    for i, s in enumerate(seqs):
        ids[i * S:i * S + len(s)] = s
    got = model.createPlan(len(seqs), S).run_sync(ids, [len(s) for s in seqs])
    for i, s in enumerate(seqs):
        ref = oracle.forward_request(om, np.array(s))
        c = float(np.dot(got[i], ref) / (np.linalg.norm(got[i]) * np.linalg.norm(ref)))
        assert c >= 0.9999, f"request {i}: cosine {c:.6f}"
    # alone, the request takes the same kernels as in the batch: above 16
    # tokens, projections with K <= 512 are never split, in any regime
    single = model.createPlan(1, len(seqs[2])).run_sync(np.array(seqs[2], dtype=np.uint32), [len(seqs[2])])[0]
    assert np.array_equal(single.view(np.uint32), got[2].view(np.uint32))


def test_mixed_gate_up_types_cannot_combine(torch_cuda):
    """gate and up must share a type to be fused (combineQ4,
    src/webgpu/model.ts:288-292); the error names both parts."""
    dims = rt.make_dims(hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=256, layers=1, vocab=64,
                        merge_after_layer=1)
    t = synth.model_tensors(dims, seed=5, fused=False)
    w = 0.02 * synth.normal(6, 256 * 256).reshape(256, 256)
    t["blk.0.ffn_up.weight"] = (14, [256, 256], synth.quantize_q6k(w).tobytes())
    with pytest.raises(rt.NemoError, match="cannot combine blk.0.ffn_gate.weight, blk.0.ffn_up.weight"):
        rt.NemotronHipModel(t, dims=dims)
