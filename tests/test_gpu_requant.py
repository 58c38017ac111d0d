"""requantizeMatrixToQ40 on the GPU (nemo_requantize_q40) bit-exact with the
oracle's restatement of the reference's JavaScript (src/gguf/quantization.ts:
77-131), and the prepack tool end to end: GGUF -> .wgpack (GPU
requantization) -> model -> embeddings."""
import numpy as np
import pytest

import oracle
import synth
from gguf_writer import nemotron_metadata, write_gguf
from nemo_amd import prepack, prepacked
from nemo_amd import runtime as rt

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("type_,gen,n,k", [(12, synth.random_q4k, 37, 512), (14, synth.random_q6k, 33, 768),
                                           (2, synth.random_q40, 20, 256), (12, synth.random_q4k, 2048, 2048)])
def test_requant_bit_exact(torch_cuda, type_, gen, n, k):
    per = 256 if type_ != 2 else 32
    raw = gen(8000 + n + type_, n * k // per).tobytes()
    got = rt.requantize_q40(type_, raw, k, n)
    assert got == oracle.requantize_to_q40(raw, type_, k, n)


def test_requant_reference_kat_and_edges(torch_cuda):
    # tests/quantization.test.ts:51-59: Q6_K zero quants, scales 1 -> -32
    block = np.zeros(210, dtype=np.uint8)
    block[192:208] = 1
    block[208:210] = [0x00, 0x3C]
    out = rt.requantize_q40(14, block.tobytes(), 256, 1)
    assert len(out) == 8 * 18 and np.all(oracle.dequantize(2, out) == -32)
    # all-zero blocks, ties of |max| (the first wins), extreme scales
    d = np.array([0x0000, 0x0001, 0x7BFF, 0x3C00] * 4, dtype=np.uint16)
    sc = np.tile(np.array([[63, 0, 1, 2, 63, 5, 9, 63]]), (16, 1))
    m = np.tile(np.array([[0, 63, 1, 0, 63, 2, 0, 1]]), (16, 1))
    q = synth.randint(9, 16 * 256, 0, 16).reshape(16, 256)
    q[:, :32] = 15
    q[:, 32:64] = 0
    raw = synth.q4k_blocks(d, d[::-1].copy(), sc, m, q).reshape(-1).tobytes()
    assert rt.requantize_q40(12, raw, 256, 16) == oracle.requantize_to_q40(raw, 12, 256, 16)


def test_requant_errors(torch_cuda):
    raw = synth.random_q4k(1, 2).tobytes()
    with pytest.raises(rt.NemoError, match="K=300 is not divisible by a K-quant block"):
        rt.requantize_q40(12, raw, 300, 1)
    with pytest.raises(rt.NemoError, match="source has 288 bytes; expected 144"):
        rt.requantize_q40(12, raw, 256, 1)


def test_prepack_gpu_matches_oracle_and_runs(torch_cuda):
    dims = rt.make_dims(hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, layers=2, vocab=300,
                        merge_after_layer=2)
    t = synth.model_tensors(dims, seed=55, embedding_type=14, fused=False)
    blob = write_gguf(nemotron_metadata(dims), [(n, d, ty, b) for n, (ty, d, b) in t.items()])
    gpu_pack = prepack.prepack_gguf(blob)
    cpu_pack = prepack.prepack_gguf(blob, requantize=lambda ty, b, k, n: oracle.requantize_to_q40(bytes(b), ty, k, n))
    assert gpu_pack == cpu_pack
    pack = prepacked.parse_prepacked_model(gpu_pack)
    model = rt.NemotronHipModel(pack, dims=dims)
    # the oracle on the packed Q4_0 weights: fused rows [q; k; v] and [gate; up]
    ot = {}
    for name, (ty, d, b) in t.items():
        if len(d) == 2 and name != "token_embd.weight":
            ot[name] = (2, d, oracle.requantize_to_q40(b, ty, d[0], d[1]))
        else:
            ot[name] = (ty, d, b)
    om = synth.oracle_model(dims, ot)
    seq = [1] + list(synth.randint(56, 39, 2, 300))
    got = model.createPlan(1, 40).run_sync(np.array(seq, dtype=np.uint32), [40])[0]
    ref = oracle.forward_request(om, np.array(seq))
    assert float(np.dot(got, ref) / (np.linalg.norm(got) * np.linalg.norm(ref))) >= 0.9999
