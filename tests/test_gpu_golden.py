"""The HIP path against the committed golden fixtures (tests/golden/*.json)
through the C ABI: decoding bit-exact, the tiny encoder's embeddings within
cosine 0.9999 of the oracle's frozen values."""
import json
import os

import numpy as np
import pytest

import synth
from nemo_amd import runtime as rt

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "q4_0"])
def test_dequantize_matches_golden(torch_cuda, name):
    torch = torch_cuda
    v = _load("codec_vectors.json")[name]
    raw = np.frombuffer(bytes.fromhex(v["blocks"]), dtype=np.uint8)
    want = np.array(v["f32_bits"], np.uint32)
    d_raw = torch.from_numpy(raw.copy()).cuda()
    out = torch.empty(want.size, dtype=torch.float32, device="cuda")
    rt.dequantize_device(v["type"], d_raw.data_ptr(), want.size, out.data_ptr(), 0)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want)


def test_tiny_encoder_matches_golden(torch_cuda):
    g = _load("tiny_forward.json")
    dims = rt.make_dims(**g["dims"])
    model = rt.NemotronHipModel(synth.model_tensors(dims, seed=g["seed"]), dims=dims)
    reqs = g["requests"]
    S = max(len(r) for r in reqs)
    ids = np.full(len(reqs) * S, 11, dtype=np.uint32)
    for i, r in enumerate(reqs):
        ids[i * S:i * S + len(r)] = r
    got = model.createPlan(len(reqs), S).run_sync(ids, [len(r) for r in reqs])
    for i, bits in enumerate(g["embeddings_f32_bits"]):
        want = np.array(bits, np.uint32).view(np.float32).astype(np.float64)
        c = float(np.dot(got[i], want) / (np.linalg.norm(got[i]) * np.linalg.norm(want)))
        assert c >= 0.9999, f"request {i}: cosine {c:.6f}"
