"""The JavaScript host on the GPU: a .wgpack of the tiny golden model's raw
tensors is loaded through parsePrepackedModel -> NemotronHipModel, embedded
through NemotronEmbeddingEngine, and compared with the frozen oracle
embeddings (tests/js/gpu.test.js)."""
import json
import os
import shutil
import subprocess

import pytest

import synth
from nemo_amd import prepacked as pp
from nemo_amd import runtime as rt

HERE = os.path.dirname(os.path.abspath(__file__))
NODE = shutil.which("node")
pytestmark = [pytest.mark.gpu, pytest.mark.skipif(NODE is None, reason="node is not installed")]


def test_js_host_on_gpu(tmp_path):
    golden_path = os.path.join(HERE, "golden", "tiny_forward.json")
    with open(golden_path) as f:
        g = json.load(f)
    dims = rt.make_dims(**g["dims"])
    tensors = synth.model_tensors(dims, seed=g["seed"])
    pack = pp.build_prepacked_file("synthetic", 0, {"general.name": "tiny golden"},
                                   [pp.raw_tensor(name, d, t, data) for name, (t, d, data) in tensors.items()])
    path = tmp_path / "tiny.wgpack"
    path.write_bytes(pack)
    r = subprocess.run([NODE, os.path.join(HERE, "js", "gpu.test.js"), str(path), golden_path], capture_output=True,
                       text=True, timeout=180)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "5/5 passed" in r.stdout


def test_js_prepack_matches_python(tmp_path):
    """node js/prepack.js on a GGUF gives the same .wgpack bytes as the
    Python tool (both requantize on the GPU)."""
    from gguf_writer import nemotron_metadata, write_gguf
    from nemo_amd import prepack
    dims = rt.make_dims(hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=256, layers=2, vocab=64,
                        merge_after_layer=2)
    t = synth.model_tensors(dims, seed=17, embedding_type=14, fused=False)
    src = tmp_path / "m.gguf"
    src.write_bytes(write_gguf(nemotron_metadata(dims), [(n, d, ty, b) for n, (ty, d, b) in t.items()]))
    out = tmp_path / "m.wgpack"
    script = os.path.join(os.path.dirname(HERE), "nemotron-3-embed-webgpu_amd", "js", "prepack.js")
    r = subprocess.run([NODE, script, str(src), str(out)], capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stdout + r.stderr
    assert out.read_bytes() == prepack.prepack_gguf(src.read_bytes())
