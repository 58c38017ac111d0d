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
    assert "4/4 passed" in r.stdout
