"""The JavaScript host (nemotron-3-embed-webgpu_amd/js) under Node: engine
behaviour, the pack format and the addon surface without a GPU, and a pack
built by the JS host byte-identical to the Python builder's."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from nemo_amd import prepacked as pp

HERE = os.path.dirname(os.path.abspath(__file__))
NODE = shutil.which("node")
pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def _node(script, *args):
    r = subprocess.run([NODE, os.path.join(HERE, "js", script), *args], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def test_js_engine():
    assert "6/6 passed" in _node("engine.test.js")


def test_js_host_and_cross_language_pack(tmp_path):
    out = tmp_path / "js.wgpack"
    assert "3/3 passed" in _node("host.test.js", str(out))
    n, k = 40, 64
    raw = bytes(((i * 37 + 11) & 255) for i in range(n * (k // 32) * 18))
    packed = pp.pack_q40_tile32("m", [{"name": "a", "k": k, "n": 10, "bytes": raw[:10 * 2 * 18]},
                                      {"name": "b", "k": k, "n": 30, "bytes": raw[10 * 2 * 18:]}])
    norm = pp.raw_tensor("norm", [4], 0, bytes([7] * 16))
    want = pp.build_prepacked_file("feed", 123, {"general.name": "cross"}, [norm, packed])
    assert out.read_bytes() == want
