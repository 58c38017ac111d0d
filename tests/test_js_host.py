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


def test_js_plan_lifetime():
    """destroy() with runs in flight, against a stand-in addon (tests/js/lifecycle.test.js)."""
    assert "4/4 passed" in _node("lifecycle.test.js")


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


def test_js_gguf_reader_matches_python(tmp_path):
    """The JS host's GGUFReader and the Python one agree on a file with every
    metadata value type and every tensor type; 64-bit values are BigInt in JS
    (src/gguf/reader.ts:121-130)."""
    import json
    import sys
    sys.path.insert(0, HERE)
    from gguf_writer import nemotron_metadata, write_gguf
    from test_gguf import _sample
    from nemo_amd import gguf, runtime as rt
    md, tensors = _sample(64)
    d = rt.make_dims(hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, layers=2, vocab=40)
    md += nemotron_metadata(d)
    tensors.append(("token_embd.weight", [256, 40], 1, bytes(256 * 40 * 2)))
    path = tmp_path / "m.gguf"
    path.write_bytes(write_gguf(md, tensors, alignment=64))
    py = gguf.GGUFReader(path.read_bytes()).parse()
    js = json.loads(_node("gguf_dump.js", str(path)))
    assert (js["version"], js["alignment"], js["dataOffset"]) == (py.version, py.alignment, py.dataOffset)
    assert js["tensors"] == list(py.tensors.values())
    for key, value in py.metadata.items():
        got = js["metadata"][key]
        if key in ("a.u64", "a.i64"):
            assert got == f"bigint:{value}"
        elif isinstance(value, float):
            assert got == pytest.approx(value)
        else:
            assert got == value
    assert js["dims"]["hidden"] == 256 and js["dims"]["layers"] == 2 and js["dims"]["vocab"] == 40
    assert js["dims"]["mergeAfterLayer"] == 2
    filtered = json.loads(_node("gguf_dump.js", str(path), "filter"))
    assert set(filtered["metadata"]) <= gguf.NEMOTRON3_METADATA_KEYS


def test_pack_header_json_matches_javascript():
    """The Python pack builder writes its JSON header as JSON.stringify does
    (number formatting, UTF-8 text), so both hosts produce identical packs."""
    import json
    import random
    from nemo_amd.prepacked import js_json
    rng = random.Random(5)
    vals = [1e6, 9.999999747378752e-06, 1e21, 1e20, 1e-7, 1.2e-7, 5e-324, 1.7976931348623157e308, -0.5, 65504.0]
    vals += [rng.uniform(-1, 1) * 10 ** rng.randint(-30, 30) for _ in range(500)]
    value = {"v": vals, "s": "héllo\n\t\u0001\"x\\", "i": [0, -3, 2 ** 52], "b": [True, False, None]}
    r = subprocess.run([NODE, "-e", "process.stdout.write(JSON.stringify(" + json.dumps(value) + "))"],
                       capture_output=True, text=True, timeout=60)
    assert js_json(value) == r.stdout
