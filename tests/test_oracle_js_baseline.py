"""The plain-JavaScript CPU baseline (oracle/q4k_matmul_cpu.js, what
bench.py times on the box's Node) computes the same Y = X W^T as the C
oracle's restatement of the reference's CPU check (src/main.ts:97-104 with
dequantizeQ4KBlock, src/gguf/quantization.ts:19-38), bit for bit, including
blocks with subnormal and extreme scales."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle
import synth

NODE = shutil.which("node")
SCRIPT = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "q4k_matmul_cpu.js")
pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def test_js_baseline_equals_c_oracle(tmp_path):
    m, n, k = 3, 24, 512
    w = synth.random_q4k(1101, n * k // 256).reshape(-1, 144)
    w[0, 0:2] = [0x01, 0x00]        # d = smallest subnormal
    w[1, 2:4] = [0xff, 0x7b]        # dmin = 65504
    w[2, 0:4] = [0x00, 0x00, 0x00, 0x80]  # d = +0, dmin = -0
    x = synth.normal(1108, m * k).astype(np.float16).reshape(m, k)
    (tmp_path / "w.bin").write_bytes(w.tobytes())
    (tmp_path / "x.bin").write_bytes(x.tobytes())
    r = subprocess.run([NODE, SCRIPT, str(tmp_path / "w.bin"), str(tmp_path / "x.bin"), str(m), str(n), str(k), "1",
                        str(tmp_path / "y.bin")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    info = json.loads(r.stdout)
    got = np.frombuffer((tmp_path / "y.bin").read_bytes(), np.float64).reshape(m, n)
    want = oracle.q4k_matmul_cpu(w.reshape(-1), x, m, n, k)
    assert np.array_equal(got, want)
    seq = 0.0
    for v in got.reshape(-1).tolist():  # summed in order, as the script does
        seq += v
    assert info["checksum"] == seq
    assert info["node"].startswith("v") and len(info["ms"]) == 1
