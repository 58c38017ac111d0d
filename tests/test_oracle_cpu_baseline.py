"""The all-cores CPU baseline (OpenMP over weight rows) computes every output
with the same loop as the one-thread restatement of the reference's CPU check
(src/main.ts:97-104 with dequantizeQ4KBlock, src/gguf/quantization.ts:19-38),
so its results are the same bits for any thread count, and both equal the
float64 dot of the dequantized matrix."""
import numpy as np
import pytest

import oracle
import synth


@pytest.mark.parametrize("threads", [1, 2, 3, 8])
def test_all_cores_baseline_same_bits(threads):
    m, n, k = 5, 37, 768
    w = synth.random_q4k(1201, n * k // 256)
    x = synth.normal(1208, m * k).astype(np.float16).reshape(m, k)
    single = oracle.q4k_matmul_cpu(w, x, m, n, k)
    assert np.array_equal(oracle.q4k_matmul_cpu_mt(w, x, m, n, k, threads), single)
    # and the product itself: dequantized rows against the float64 dot
    deq = oracle.dequantize(12, w).reshape(n, k).astype(np.float64)
    ref = x.astype(np.float64) @ deq.T
    np.testing.assert_allclose(single, ref, rtol=1e-12, atol=1e-12)
