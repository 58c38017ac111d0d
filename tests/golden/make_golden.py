"""Writes the golden fixtures of tests/golden/ from the oracle.

    python tests/golden/make_golden.py

codec_vectors.json  seeded Q4_K / Q6_K / Q4_0 blocks (hex) with their
                    float32 decodes (bit patterns) and a float32 -> binary16
                    sample (src/gguf/quantization.ts, src/math/f16.ts), plus
                    the reference's own known-answer vectors restated as data
                    (tests/quantization.test.ts, tests/prepacked-format.test.ts,
                    tests/model-config.test.ts).
tiny_forward.json   a seeded tiny encoder (weights rebuilt by tests/synth.py
                    from the recorded seed) and the float32 embeddings the
                    oracle forward gives for four ragged requests
                    (src/webgpu/model.ts:146-176).

The oracle is the checker these fixtures freeze: tests/test_golden.py
re-derives them and the GPU tests compare the HIP path against them.
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.dirname(HERE)]

import numpy as np  # noqa: E402

import oracle  # noqa: E402
import synth  # noqa: E402

TINY = dict(hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, layers=3, vocab=300,
            merge_after_layer=1, kv_stride_threshold=24)
TINY_SEED = 4242
TINY_REQUESTS = [
    [1] + list(range(40, 69)),                      # 30 tokens: stride-3 keys in every layer (30 > 24)
    [1, 7, 99, 250],
    [1],
    [1] + [int(t) for t in synth.randint(77, 17, 2, 300)],
]


def codec_vectors() -> dict:
    out = {}
    for name, type_, gen, nb, seed in (("q4_k", 12, synth.random_q4k, 6, 101), ("q6_k", 14, synth.random_q6k, 6, 102),
                                        ("q4_0", 2, synth.random_q40, 24, 103)):
        raw = gen(seed, nb)
        out[name] = {"type": type_, "blocks": raw.tobytes().hex(),
                     "f32_bits": oracle.dequantize(type_, raw).view(np.uint32).tolist()}
    sample = (synth.normal(104, 512) * np.exp2(synth.randint(105, 512, -26, 17))).astype(np.float32)
    out["f32_to_f16"] = {"f32_bits": sample.view(np.uint32).tolist(),
                         "f16_bits": oracle.float_to_half(sample).tolist()}
    out["reference_kats"] = {
        "half_to_float": [[0x3C00, 1.0], [0xC000, -2.0], [0x0000, 0.0]],
        "contextual_merged_length": [[1, 1], [15, 10], [50, 32], [150, 96], [500, 320], [1500, 960], [5000, 3200]],
        "tile32_record0": [0x00, 0x3C, 0x00, 0x00, 0x00, 0x11, 0x22, 0x33],
        "tile32_record1": [0x00, 0x40, 0x00, 0x00, 0xFF, 0xEE, 0xDD, 0xCC],
    }
    return out


def tiny_forward() -> dict:
    dims = oracle.Dims(**TINY)
    model = synth.oracle_model(dims, synth.model_tensors(dims, seed=TINY_SEED))
    emb = [oracle.forward_request(model, np.array(r)) for r in TINY_REQUESTS]
    return {"dims": TINY, "seed": TINY_SEED, "requests": TINY_REQUESTS,
            "embeddings_f32_bits": [e.view(np.uint32).tolist() for e in emb]}


def main() -> None:
    for name, data in (("codec_vectors.json", codec_vectors()), ("tiny_forward.json", tiny_forward())):
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(data, f, separators=(",", ":"))
        print(f"wrote {name}")


if __name__ == "__main__":
    main()
