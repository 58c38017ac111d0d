"""Throughput benchmark: 16 concurrent 150-token requests through the 16-layer
Nemotron-3-Embed encoder on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W]

One step = one execution-plan run over one batch of 16 requests x 150 tokens
(token ids and embeddings resident in HBM; the host hands over only the
lengths). The model is the benchmark configuration's encoder (hidden 2048,
32 query heads x 64, 8 KV heads, FFN 8192, 16 layers, vocabulary 131072) with
seeded synthetic weights: N(0, 0.02) quantized to Q4_K (ffn_down Q6_K), an
f16 N(0, 0.02) token table, norm weights 1.

Printed JSON (one line on stdout):
  value        embeddings/s over exactly K timed steps (HIP events)
  roofline     the dominant kernel (the Q4_K gate/up GEMM): algorithmic flops
               per launch / its average launch duration, from HIP events
               bracketing every launch on the plan's stream, against the dense
               fp16 MFMA peak
  cpu_baseline the oracle's CPU forward of the same encoder (float64 numpy,
               binary16 storage) on a bounded sample of the workload
Progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nemotron-3-embed-webgpu_amd"))

BATCH, TOKENS = 16, 150
SEED = 1003
MFMA_F16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def workload_ids(vocab: int):
    import numpy as np
    rng = np.random.default_rng(SEED + 1)
    ids = rng.integers(1, vocab, size=(BATCH, TOKENS), dtype=np.int64).astype(np.uint32)
    ids[:, 0] = 1  # BOS
    return ids.reshape(-1), np.full(BATCH, TOKENS, dtype=np.uint32)


def gate_up_flops(dims) -> tuple[float, int]:
    """Algorithmic flops of every gate/up GEMM launch of one step, and the
    launch count: 2 * rows * (2 F) * hidden per layer; rows = 16 * 150 in the
    layers before the merge, 16 * ceil(0.64 * 150) after it."""
    from nemo_amd.runtime import contextual_merged_length
    rows_full, rows_merged = BATCH * TOKENS, BATCH * contextual_merged_length(TOKENS)
    per_row = 2.0 * (2 * dims.intermediate) * dims.hidden
    total = 0.0
    for layer in range(dims.layers):
        total += per_row * (rows_full if layer < dims.merge_after_layer else rows_merged)
    return total, dims.layers


def step_flops(dims) -> float:
    """All projection flops of one step (QKV, O, gate/up, down)."""
    from nemo_amd.runtime import contextual_merged_length
    H, F = dims.hidden, dims.intermediate
    QKV = (dims.q_heads + 2 * dims.kv_heads) * dims.head_dim
    QW = dims.q_heads * dims.head_dim
    per_row = 2.0 * (H * QKV + QW * H + H * 2 * F + F * H)
    rows_full, rows_merged = BATCH * TOKENS, BATCH * contextual_merged_length(TOKENS)
    return sum(per_row * (rows_full if l < dims.merge_after_layer else rows_merged) for l in range(dims.layers))


def cpu_baseline(model, dims, ids, budget_s: float = 20.0) -> dict:
    """Time the oracle's forward (numpy, float64 BLAS) for whole requests of the
    same workload until about `budget_s` seconds of CPU work are spent."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle
    import synth
    from threadpoolctl import threadpool_limits
    threads = min(16, os.cpu_count() or 1)
    log(f"cpu baseline: reading back and dequantizing weights ({threads} BLAS threads)")
    tensors = {}
    names = ["token_embd.weight", "output_norm.weight"] + [
        f"blk.{l}.{t}.weight" for l in range(dims.layers)
        for t in ("attn_qkv", "attn_output", "ffn_gate_up", "ffn_down", "attn_norm", "ffn_norm")]
    for name in names:
        typ, d, data = model.get_tensor(name)
        tensors[name] = (typ, [x for x in d if x != 1] or [1], data)
    om = synth.oracle_model(dims, tensors)
    del tensors
    done, elapsed = 0, 0.0
    with threadpool_limits(limits=threads):
        while elapsed < budget_s and done < BATCH:
            t0 = time.perf_counter()
            oracle.forward_request(om, ids[done * TOKENS:(done + 1) * TOKENS].astype(np.int64))
            elapsed += time.perf_counter() - t0
            done += 1
            log(f"cpu baseline: {done} request(s) in {elapsed:.1f} s")
    return {"value": done / elapsed, "unit": "embeddings/s", "cores": threads, "kind": "port",
            "sample": f"{done} of the 16 requests (150 tokens each) through all {dims.layers} layers, "
                      f"oracle forward (numpy float64, binary16 storage), {elapsed:.1f} s"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build runs the encoder pass on a single MI355X "
              "(requests are independent; see DESIGN.md for how the path would shard).", file=sys.stderr)
        return 2

    import numpy as np
    import torch
    from nemo_amd import runtime as rt

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dims = rt.config_dims()
    log("synthesizing the 16-layer Q4_K model on the device")
    t0 = time.perf_counter()
    model = rt.NemotronHipModel(None, dims=dims, synthetic_seed=SEED, embedding_type=rt.TYPE_F16)
    log(f"model ready in {time.perf_counter() - t0:.1f} s")
    ids, lengths = workload_ids(dims.vocab)
    plan = model.createPlan(BATCH, TOKENS)
    d_ids = torch.from_numpy(ids.view(np.int32).copy()).cuda()
    d_out = torch.empty((BATCH, dims.hidden), dtype=torch.float32, device="cuda")
    # A dedicated stream (default priority): the plan enqueues its kernels on
    # it and the timing events are recorded on it.
    stream = torch.cuda.Stream()
    assert stream.cuda_stream != 0

    def step():
        plan.run_device(d_ids.data_ptr(), lengths, d_out.data_ptr(), stream.cuda_stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"warmup {args.warmup} done")
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    value = BATCH * 1000.0 / ms
    log(f"{args.steps} steps: {ms:.3f} ms/step, {value:.1f} embeddings/s")
    emb = d_out.cpu().numpy()
    norms = np.linalg.norm(emb, axis=1)
    assert np.all(np.isfinite(emb)) and np.all(np.abs(norms - 1) < 0.01), "embeddings are not unit vectors"

    # Dominant kernel: the gate/up GEMM. HIP events bracket each of its
    # launches (the plan's profile pass), over `steps` instrumented steps.
    stage_ms = 0.0
    for _ in range(args.steps):
        stage_ms += plan.profile(ids, lengths)["ffn_up_gate"]
    flops, launches = gate_up_flops(dims)
    avg_launch_ms = stage_ms / (args.steps * launches)
    achieved = flops / launches / (avg_launch_ms * 1e-3) / 1e12
    log(f"gate/up GEMM: {avg_launch_ms * 1e3:.1f} us per launch, {achieved:.1f} TFLOP/s")
    all_flops = step_flops(dims)

    result = {
        "metric": "embeddings/sec @16x150 tok",
        "value": round(value, 2),
        "unit": "embeddings/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded ids; device-synthesized N(0,0.02) weights quantized to Q4_K/Q6_K)",
        "config": {"workload": "16 concurrent requests x 150 tokens, 16-layer encoder", "batch": BATCH,
                   "tokens_per_request": TOKENS, "hidden": dims.hidden, "q_heads": dims.q_heads,
                   "kv_heads": dims.kv_heads, "head_dim": dims.head_dim, "intermediate": dims.intermediate,
                   "layers": dims.layers, "vocab": dims.vocab, "weights": "Q4_K (ffn_down Q6_K)",
                   "parallelism": "single GPU"},
        "projection_tflops": round(all_flops / (ms * 1e-3) / 1e12, 1),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "gate/up Q4_K GEMM", "avg_launch_us": round(avg_launch_ms * 1e3, 2)},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(model, dims, ids)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
