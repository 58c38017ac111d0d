"""Closed-loop embedding benchmark (scripts/bench-lib.ts, scripts/workloads.ts).

``benchmark_target`` runs ``concurrency`` workers that each send the next
input, await its embedding and repeat until the deadline; it reports
requests/s, tokens/s and nearest-rank latency percentiles of the successful
requests, as the reference's harness does. ``comparison_workload`` gives the
fixed-length inputs of the published comparison (COMPARISON_TOKEN_COUNTS):
``tokens - 1`` words that a word-level tokenizer maps to one token each, BOS
making up the last one.
"""
from __future__ import annotations

import asyncio
import math
import time
from dataclasses import dataclass

COMPARISON_TOKEN_COUNTS = (15, 50, 150, 500, 1500, 5000)  # scripts/workloads.ts:9


def percentile(sorted_values, fraction: float) -> float:
    """Nearest rank (scripts/bench-lib.ts:28-32)."""
    if len(sorted_values) == 0:
        return math.nan
    index = min(len(sorted_values) - 1, math.ceil(len(sorted_values) * fraction) - 1)
    return sorted_values[index]


@dataclass
class BenchmarkOptions:
    concurrency: int
    duration_ms: float
    warmup_requests: int
    inputs: list
    tokens_per_input: int


async def benchmark_target(target, options: BenchmarkOptions) -> dict:
    """scripts/bench-lib.ts:34-96. `target` has `name` and an async
    `embed(input)` returning a sequence of floats."""
    if options.concurrency < 1:
        raise ValueError("concurrency must be >= 1")
    if not options.inputs:
        raise ValueError("at least one input is required")
    for i in range(options.warmup_requests):
        await target.embed(options.inputs[i % len(options.inputs)])
    deadline = time.perf_counter() + options.duration_ms / 1000.0
    latencies: list[float] = []
    state = {"requests": 0, "errors": 0, "dims": 0, "next": 0}
    started = time.perf_counter()

    async def worker():
        while time.perf_counter() < deadline:
            item = options.inputs[state["next"] % len(options.inputs)]
            state["next"] += 1
            t0 = time.perf_counter()
            try:
                embedding = await target.embed(item)
                state["dims"] = state["dims"] or len(embedding)
                if len(embedding) != state["dims"]:
                    raise ValueError(f"embedding dimension changed to {len(embedding)}")
                state["requests"] += 1
            except Exception:  # counted, as the reference counts failed requests
                state["errors"] += 1
            finally:
                latencies.append((time.perf_counter() - t0) * 1000.0)

    await asyncio.gather(*[worker() for _ in range(options.concurrency)])
    elapsed_ms = (time.perf_counter() - started) * 1000.0
    latencies.sort()
    ok = latencies[:state["requests"]]
    rps = state["requests"] / (elapsed_ms / 1000.0)
    return {
        "target": target.name, "concurrency": options.concurrency, "requests": state["requests"],
        "errors": state["errors"], "elapsedMs": elapsed_ms, "requestsPerSecond": rps,
        "tokensPerSecond": rps * options.tokens_per_input,
        "latencyMs": {"p50": percentile(ok, 0.5), "p95": percentile(ok, 0.95), "p99": percentile(ok, 0.99),
                      "mean": (sum(ok) / state["requests"]) if state["requests"] else math.nan},
        "embeddingDimensions": state["dims"],
    }


def comparison_workload(tokens: int) -> dict:
    """scripts/workloads.ts:25-33: one input of tokens - 1 words."""
    return {"name": "acceptance", "nominalTokens": tokens, "inputs": [" ".join(["vector"] * (tokens - 1))]}


__all__ = ["COMPARISON_TOKEN_COUNTS", "BenchmarkOptions", "benchmark_target", "comparison_workload", "percentile"]
