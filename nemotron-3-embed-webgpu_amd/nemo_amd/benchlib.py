"""Closed-loop embedding benchmark (scripts/bench-lib.ts, scripts/workloads.ts).

``benchmark_target`` runs ``concurrency`` workers that each send the next
input, await its embedding and repeat until the deadline; it reports
requests/s, tokens/s and nearest-rank latency percentiles of the successful
requests, as the reference's harness does. ``comparison_workload`` gives the
fixed-length inputs of the published comparison (COMPARISON_TOKEN_COUNTS):
``tokens - 1`` words that a word-level tokenizer maps to one token each, BOS
making up the last one. ``comparison_matrix`` runs the published
comparison itself (one request alone, then 16 at once in native batches) on
an ``EmbeddingRuntime``, as the reference's browser matrix does.
"""
from __future__ import annotations

import asyncio
import math
import time
import zlib
from dataclasses import dataclass

import numpy as np

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


class _Encoded:
    def __init__(self, ids):
        self.input_ids = np.asarray([ids], dtype=np.int64)


class WordTokenizer:
    """A stand-in tokenizer with the property the comparison workloads rely on
    (scripts/workloads.ts:28-29): BOS, then one token per whitespace word.
    Word ids are a CRC-32 of the word, mapped into [2, vocab)."""

    def __init__(self, vocab: int, bos_token: int = 1):
        self.vocab = vocab
        self.bos_token = bos_token

    def __call__(self, text: str) -> _Encoded:
        words = text.split()
        return _Encoded([self.bos_token] + [2 + zlib.crc32(w.encode()) % (self.vocab - 2) for w in words])


def _dot(a, b) -> float:
    return float(np.dot(np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)))


async def comparison_matrix(runtime, tokenizer, token_counts=COMPARISON_TOKEN_COUNTS, write=print,
                            bos_token: int = 1, cosine_floor: float = 0.999) -> list[dict]:
    """The comparison matrix (src/main.ts:244-313) on `runtime`.

    Per exact token count: the comparison text is tokenized (BOS prepended if
    missing) and must give exactly that many tokens; a batch-1 plan's output
    is the reference embedding; `singleRps` is requests/s of back-to-back
    batch-1 runs (10/5/3/1 repeats for <=150/<=500/<=1500/longer); 16 requests
    are then split into native batches of min(16, or 8 from 1500 tokens, the
    storage limit's cap), every embedding of a warm-up round must have cosine
    >= `cosine_floor` with the reference, and `aggregateRps` is
    16 * repeats / elapsed over 5/3/2/1 repeats of all batches run at once.
    The reference also compares with an LM Studio endpoint; that leg has no
    counterpart here and `baselineCosine` is None."""
    results = []
    for exact in token_counts:
        text = comparison_workload(exact)["inputs"][0]
        tokens = [int(t) for t in tokenizer(text).input_ids.tolist()[0]]
        if tokens[0] != bos_token:
            tokens.insert(0, bos_token)
        if len(tokens) != exact:
            raise ValueError(f"expected {exact} tokens, tokenizer produced {len(tokens)}")

        def exact_batch(batch):
            return (np.tile(np.asarray(tokens, dtype=np.uint32), batch), np.full(batch, exact, dtype=np.uint32))

        single_plan = runtime.createPlan(1, exact)
        single = exact_batch(1)
        reference = (await single_plan.run(*single))[0]
        single_repeats = 10 if exact <= 150 else 5 if exact <= 500 else 3 if exact <= 1500 else 1
        started = time.perf_counter()
        for _ in range(single_repeats):
            await single_plan.run(*single)
        single_rps = single_repeats / (time.perf_counter() - started)
        write(f"{exact} tokens: {single_rps:.2f} req/s single")

        limit = getattr(runtime, "maxStorageBufferBindingSize", None)
        bytes_per_request = exact * 6144 * 2 * 2
        cap = 8 if exact >= 1500 else 16
        native = max(1, min(cap, math.floor(limit / bytes_per_request))) if limit is not None else cap
        sizes, remaining = [], 16
        while remaining > 0:
            sizes.append(min(native, remaining))
            remaining -= native
        plans = [runtime.createPlan(b, exact) for b in sizes]
        batches = [exact_batch(b) for b in sizes]
        warm = await asyncio.gather(*[p.run(*b) for p, b in zip(plans, batches)])
        cosines = [_dot(reference, e) for batch in warm for e in batch]
        worst = min(cosines)
        if worst < cosine_floor:
            raise ValueError(f"{exact}-token batch cosine {worst} is below {cosine_floor}")
        repeats = 5 if exact <= 150 else 3 if exact <= 500 else 2 if exact <= 1500 else 1
        started = time.perf_counter()
        for _ in range(repeats):
            await asyncio.gather(*[p.run(*b) for p, b in zip(plans, batches)])
        aggregate_rps = repeats * 16 / (time.perf_counter() - started)
        result = {"exactTokens": exact, "singleRps": single_rps, "aggregateRps": aggregate_rps,
                  "scaling": aggregate_rps / single_rps, "baselineCosine": None, "worstBatchCosine": worst,
                  "nativeBatch": native}
        results.append(result)
        write(f"{exact} tokens: {single_rps:.2f} req/s single; {aggregate_rps:.2f} req/s at 16 concurrent; "
              f"{aggregate_rps / single_rps:.2f}x scaling; native batch {native}")
        single_plan.destroy()
        for p in plans:
            p.destroy()
    return results


__all__ = ["COMPARISON_TOKEN_COUNTS", "BenchmarkOptions", "WordTokenizer", "benchmark_target", "comparison_matrix",
           "comparison_workload", "percentile"]
