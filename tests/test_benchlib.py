"""Benchmark utilities (nemo_amd/benchlib.py), as the reference's own tests
drive them (tests/bench-lib.test.ts, tests/workloads.test.ts)."""
import asyncio

import pytest

from nemo_amd import benchlib


def test_nearest_rank_percentiles():
    # tests/bench-lib.test.ts:5-8
    assert benchlib.percentile([1, 2, 3, 4], 0.5) == 2
    assert benchlib.percentile([1, 2, 3, 4], 0.95) == 4
    assert benchlib.percentile([], 0.5) != benchlib.percentile([], 0.5)  # NaN


def test_runs_the_requested_number_of_concurrent_workers():
    # tests/bench-lib.test.ts:10-30
    state = {"active": 0, "peak": 0}

    class Fake:
        name = "fake"

        async def embed(self, _):
            state["active"] += 1
            state["peak"] = max(state["peak"], state["active"])
            await asyncio.sleep(0.002)
            state["active"] -= 1
            return [1, 2, 3]

    result = asyncio.new_event_loop().run_until_complete(benchlib.benchmark_target(
        Fake(), benchlib.BenchmarkOptions(concurrency=4, duration_ms=20, warmup_requests=0, inputs=["input"],
                                          tokens_per_input=1)))
    assert state["peak"] == 4
    assert result["requests"] > 0 and result["embeddingDimensions"] == 3 and result["errors"] == 0
    assert result["latencyMs"]["p50"] <= result["latencyMs"]["p95"] <= result["latencyMs"]["p99"]


def test_errors_are_counted_and_inputs_validated():
    class Failing:
        name = "failing"

        async def embed(self, _):
            await asyncio.sleep(0.001)
            raise RuntimeError("boom")

    loop = asyncio.new_event_loop()
    result = loop.run_until_complete(benchlib.benchmark_target(
        Failing(), benchlib.BenchmarkOptions(2, 10, 0, ["x"], 1)))
    assert result["requests"] == 0 and result["errors"] > 0
    with pytest.raises(ValueError, match="concurrency must be >= 1"):
        loop.run_until_complete(benchlib.benchmark_target(Failing(), benchlib.BenchmarkOptions(0, 10, 0, ["x"], 1)))
    with pytest.raises(ValueError, match="at least one input is required"):
        loop.run_until_complete(benchlib.benchmark_target(Failing(), benchlib.BenchmarkOptions(1, 10, 0, [], 1)))


def test_comparison_workloads():
    # tests/workloads.test.ts:14-24
    assert benchlib.COMPARISON_TOKEN_COUNTS == (15, 50, 150, 500, 1500, 5000)
    for tokens in benchlib.COMPARISON_TOKEN_COUNTS:
        w = benchlib.comparison_workload(tokens)
        assert w["nominalTokens"] == tokens and len(w["inputs"]) == 1
        assert len(w["inputs"][0].split()) == tokens - 1
