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


class _FakePlan:
    def __init__(self, log, batch, sequence, vector):
        self.log, self.batch, self.sequence, self.vector = log, batch, sequence, vector
        log.append(("create", batch, sequence))

    async def run(self, ids, lengths):
        assert ids.size == self.batch * self.sequence and list(lengths) == [self.sequence] * self.batch
        assert all(ids[i * self.sequence] == 1 for i in range(self.batch))  # BOS leads every request
        await asyncio.sleep(0)
        return [self.vector(self.batch, i) for i in range(self.batch)]

    def destroy(self):
        self.log.append(("destroy", self.batch, self.sequence))


class _FakeRuntime:
    def __init__(self, limit=None, vector=None):
        self.maxStorageBufferBindingSize = limit
        self.log = []
        self.vector = vector or (lambda batch, i: [1.0, 0.0])

    def createPlan(self, batch, sequence):  # noqa: N802
        return _FakePlan(self.log, batch, sequence, self.vector)


def _matrix(runtime, counts, **kw):
    return asyncio.new_event_loop().run_until_complete(benchlib.comparison_matrix(
        runtime, benchlib.WordTokenizer(1000), counts, write=lambda _: None, **kw))


def test_matrix_plans_follow_the_native_batch_rule():
    # src/main.ts:281-285: 16 requests in native batches, 8 from 1500 tokens
    rt = _FakeRuntime()
    results = _matrix(rt, (15, 1500))
    creates = [e[1:] for e in rt.log if e[0] == "create"]
    assert creates == [(1, 15), (16, 15), (1, 1500), (8, 1500), (8, 1500)]
    assert sorted(e[1:] for e in rt.log if e[0] == "destroy") == sorted(creates)
    assert [r["nativeBatch"] for r in results] == [16, 8]
    assert all(r["worstBatchCosine"] == 1.0 and r["baselineCosine"] is None for r in results)
    assert all(abs(r["scaling"] - r["aggregateRps"] / r["singleRps"]) < 1e-9 for r in results)


def test_matrix_storage_limit_caps_the_native_batch():
    # 150 tokens x 6144 x 4 bytes per request: a 16 MiB limit fits 4
    rt = _FakeRuntime(limit=16 * 1024 * 1024)
    results = _matrix(rt, (150,))
    assert results[0]["nativeBatch"] == 4
    assert [e[1] for e in rt.log if e[0] == "create"] == [1, 4, 4, 4, 4]


def test_matrix_rejects_divergent_batches_and_wrong_token_counts():
    rt = _FakeRuntime(vector=lambda batch, i: [1.0, 0.0] if batch == 1 or i else [0.99, 0.14])
    with pytest.raises(ValueError, match="15-token batch cosine"):
        _matrix(rt, (15,))

    def short(text):
        return benchlib.WordTokenizer(1000)(" ".join(text.split()[:-1]))

    with pytest.raises(ValueError, match="expected 50 tokens, tokenizer produced 49"):
        asyncio.new_event_loop().run_until_complete(benchlib.comparison_matrix(
            _FakeRuntime(), short, (50,), write=lambda _: None))


def test_word_tokenizer_gives_bos_plus_one_token_per_word():
    tok = benchlib.WordTokenizer(131072)
    ids = tok(benchlib.comparison_workload(150)["inputs"][0]).input_ids.tolist()[0]
    assert len(ids) == 150 and ids[0] == 1 and len(set(ids[1:])) == 1 and 2 <= ids[1] < 131072
