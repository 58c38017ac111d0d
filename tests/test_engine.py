"""The micro-batching engine (src/webgpu/embedding-engine.ts) with fake
runtimes, as the reference's own tests drive it
(tests/embedding-engine.test.ts:5-50), plus the failure paths those tests
leave open: a failing run rejects its whole batch and later batches still run.
"""
import asyncio

import numpy as np
import pytest

from nemo_amd.engine import NemotronEmbeddingEngine


class _Ids:
    def __init__(self, rows):
        self._rows = rows

    def tolist(self):
        return self._rows


class _Tok:
    def __init__(self, ids):
        self.input_ids = _Ids(ids)


def _run(coro):
    return asyncio.new_event_loop().run_until_complete(coro)


def test_coalesces_sixteen_requests_and_preserves_order():
    # tests/embedding-engine.test.ts:5-23
    calls = []

    class Runtime:
        maxStorageBufferBindingSize = None

        def createPlan(self, batch, sequence):  # noqa: N802
            class Plan:
                async def run(self, ids, lengths):
                    calls.append({"batch": batch, "sequence": sequence, "ids": list(ids), "lengths": list(lengths)})
                    return [np.array([ids[i * sequence + 1]], np.float32) for i in range(batch)]
            return Plan()

    async def main():
        engine = NemotronEmbeddingEngine(Runtime(), lambda text: _Tok([[int(text)]]), 16, 0, 99)
        return await asyncio.gather(*[engine.embed(str(i + 1)) for i in range(16)])

    results = _run(main())
    assert len(calls) == 1
    assert calls[0]["batch"] == 16 and calls[0]["sequence"] == 2 and calls[0]["lengths"] == [2] * 16
    assert [float(r[0]) for r in results] == [float(i + 1) for i in range(16)]


def test_pads_mixed_lengths_after_final_token():
    # tests/embedding-engine.test.ts:25-36
    recorded = []

    class Runtime:
        maxStorageBufferBindingSize = None

        def createPlan(self, batch, sequence):  # noqa: N802
            class Plan:
                async def run(self, ids, lengths):
                    recorded.extend(int(i) for i in ids)
                    return [np.zeros(1, np.float32) for _ in range(batch)]
            return Plan()

    async def main():
        engine = NemotronEmbeddingEngine(Runtime(), lambda t: _Tok([[int(x) for x in t.split(",")]]), 16, 0, 99, 99)
        await asyncio.gather(engine.embed("1"), engine.embed("2,3"))

    _run(main())
    assert recorded == [99, 1, 99, 99, 2, 3]


def test_splits_batches_at_the_storage_limit():
    # tests/embedding-engine.test.ts:38-50
    batches = []

    class Runtime:
        maxStorageBufferBindingSize = 2 * 6144 * 2 * 2

        def createPlan(self, batch, sequence):  # noqa: N802
            class Plan:
                async def run(self, ids, lengths):
                    batches.append(batch)
                    return [np.zeros(1, np.float32) for _ in range(batch)]
            return Plan()

    async def main():
        engine = NemotronEmbeddingEngine(Runtime(), lambda t: _Tok([[1]]), 16, 0, 1)
        await asyncio.gather(*[engine.embed("x") for _ in range(5)])

    _run(main())
    assert batches == [2, 2, 1]


def test_long_context_cap_and_plan_cache():
    """Sequences of 1500+ tokens run at most 8 per batch
    (src/webgpu/embedding-engine.ts:68); plans are cached per batch:sequence."""
    created, runs = [], []

    class Runtime:
        maxStorageBufferBindingSize = None

        def createPlan(self, batch, sequence):  # noqa: N802
            created.append((batch, sequence))

            class Plan:
                async def run(self, ids, lengths):
                    runs.append(batch)
                    return [np.zeros(1, np.float32) for _ in range(batch)]
            return Plan()

    async def main():
        engine = NemotronEmbeddingEngine(Runtime(), lambda t: _Tok([[1] * 1500]), 16, 0, 1)
        await asyncio.gather(*[engine.embed("x") for _ in range(16)])

    _run(main())
    assert runs == [8, 8]
    assert created == [(8, 1500)]


def test_failed_run_rejects_whole_batch_and_queue_drains():
    """src/webgpu/embedding-engine.ts:84-93: every request of a failing batch
    rejects with the run's error; requests queued behind it still run."""
    runs = []

    class Runtime:
        maxStorageBufferBindingSize = None

        def createPlan(self, batch, sequence):  # noqa: N802
            class Plan:
                async def run(self, ids, lengths):
                    runs.append(batch)
                    if len(runs) == 1:
                        raise RuntimeError("device lost")
                    return [np.full(1, i, np.float32) for i in range(batch)]
            return Plan()

    async def main():
        engine = NemotronEmbeddingEngine(Runtime(), lambda t: _Tok([[1, int(t)]]), 2, 0, 1)
        return await asyncio.gather(*[engine.embed(str(i)) for i in range(5)], return_exceptions=True)

    results = _run(main())
    assert runs == [2, 2, 1]
    assert all(isinstance(r, RuntimeError) and str(r) == "device lost" for r in results[:2])
    assert [float(r[0]) for r in results[2:]] == [0.0, 1.0, 0.0]


def test_bos_prepended_once_and_batch_size_bounds():
    seen = []

    class Runtime:
        maxStorageBufferBindingSize = None

        def createPlan(self, batch, sequence):  # noqa: N802
            class Plan:
                async def run(self, ids, lengths):
                    seen.append((list(ids), list(lengths)))
                    return [np.zeros(1, np.float32) for _ in range(batch)]
            return Plan()

    async def main():
        engine = NemotronEmbeddingEngine(Runtime(), lambda t: _Tok([[int(x) for x in t.split(",")]]))
        await asyncio.gather(engine.embed("1,4"), engine.embed("4"))

    _run(main())
    assert seen == [([1, 4, 1, 4], [2, 2])]
    for bad in (0, 17):
        with pytest.raises(ValueError, match="maxBatchSize must be between 1 and 16"):
            NemotronEmbeddingEngine(None, None, bad)
