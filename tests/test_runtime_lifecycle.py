"""Plan lifetime in the Python host without a GPU: the in-flight run count
of NemotronHipPlan against a stand-in for libnemo that records calls and
holds a run until the test releases it. destroy() while a run is pending
must close the plan to new calls at once, let the pending run resolve, and
free the native plan exactly once, after it (WebGPU's destroy() is safe
with queued work, src/webgpu/model.ts:141-144)."""
import asyncio
import ctypes
import threading
import types

import numpy as np
import pytest

from nemo_amd import _lib, runtime as rt


class FakeLib:
    def __init__(self, fail_runs=False):
        self.calls = []
        self.started = threading.Event()
        self.release = threading.Event()
        self.fail_runs = fail_runs

    def nemo_plan_create(self, model, batch, sequence, out):
        out._obj.value = 0x1234
        self.calls.append("create")
        return 0

    def nemo_plan_run(self, plan, ids, n_ids, lengths, n_lengths, out):
        self.calls.append("run")
        self.started.set()
        assert self.release.wait(10)
        return 1 if self.fail_runs else 0

    def nemo_plan_destroy(self, plan):
        assert getattr(plan, "value", plan) == 0x1234
        self.calls.append("destroy")
        return 0

    def nemo_last_error(self):
        return b"run failed"


@pytest.fixture
def fake(monkeypatch):
    lib = FakeLib()
    monkeypatch.setattr(_lib, "load", lambda: lib)
    return lib


MODEL = types.SimpleNamespace(ptr=ctypes.c_void_p(1), hidden=4)


def test_destroy_while_run_pending_defers_the_free(fake):
    async def scenario():
        plan = rt.NemotronHipPlan(MODEL, 2, 3)
        pending = plan.run(np.arange(6), [3, 3])  # counted in flight as the call returns
        assert plan.pending == 1
        loop = asyncio.get_running_loop()
        assert await loop.run_in_executor(None, fake.started.wait, 10)
        plan.destroy()
        assert "destroy" not in fake.calls and plan.pending == 1
        with pytest.raises(rt.NemoError, match="plan was destroyed"):
            plan.run(np.arange(6), [3, 3])
        with pytest.raises(rt.NemoError, match="plan was destroyed"):
            plan.run_sync(np.arange(6), [3, 3])
        fake.release.set()
        out = await pending
        assert len(out) == 2 and all(v.shape == (4,) for v in out)
        assert fake.calls == ["create", "run", "destroy"] and plan.pending == 0
        plan.destroy()  # idempotent
        assert fake.calls.count("destroy") == 1

    asyncio.run(scenario())


def test_destroy_before_the_run_starts_still_resolves(fake):
    async def scenario():
        plan = rt.NemotronHipPlan(MODEL, 1, 2)
        fake.release.set()
        pending = plan.run(np.arange(2), [2])
        plan.destroy()  # the executor thread may not have started yet
        out = await pending
        assert len(out) == 1
        assert fake.calls == ["create", "run", "destroy"]

    asyncio.run(scenario())


def test_destroy_without_runs_frees_at_once(fake):
    plan = rt.NemotronHipPlan(MODEL, 1, 2)
    plan.destroy()
    assert fake.calls == ["create", "destroy"]
    with pytest.raises(rt.NemoError, match="plan was destroyed"):
        plan.run_sync(np.arange(2), [2])


def test_failed_run_settles_the_count(fake):
    fake.fail_runs = True

    async def scenario():
        plan = rt.NemotronHipPlan(MODEL, 1, 2)
        fake.release.set()
        pending = plan.run(np.arange(2), [2])
        plan.destroy()
        with pytest.raises(rt.NemoError, match="run failed"):
            await pending
        assert fake.calls == ["create", "run", "destroy"] and plan.pending == 0

    asyncio.run(scenario())


def test_run_awaited_from_asyncio_run(fake):
    """asyncio.run(plan.run(ids, lengths)): with no loop running when run() is
    called, it returns a coroutine that enters the run when awaited."""
    plan = rt.NemotronHipPlan(MODEL, 1, 2)
    fake.release.set()
    coro = plan.run(np.arange(2), [2])
    assert plan.pending == 0  # not entered until awaited
    out = asyncio.run(coro)
    assert len(out) == 1 and out[0].shape == (4,)
    assert fake.calls == ["create", "run"] and plan.pending == 0
    plan.destroy()
    assert fake.calls == ["create", "run", "destroy"]


def test_unawaited_coroutine_leaves_no_run_counted(fake):
    plan = rt.NemotronHipPlan(MODEL, 1, 2)
    coro = plan.run(np.arange(2), [2])
    coro.close()
    assert plan.pending == 0
    plan.destroy()
    assert fake.calls == ["create", "destroy"]


def test_coroutine_awaited_after_destroy_fails(fake):
    plan = rt.NemotronHipPlan(MODEL, 1, 2)
    coro = plan.run(np.arange(2), [2])
    plan.destroy()
    with pytest.raises(rt.NemoError, match="plan was destroyed"):
        asyncio.run(coro)
    assert fake.calls == ["create", "destroy"]
