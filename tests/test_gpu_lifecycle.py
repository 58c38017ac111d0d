"""Plan lifetime and stream ordering on the GPU (regressions of the fixed
paths; tests/test_runtime_lifecycle.py checks the host logic without a GPU):

* destroy() while runs are pending: they resolve with the right embeddings,
  later calls fail with 'plan was destroyed', the native plan is freed once
  (src/webgpu/model.ts:141-144);
* one plan driven on two caller streams in turn (nemo_plan_run_device): the
  second run waits for the first on the device, since both use the plan's
  buffers, so each output equals that request run alone;
* read_buffer after a run on a caller's stream sees that run's activations;
* an enqueue that fails partway on a caller's stream still orders the plan's
  later runs, reads and destroy after the kernels it queued.
"""
import asyncio

import numpy as np
import pytest

import synth
from nemo_amd import _lib
from nemo_amd import runtime as rt

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    dims = rt.make_dims(hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, layers=2, vocab=300,
                        merge_after_layer=1)
    m = rt.NemotronHipModel(synth.model_tensors(dims, seed=77), dims=dims)
    yield m


def _batch(requests, S):
    ids = np.full(len(requests) * S, 11, dtype=np.uint32)
    for i, r in enumerate(requests):
        ids[i * S:i * S + len(r)] = r
    return ids, [len(r) for r in requests]


def test_destroy_while_runs_pending(torch_cuda, model):
    reqs = [[1] + list(range(2, 40)), [1, 5, 9], [1] + list(range(100, 160))]
    S = max(len(r) for r in reqs)
    ids, lengths = _batch(reqs, S)
    ref_plan = model.createPlan(len(reqs), S)
    want = ref_plan.run_sync(ids, lengths)
    ref_plan.destroy()

    async def scenario():
        plan = model.createPlan(len(reqs), S)
        runs = [plan.run(ids, lengths) for _ in range(3)]
        plan.destroy()
        with pytest.raises(rt.NemoError, match="plan was destroyed"):
            plan.run(ids, lengths)
        outs = await asyncio.gather(*runs)
        assert plan.pending == 0 and not plan._ptr
        return outs

    for out in asyncio.run(scenario()):
        for got, ref in zip(out, want):
            assert np.array_equal(got, ref)


def test_runs_on_two_caller_streams_are_ordered(torch_cuda, model):
    torch = torch_cuda
    S = 150
    reqs_a = [[1] + list(synth.randint(5, S - 1, 2, 300))]
    reqs_b = [[1] + list(synth.randint(6, 99, 2, 300))]
    plan = model.createPlan(1, S)
    want_b = plan.run_sync(*_batch(reqs_b, S))[0]
    want_a = plan.run_sync(*_batch(reqs_a, S))[0]
    norm_a = plan.read_buffer("norm_merged").copy()  # request a's activations, from its blocking run
    ids_a = torch.from_numpy(_batch(reqs_a, S)[0].view(np.int32).copy()).cuda()
    ids_b = torch.from_numpy(_batch(reqs_b, S)[0].view(np.int32).copy()).cuda()
    out_a = torch.zeros(256, dtype=torch.float32, device="cuda")
    out_b = torch.zeros(256, dtype=torch.float32, device="cuda")
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    # the zero fills above ran on the current stream; the plan's runs on s1 and s2 come after them
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    for _ in range(5):
        plan.run_device(ids_b.data_ptr(), [len(reqs_b[0])], out_b.data_ptr(), s2.cuda_stream)
        plan.run_device(ids_a.data_ptr(), [len(reqs_a[0])], out_a.data_ptr(), s1.cuda_stream)
    # The last run (request a, on s1) wrote the plan's activation buffers
    # after every run of b: read_buffer waits for it although it went to a
    # caller's stream, and sees a's activations, not b's.
    got_norm = plan.read_buffer("norm_merged")
    torch.cuda.synchronize()
    assert np.array_equal(out_a.cpu().numpy(), want_a)
    assert np.array_equal(out_b.cpu().numpy(), want_b)
    assert np.array_equal(got_norm.view(np.uint16), norm_a.view(np.uint16))
    plan.destroy()


def test_failed_enqueue_on_caller_stream_is_waited_for(torch_cuda, model):
    """An enqueue that fails partway (here a HIP status check made to fail by
    the library's testing hook, after some of the graph's kernels are
    queued) on a caller's stream: the call raises, returns only once that
    stream has drained (its queued kernels still use the plan's buffers),
    and the plan stays usable: a run on its own stream gives the request's
    embedding, and destroy() then succeeds."""
    torch = torch_cuda
    L = _lib.load()
    S = 150
    reqs = [[1] + list(synth.randint(7, S - 1, 2, 300))]
    ids, lengths = _batch(reqs, S)
    plan = model.createPlan(1, S)
    want = plan.run_sync(ids, lengths)[0]
    d_ids = torch.from_numpy(ids.view(np.int32).copy()).cuda()
    d_out = torch.zeros(256, dtype=torch.float32, device="cuda")
    a = torch.randn(2048, 2048, device="cuda")
    s1 = torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s1):
        for _ in range(8):  # keeps s1 busy, so the plan's kernels queue behind this work
            a = torch.tanh(a @ a)
    for checks in (6, 15):  # mid-way through the first and the second layer's launches
        L.nemo_debug_fail_after(checks)
        try:
            with pytest.raises(_lib.NemoError, match="injected failure"):
                plan.run_device(d_ids.data_ptr(), lengths, d_out.data_ptr(), s1.cuda_stream)
        finally:
            L.nemo_debug_fail_after(0)
        assert s1.query(), "the failed call returned before its stream drained"
    got = plan.run_sync(ids, lengths)[0]
    assert np.array_equal(got, want)
    plan.run_device(d_ids.data_ptr(), lengths, d_out.data_ptr(), s1.cuda_stream)
    plan.destroy()
    assert s1.query(), "destroy returned before the plan's work on the caller's stream"
    assert np.array_equal(d_out.cpu().numpy(), want)
