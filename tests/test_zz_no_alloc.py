"""nemo_weight_matmul_static, the matmul entry point that allocates nothing
(its scratch is the library's static per-GPU array), against
nemo_weight_matmul on the same inputs: bit for bit, on two calls in a row
whose second input is smaller, for every algorithm and each kind of scratch
(GEMV and split-K fp32 partial sums, the two-pass f16 expansion at the
array's full size), and the rejection of a call whose scratch would not fit.
Both entry points are called through the C ABI."""
import ctypes

import numpy as np
import pytest

import synth
from nemo_amd import _lib
from nemo_amd import runtime as rt

pytestmark = pytest.mark.gpu

GEN = {12: synth.random_q4k, 14: synth.random_q6k, 2: synth.random_q40}
NAN16 = 0x7E00  # every output element must be written


def _weight(type_, n, k, seed):
    raw = GEN[type_](seed, n * k // (32 if type_ == 2 else 256))
    return rt.QuantWeight(type_, n, k, raw.tobytes())


def _call(fn, w, dx, m, dy, algo):
    _lib.check(fn(w._ptr, ctypes.c_void_p(dx.data_ptr()), m, ctypes.c_void_p(dy.data_ptr()), algo,
                  ctypes.c_void_p(None)))


def _both(torch, w, x16, m, algo):
    """Y from nemo_weight_matmul_static, then from nemo_weight_matmul, for the
    first m rows of x16."""
    L = _lib.load()
    n = w.n
    dx = torch.from_numpy(x16[:m].view(np.int16).copy()).cuda()
    ys = []
    for fn in (L.nemo_weight_matmul_static, L.nemo_weight_matmul):
        dy = torch.full((m, n), NAN16, dtype=torch.int16, device="cuda")
        _call(fn, w, dx, m, dy, algo)
        torch.cuda.synchronize()
        ys.append(dy.cpu().numpy())
    return ys


CASES = [
    # (type, n, k, algo, m of the first call, m of the second)
    (14, 2048, 8192, _lib.MATMUL_GEMV, 160, 15),         # GEMV, K split 4 ways: fp32 partials
    (12, 2048, 2048, _lib.MATMUL_GEMV, 48, 1),           # GEMV, unsplit: no scratch
    (12, 5120, 2048, _lib.MATMUL_GEMM_SPLIT, 64, 17),    # 64-row tiles, K split 4 ways: fp32 partials
    (2, 2048, 3072, _lib.MATMUL_GEMM_SPLIT, 50, 33),     # Q4_0, 6 chunks
    (12, 16384, 2048, _lib.MATMUL_TWO_PASS, 600, 300),   # f16 expansion: the full 64 MiB
    (14, 2048, 8192, _lib.MATMUL_AUTO, 2400, 1536),      # the plan's down projection shape
    (12, 3072, 2048, _lib.MATMUL_AUTO, 170, 100),        # AUTO: tiles, then the GEMV
    (12, 384, 512, _lib.MATMUL_GEMM, 333, 70),           # fused tiles: no scratch
    (2, 256, 512, _lib.MATMUL_GEMM_MID, 65, 1),
]


@pytest.mark.parametrize("type_,n,k,algo,m1,m2", CASES)
def test_static_scratch_matches_allocating_entry_point(torch_cuda, type_, n, k, algo, m1, m2):
    torch = torch_cuda
    seed = 9301 + n + k + type_ + algo
    w = _weight(type_, n, k, seed)
    x16 = synth.normal(seed + 1, m1 * k).astype(np.float16).reshape(m1, k)
    for m in (m1, m2):
        got, want = _both(torch, w, x16, m, algo)
        assert np.array_equal(got, want), f"m={m}: {np.count_nonzero(got != want)} elements differ"
        assert np.all(np.isfinite(got.view(np.float16))), f"m={m}: an output element was not written"
    w.destroy()


def test_static_scratch_rejects_oversize(torch_cuda):
    """A two-pass expansion of 16640 x 2048 halves (66.6 MB) exceeds the
    64 MiB array: the call fails with NEMO_ERR_INVALID and launches nothing;
    a call that fits still runs afterwards."""
    torch = torch_cuda
    n, k = 16640, 2048
    assert n * k * 2 > _lib.STATIC_SCRATCH_BYTES
    w = _weight(12, n, k, 9401)
    x16 = synth.normal(9402, 300 * k).astype(np.float16).reshape(300, k)
    dx = torch.from_numpy(x16.view(np.int16).copy()).cuda()
    dy = torch.full((300, n), NAN16, dtype=torch.int16, device="cuda")
    L = _lib.load()
    with pytest.raises(_lib.NemoError) as e:
        _call(L.nemo_weight_matmul_static, w, dx, 300, dy, _lib.MATMUL_TWO_PASS)
    assert e.value.status == 1  # NEMO_ERR_INVALID
    assert "static scratch holds 67108864" in str(e.value)
    torch.cuda.synchronize()
    assert bool((dy == NAN16).all())
    got, want = _both(torch, w, x16, 120, _lib.MATMUL_GEMV)
    assert np.array_equal(got, want)
    w.destroy()


GRAPH_CASES = [
    # (type, n, k, algo, m): the scratch kinds, each captured into a HIP graph
    (12, 16384, 2048, _lib.MATMUL_TWO_PASS, 600),   # f16 expansion, then the f16 MFMA GEMM
    (12, 5120, 2048, _lib.MATMUL_GEMM_SPLIT, 64),   # 64-row tiles, fp32 partials, fixed-order reduction
    (14, 2048, 8192, _lib.MATMUL_GEMV, 160),        # GEMV with K split 4 ways, fp32 partials
]


@pytest.mark.parametrize("type_,n,k,algo,m", GRAPH_CASES)
def test_static_scratch_under_graph_capture(torch_cuda, type_, n, k, algo, m):
    """nemo_weight_matmul_static captured into a HIP graph (torch.cuda.graph)
    after one eager call of the same shape, which configures its kernels.
    The paths record no memset (every kernel writes each scratch element it
    reads). The graph is replayed three times with a new X written in place
    before each replay and eager calls of the allocating entry point between
    replays; every replay must equal the eager result for its X bit for bit."""
    torch = torch_cuda
    L = _lib.load()
    seed = 9501 + n + k + type_ + algo
    w = _weight(type_, n, k, seed)
    xs = [synth.normal(seed + 1 + i, m * k).astype(np.float16).reshape(m, k) for i in range(4)]
    dx = torch.from_numpy(xs[0].view(np.int16).copy()).cuda()
    dy = torch.full((m, n), NAN16, dtype=torch.int16, device="cuda")
    dref = torch.full((m, n), NAN16, dtype=torch.int16, device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        _lib.check(L.nemo_weight_matmul_static(w._ptr, ctypes.c_void_p(dx.data_ptr()), m,
                                               ctypes.c_void_p(dy.data_ptr()), algo,
                                               ctypes.c_void_p(stream.cuda_stream)))
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        _lib.check(L.nemo_weight_matmul_static(w._ptr, ctypes.c_void_p(dx.data_ptr()), m,
                                               ctypes.c_void_p(dy.data_ptr()), algo,
                                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    for i in range(1, 4):
        dx.copy_(torch.from_numpy(xs[i].view(np.int16).copy()))
        dy.fill_(NAN16)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = dy.cpu().numpy()
        _call(L.nemo_weight_matmul, w, dx, m, dref, algo)
        torch.cuda.synchronize()
        want = dref.cpu().numpy()
        assert np.array_equal(got, want), f"replay {i}: {np.count_nonzero(got != want)} elements differ"
        assert np.all(np.isfinite(got.view(np.float16)))
    del g
    w.destroy()
