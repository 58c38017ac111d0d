"""Host-side mirror of the reference's embedding runtime over libnemo.

``NemotronHipModel`` takes the place of ``NemotronWebGPUModel``
(src/webgpu/model.ts:236-329) and ``NemotronHipPlan`` of
``NemotronExecutionPlan`` (src/webgpu/model.ts:58-234); together they
implement the ``EmbeddingRuntime`` / ``EmbeddingPlan`` interfaces of
src/webgpu/embedding-engine.ts:7-14. ``QuantMatmul`` mirrors
``QuantMatmulKernel`` (src/webgpu/quant-matmul.ts:438-563).

Every method calls the C ABI (include/nemo.h); nothing here computes.
"""
from __future__ import annotations

import asyncio
import ctypes
import math
import threading
from typing import Awaitable, Iterable

import numpy as np

from . import _lib
from ._lib import TYPE_F16, TYPE_F32, TYPE_Q4_0, TYPE_Q4_K, TYPE_Q6_K, Dims, NemoError, check

HIDDEN = 2048
TOKEN_SAMPLE_RATIO = 0.64


def contextual_merged_length(sequence: int) -> int:
    """src/webgpu/model.ts:30-32."""
    return max(1, math.ceil(sequence * TOKEN_SAMPLE_RATIO))


def reference_dims() -> Dims:
    """The reference model's constants (src/webgpu/model.ts:19-28)."""
    d = Dims()
    _lib.load().nemo_dims_reference(ctypes.byref(d))
    return d


def config_dims() -> Dims:
    """The benchmark configuration's encoder: hidden 2048, 32 query heads x 64,
    8 KV heads, FFN 8192, 16 layers, vocabulary 131072."""
    d = reference_dims()
    d.q_heads, d.kv_heads, d.head_dim, d.intermediate = 32, 8, 64, 8192
    return d


def make_dims(**kw) -> Dims:
    d = reference_dims()
    for k, v in kw.items():
        setattr(d, k, v)
    return d


class HipContext:
    """One HIP device (replaces requestWebGPUDevice, src/webgpu/device.ts:6-24)."""

    _shared: dict[int, "HipContext"] = {}

    def __init__(self, device: int = 0):
        L = _lib.load()
        self.device = device
        self._ptr = ctypes.c_void_p()
        check(L.nemo_init(device, ctypes.byref(self._ptr)))

    @classmethod
    def shared(cls, device: int = 0) -> "HipContext":
        if device not in cls._shared:
            cls._shared[device] = cls(device)
        return cls._shared[device]

    @property
    def ptr(self):
        return self._ptr


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


class NemotronHipPlan:
    """An execution plan for `batch` requests of up to `sequence` tokens
    (NemotronExecutionPlan, src/webgpu/model.ts:58-234).

    Runs in flight are counted: ``destroy()`` while some are pending closes
    the plan to new calls at once and frees it when the last one settles,
    so a pending run resolves normally (WebGPU's destroy() is likewise safe
    with work already queued, src/webgpu/model.ts:141-144).
    """

    def __init__(self, model: "NemotronHipModel", batch: int, sequence: int):
        self.model = model
        self.batch = batch
        self.inputSequence = sequence
        self.sequence = contextual_merged_length(sequence)
        self._ptr = ctypes.c_void_p()
        self._lock = threading.Lock()
        self._pending = 0
        self._closed = False
        check(_lib.load().nemo_plan_create(model.ptr, batch, sequence, ctypes.byref(self._ptr)))

    # -- runs in flight ------------------------------------------------------

    def _enter(self) -> None:
        with self._lock:
            if self._closed or not self._ptr:
                raise NemoError(1, "plan was destroyed")
            self._pending += 1

    def _leave(self) -> None:
        with self._lock:
            self._pending -= 1
            last = self._closed and self._pending == 0
        if last:
            self._free()

    def _free(self) -> None:
        with self._lock:
            ptr, self._ptr = self._ptr, None
        if ptr:
            check(_lib.load().nemo_plan_destroy(ptr))

    # -- EmbeddingPlan -------------------------------------------------------

    def _run_entered(self, ids: np.ndarray, lengths: np.ndarray) -> list[np.ndarray]:
        try:
            out = np.empty((self.batch, self.model.hidden), dtype=np.float32)
            u32p = ctypes.POINTER(ctypes.c_uint32)
            check(_lib.load().nemo_plan_run(self._ptr, ids.ctypes.data_as(u32p), ids.size,
                                            lengths.ctypes.data_as(u32p), lengths.size,
                                            out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
            return [out[i].copy() for i in range(self.batch)]
        finally:
            self._leave()

    def run_sync(self, ids, lengths) -> list[np.ndarray]:
        """Blocking run: ids [batch * sequence] (padded after each request),
        lengths [batch] -> `batch` float32 [hidden] embeddings."""
        ids, lengths = _u32(ids).reshape(-1), _u32(lengths).reshape(-1)
        self._enter()
        return self._run_entered(ids, lengths)

    def run(self, ids, lengths) -> "Awaitable[list[np.ndarray]]":
        """EmbeddingPlan.run (src/webgpu/embedding-engine.ts:8): awaitable.

        Called inside a running event loop it returns a future: the run is
        counted in flight as this call returns (as the reference's run has
        written its buffers and submitted by then) and executes on a worker
        thread of that loop, so that distinct plans overlap. Called with no
        loop running (``asyncio.run(plan.run(ids, lengths))``) it returns a
        coroutine that enters the run when it is first awaited, on the loop
        that awaits it; a coroutine never awaited leaves no run counted."""
        ids, lengths = _u32(ids).reshape(-1).copy(), _u32(lengths).reshape(-1).copy()
        try:
            loop = asyncio.get_running_loop()
        except RuntimeError:
            return self._run_later(ids, lengths)
        self._enter()
        try:
            return loop.run_in_executor(None, self._run_entered, ids, lengths)
        except BaseException:
            self._leave()
            raise

    async def _run_later(self, ids: np.ndarray, lengths: np.ndarray) -> list[np.ndarray]:
        self._enter()
        try:
            fut = asyncio.get_running_loop().run_in_executor(None, self._run_entered, ids, lengths)
        except BaseException:
            self._leave()
            raise
        return await fut

    def run_device(self, d_ids: int, lengths, d_out: int, stream: int = 0) -> None:
        """Enqueue on `stream` with ids and output already in device memory."""
        lengths = _u32(lengths).reshape(-1)
        self._enter()
        try:
            check(_lib.load().nemo_plan_run_device(self._ptr, ctypes.c_void_p(d_ids),
                                                   lengths.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                                   lengths.size, ctypes.c_void_p(d_out),
                                                   ctypes.c_void_p(stream or None)))
        finally:
            self._leave()

    def profile(self, ids, lengths) -> dict[str, float]:
        """Milliseconds per stage (src/webgpu/model.ts:178-224)."""
        L = _lib.load()
        ids, lengths = _u32(ids).reshape(-1), _u32(lengths).reshape(-1)
        n = L.nemo_profile_stage_count()
        ms = np.zeros(n, dtype=np.float32)
        u32p = ctypes.POINTER(ctypes.c_uint32)
        self._enter()
        try:
            check(L.nemo_plan_profile(self._ptr, ids.ctypes.data_as(u32p), ids.size, lengths.ctypes.data_as(u32p),
                                      lengths.size, ms.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n))
        finally:
            self._leave()
        return {L.nemo_profile_stage_name(i).decode(): float(ms[i]) for i in range(n)}

    def read_buffer(self, name: str) -> np.ndarray:
        """A plan activation buffer after the last run (f16 rows, or the
        float32 embeddings), as a flat array."""
        L = _lib.load()
        n = ctypes.c_size_t(0)
        self._enter()
        try:
            check(L.nemo_plan_read_buffer(self._ptr, name.encode(), None, ctypes.byref(n)))
            buf = np.empty(n.value, dtype=np.uint8)
            check(L.nemo_plan_read_buffer(self._ptr, name.encode(), buf.ctypes.data_as(ctypes.c_void_p),
                                          ctypes.byref(n)))
        finally:
            self._leave()
        return buf.view(np.float32 if name == "embeddings" else np.float16)

    def destroy(self) -> None:
        """destroy() (src/webgpu/model.ts:141-144): later calls fail with
        'plan was destroyed'; the device memory is released now, or when
        the last run in flight settles."""
        with self._lock:
            if self._closed:
                return
            self._closed = True
            pending = self._pending
        if pending == 0:
            self._free()

    @property
    def pending(self) -> int:
        """Runs (and other calls) of the plan in flight."""
        return self._pending

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class NemotronHipModel:
    """Weights on one device; implements EmbeddingRuntime.

    ``source`` is a ``PrepackedModel`` (src/prepacked/format.ts:54-59), a
    parsed ``GGUFModel`` (src/gguf/types.ts:37-44; dims default to its
    metadata), a mapping name -> (ggml_type, dims, bytes), or None together
    with ``synthetic_seed`` for seeded synthetic weights (``overrides``, a
    mapping of the same form, then replaces some of them).
    """

    # No per-binding storage limit on HIP: the engine's storage cap does not
    # apply (src/webgpu/embedding-engine.ts:64-66 treats undefined as infinity).
    maxStorageBufferBindingSize = None

    def __init__(self, source=None, dims: Dims | None = None, device: int = 0, synthetic_seed: int | None = None,
                 embedding_type: int = TYPE_F16, overrides: dict | None = None):
        self.ctx = HipContext.shared(device)
        is_gguf = hasattr(source, "dataOffset") and hasattr(source, "metadata") and hasattr(source, "version")
        if dims is None and is_gguf:
            from .gguf import dims_from_metadata
            dims = dims_from_metadata(source)
        self.dims = dims if dims is not None else reference_dims()
        self.hidden = self.dims.hidden
        self._ptr = ctypes.c_void_p()
        L = _lib.load()
        check(L.nemo_model_create(self.ctx.ptr, ctypes.byref(self.dims), ctypes.byref(self._ptr)))
        if source is None:
            if synthetic_seed is None:
                raise ValueError("either a source or synthetic_seed is required")
            check(L.nemo_model_synthesize(self._ptr, int(synthetic_seed), int(embedding_type)))
            # tensors given alongside replace their synthetic counterparts
            for name, (ggml_type, dims_, data) in (overrides or {}).items():
                self.set_tensor(name, ggml_type, dims_, data)
        elif hasattr(source, "header") and hasattr(source, "tensors"):
            self._load_prepacked(source)
        elif is_gguf:
            # src/webgpu/model.ts:281-304: every tensor uploaded, q/k/v and
            # gate/up fused at finalize
            view = memoryview(source.buffer)
            for t in source.tensors.values():
                self.set_tensor(t["name"], t["type"], t["dimensions"],
                                view[t["byteOffset"]:t["byteOffset"] + t["byteLength"]])
        else:
            for name, (ggml_type, dims_, data) in source.items():
                self.set_tensor(name, ggml_type, dims_, data)
        check(L.nemo_model_finalize(self._ptr))

    @property
    def ptr(self):
        return self._ptr

    def set_tensor(self, name: str, ggml_type: int, dims: Iterable[int], data) -> None:
        buf = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8) if isinstance(data, (bytes, bytearray, memoryview)) else np.asarray(data).reshape(-1).view(np.uint8))
        d = (ctypes.c_int64 * len(list(dims)))(*[int(x) for x in dims])
        check(_lib.load().nemo_model_set_tensor(self._ptr, name.encode(), int(ggml_type), d, len(d),
                                                buf.ctypes.data_as(ctypes.c_void_p), buf.size))

    def _load_prepacked(self, pack) -> None:
        """src/webgpu/model.ts:263-279: every tensor of the pack is uploaded;
        compact Q4_0 tile32 matrices as TYPE_Q4_0_TILE32 records."""
        from .prepacked import PREPACKED_STORAGE_COMPACT
        view = memoryview(pack.buffer)
        for t in pack.tensors.values():
            type_ = _lib.TYPE_Q4_0_TILE32 if t["storage"] == PREPACKED_STORAGE_COMPACT else t["type"]
            self.set_tensor(t["name"], type_, t["dimensions"], view[t["byteOffset"]:t["byteOffset"] + t["byteLength"]])

    def get_tensor(self, name: str) -> tuple[int, list[int], bytes]:
        """(ggml_type, dims, GGUF bytes) of a tensor as held on the device."""
        L = _lib.load()
        n = ctypes.c_size_t(0)
        t = ctypes.c_int32()
        dims = (ctypes.c_int64 * 4)()
        check(L.nemo_model_get_tensor(self._ptr, name.encode(), ctypes.byref(t), dims, None, ctypes.byref(n)))
        buf = np.empty(n.value, dtype=np.uint8)
        check(L.nemo_model_get_tensor(self._ptr, name.encode(), None, None, buf.ctypes.data_as(ctypes.c_void_p),
                                      ctypes.byref(n)))
        return t.value, [int(x) for x in dims], buf.tobytes()

    def createPlan(self, batch: int, sequence: int) -> NemotronHipPlan:  # noqa: N802 (reference name)
        """src/webgpu/model.ts:328."""
        return NemotronHipPlan(self, batch, sequence)

    create_plan = createPlan

    def destroy(self) -> None:
        if self._ptr:
            check(_lib.load().nemo_model_destroy(self._ptr))
            self._ptr = None


class QuantWeight:
    """One quantized matrix on the device (the weight buffer of
    QuantMatmulKernel.createRun, src/webgpu/quant-matmul.ts:503-509)."""

    def __init__(self, ggml_type: int, n: int, k: int, data, device: int = 0):
        self.ctx = HipContext.shared(device)
        self.type, self.n, self.k = ggml_type, n, k
        buf = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8))
        self._ptr = ctypes.c_void_p()
        check(_lib.load().nemo_weight_create(self.ctx.ptr, ggml_type, n, k, buf.ctypes.data_as(ctypes.c_void_p),
                                             buf.size, ctypes.byref(self._ptr)))

    def matmul(self, d_x: int, m: int, d_y: int, algo: int = _lib.MATMUL_AUTO, stream: int = 0) -> None:
        """Y[m, n] = f16(X[m, k] W^T) on device pointers."""
        check(_lib.load().nemo_weight_matmul(self._ptr, ctypes.c_void_p(d_x), m, ctypes.c_void_p(d_y), algo,
                                             ctypes.c_void_p(stream or None)))

    def matmul_static(self, d_x: int, m: int, d_y: int, algo: int = _lib.MATMUL_AUTO, stream: int = 0) -> None:
        """matmul() without allocating: scratch in the library's per-GPU static
        array (nemo_weight_matmul_static; calls on one GPU must not overlap)."""
        check(_lib.load().nemo_weight_matmul_static(self._ptr, ctypes.c_void_p(d_x), m, ctypes.c_void_p(d_y), algo,
                                                    ctypes.c_void_p(stream or None)))

    def dequantize(self, d_out: int, stream: int = 0) -> None:
        check(_lib.load().nemo_weight_dequantize(self._ptr, ctypes.c_void_p(d_out), ctypes.c_void_p(stream or None)))

    def destroy(self) -> None:
        if self._ptr:
            check(_lib.load().nemo_weight_destroy(self._ptr))
            self._ptr = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def dequantize_device(ggml_type: int, d_raw: int, n_values: int, d_out_f32: int = 0, d_out_f16: int = 0,
                      stream: int = 0) -> None:
    """Decode raw GGUF blocks already in device memory."""
    check(_lib.load().nemo_dequantize(ggml_type, ctypes.c_void_p(d_raw), n_values, ctypes.c_void_p(d_out_f32 or None),
                                      ctypes.c_void_p(d_out_f16 or None), ctypes.c_void_p(stream or None)))


def probe_stream(d_src: int, nbytes: int, loads_per_thread: int, d_sink: int, stream: int = 0) -> None:
    """Roofline probe: one kernel reading `nbytes` at d_src once with
    coalesced 16-byte loads (nbytes == 0: one empty launch); d_sink holds 256
    uint32 (include/nemo.h nemo_probe_stream)."""
    check(_lib.load().nemo_probe_stream(ctypes.c_void_p(d_src or None), nbytes, loads_per_thread,
                                        ctypes.c_void_p(d_sink or None), ctypes.c_void_p(stream or None)))


def requantize_q40(src_type: int, data, k: int, n: int, device: int = 0) -> bytes:
    """requantizeMatrixToQ40 (src/gguf/quantization.ts:101-131) on the GPU:
    raw GGUF Q4_K / Q6_K / Q4_0 bytes of an n x k matrix -> GGUF Q4_0 bytes."""
    ctx = HipContext.shared(device)
    src = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8))
    out = np.empty(n * (k // 32) * 18, dtype=np.uint8)
    check(_lib.load().nemo_requantize_q40(ctx.ptr, int(src_type), src.ctypes.data_as(ctypes.c_void_p), src.size,
                                          int(k), int(n), out.ctypes.data_as(ctypes.c_void_p), out.size))
    return out.tobytes()


__all__ = [
    "TYPE_F16", "TYPE_F32", "TYPE_Q4_0", "TYPE_Q4_K", "TYPE_Q6_K", "Dims", "NemoError", "HipContext",
    "NemotronHipModel", "NemotronHipPlan", "QuantWeight", "contextual_merged_length", "reference_dims",
    "config_dims", "make_dims", "dequantize_device", "requantize_q40",
]
