"""ctypes binding of libnemo.so (the C ABI declared in include/nemo.h).

The library is loaded from the package directory (next to ``csrc/``). There
is no fallback: if it is missing or a call fails, an exception is raised.
"""
from __future__ import annotations

import ctypes
import os

PACKAGE_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PACKAGE_DIR, "libnemo.so")

NEMO_OK = 0
STATUS_NAMES = {1: "invalid", 2: "missing", 3: "device", 4: "out of memory", 5: "unsupported"}

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 2, 12, 14
TYPE_Q4_0_TILE32 = 258  # wgpack q4_0-tile32-compact records (include/nemo.h)
MATMUL_AUTO, MATMUL_GEMM, MATMUL_GEMV, MATMUL_TWO_PASS, MATMUL_GEMM_MID, MATMUL_GEMM_SPLIT = 0, 1, 2, 3, 4, 5
STATIC_SCRATCH_BYTES = 64 << 20  # NEMO_STATIC_SCRATCH_BYTES

# Every symbol include/nemo.h declares.
EXPORTED = [
    "nemo_dims_reference", "nemo_last_error", "nemo_version", "nemo_debug_fail_after", "nemo_init", "nemo_shutdown",
    "nemo_model_create", "nemo_model_set_tensor", "nemo_model_synthesize", "nemo_model_finalize",
    "nemo_model_get_tensor", "nemo_model_destroy", "nemo_plan_create", "nemo_plan_run", "nemo_plan_run_device",
    "nemo_plan_profile", "nemo_profile_stage_count", "nemo_profile_stage_name", "nemo_plan_destroy",
    "nemo_plan_shape", "nemo_plan_read_buffer",
    "nemo_weight_create", "nemo_weight_destroy", "nemo_weight_matmul", "nemo_weight_matmul_static",
    "nemo_weight_dequantize", "nemo_dequantize",
    "nemo_requantize_q40", "nemo_probe_stream",
]


class NemoError(RuntimeError):
    """A libnemo call failed; ``status`` is the nemo_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class Dims(ctypes.Structure):
    """nemo_dims (include/nemo.h)."""
    _fields_ = [
        ("hidden", ctypes.c_int32), ("q_heads", ctypes.c_int32), ("kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("intermediate", ctypes.c_int32), ("layers", ctypes.c_int32),
        ("vocab", ctypes.c_int32), ("merge_after_layer", ctypes.c_int32), ("rms_epsilon", ctypes.c_float),
        ("rope_theta", ctypes.c_float), ("kv_stride_threshold", ctypes.c_int32), ("kv_stride", ctypes.c_int32),
        ("kv_dense_before_merge", ctypes.c_int32),
    ]


_lib = None


def load() -> ctypes.CDLL:
    """Load libnemo.so; raise if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libnemo.so not found at {LIB_PATH}; run __graft_entry__.build() first")
    L = ctypes.CDLL(LIB_PATH)
    vp, sz, i32, u64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_uint64
    u32p = ctypes.POINTER(ctypes.c_uint32)
    i64p = ctypes.POINTER(ctypes.c_int64)
    f32p = ctypes.POINTER(ctypes.c_float)
    pp = ctypes.POINTER(ctypes.c_void_p)
    sig = {
        "nemo_dims_reference": (None, [ctypes.POINTER(Dims)]),
        "nemo_last_error": (ctypes.c_char_p, []),
        "nemo_version": (ctypes.c_char_p, []),
        "nemo_debug_fail_after": (None, [i32]),
        "nemo_init": (i32, [i32, pp]),
        "nemo_shutdown": (i32, [vp]),
        "nemo_model_create": (i32, [vp, ctypes.POINTER(Dims), pp]),
        "nemo_model_set_tensor": (i32, [vp, ctypes.c_char_p, i32, i64p, i32, vp, sz]),
        "nemo_model_synthesize": (i32, [vp, u64, i32]),
        "nemo_model_finalize": (i32, [vp]),
        "nemo_model_get_tensor": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(i32), i64p, vp, ctypes.POINTER(sz)]),
        "nemo_model_destroy": (i32, [vp]),
        "nemo_plan_create": (i32, [vp, i32, i32, pp]),
        "nemo_plan_run": (i32, [vp, u32p, sz, u32p, sz, f32p]),
        "nemo_plan_run_device": (i32, [vp, vp, u32p, sz, vp, vp]),
        "nemo_plan_profile": (i32, [vp, u32p, sz, u32p, sz, f32p, i32]),
        "nemo_profile_stage_count": (i32, []),
        "nemo_profile_stage_name": (ctypes.c_char_p, [i32]),
        "nemo_plan_destroy": (i32, [vp]),
        "nemo_plan_shape": (i32, [vp, ctypes.POINTER(i32), ctypes.POINTER(i32), ctypes.POINTER(i32)]),
        "nemo_plan_read_buffer": (i32, [vp, ctypes.c_char_p, vp, ctypes.POINTER(sz)]),
        "nemo_weight_create": (i32, [vp, i32, i32, i32, vp, sz, pp]),
        "nemo_weight_destroy": (i32, [vp]),
        "nemo_weight_matmul": (i32, [vp, vp, i32, vp, i32, vp]),
        "nemo_weight_matmul_static": (i32, [vp, vp, i32, vp, i32, vp]),
        "nemo_weight_dequantize": (i32, [vp, vp, vp]),
        "nemo_dequantize": (i32, [i32, vp, ctypes.c_int64, vp, vp, vp]),
        "nemo_requantize_q40": (i32, [vp, i32, vp, sz, ctypes.c_int64, ctypes.c_int64, vp, sz]),
        "nemo_probe_stream": (i32, [vp, sz, i32, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(status: int) -> None:
    if status != NEMO_OK:
        msg = load().nemo_last_error().decode()
        raise NemoError(status, msg or STATUS_NAMES.get(status, str(status)))
