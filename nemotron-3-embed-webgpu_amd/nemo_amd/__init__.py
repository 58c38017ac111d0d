"""MI355X-native Nemotron-3-Embed encoder runtime (host side).

The compute lives in libnemo.so (HIP, gfx950) behind the C ABI of
include/nemo.h; this package binds it and mirrors the reference's TypeScript
host interfaces: the embedding runtime and plan (runtime.py), the
micro-batching engine (engine.py) and the model pack format (prepacked.py).
"""
from . import _lib
from .engine import NemotronEmbeddingEngine
from .prepacked import build_prepacked_file, pack_q40_tile32, parse_prepacked_model, raw_tensor
from .runtime import (TYPE_F16, TYPE_F32, TYPE_Q4_0, TYPE_Q4_K, TYPE_Q6_K, Dims, HipContext, NemoError,
                      NemotronHipModel, NemotronHipPlan, QuantWeight, config_dims, contextual_merged_length,
                      dequantize_device, make_dims, reference_dims)

__all__ = [
    "NemotronEmbeddingEngine", "build_prepacked_file", "pack_q40_tile32", "parse_prepacked_model", "raw_tensor",
    "TYPE_F16", "TYPE_F32", "TYPE_Q4_0", "TYPE_Q4_K", "TYPE_Q6_K", "Dims", "HipContext", "NemoError",
    "NemotronHipModel", "NemotronHipPlan", "QuantWeight", "config_dims", "contextual_merged_length",
    "dequantize_device", "make_dims", "reference_dims", "_lib",
]
