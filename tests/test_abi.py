"""The C ABI boundary without a GPU: libnemo.so loads, exports every function
include/nemo.h declares, the Python binding's constants equal the header's,
and the calls that need no device behave as documented."""
import ctypes
import os
import re

import pytest

import oracle
from nemo_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nemo.h")


def _header_text():
    with open(HEADER) as f:
        return f.read()


def _declared_functions():
    text = re.sub(r"/\*.*?\*/", "", _header_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:nemo_status|const char\*|void|int32_t)\s+(nemo_\w+)\s*\(", text, re.M)))


def _header_defines():
    return {k: int(v) for k, v in re.findall(r"#define\s+(NEMO_\w+)\s+(-?\d+)", _header_text())}


def test_binding_lists_every_declared_function():
    declared = _declared_functions()
    assert len(declared) >= 20
    assert sorted(_lib.EXPORTED) == declared


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [name for name in _declared_functions() if not hasattr(lib, name)]
    assert not missing, f"libnemo.so lacks {missing}"
    assert _lib.load() is not None


def test_constants_match_header():
    d = _header_defines()
    assert d["NEMO_OK"] == _lib.NEMO_OK == 0
    assert {d["NEMO_ERR_INVALID"], d["NEMO_ERR_MISSING"], d["NEMO_ERR_DEVICE"], d["NEMO_ERR_OOM"],
            d["NEMO_ERR_UNSUPPORTED"]} == set(_lib.STATUS_NAMES)
    assert (d["NEMO_TYPE_F32"], d["NEMO_TYPE_F16"], d["NEMO_TYPE_Q4_0"], d["NEMO_TYPE_Q4_K"], d["NEMO_TYPE_Q6_K"]) == (
        _lib.TYPE_F32, _lib.TYPE_F16, _lib.TYPE_Q4_0, _lib.TYPE_Q4_K, _lib.TYPE_Q6_K)
    # GGML type codes of src/gguf/types.ts:17-23
    assert (d["NEMO_TYPE_Q4_0"], d["NEMO_TYPE_Q4_K"], d["NEMO_TYPE_Q6_K"]) == (
        oracle.GGML_Q4_0, oracle.GGML_Q4_K, oracle.GGML_Q6_K)
    assert (d["NEMO_MATMUL_AUTO"], d["NEMO_MATMUL_GEMM"], d["NEMO_MATMUL_GEMV"], d["NEMO_MATMUL_TWO_PASS"]) == (
        _lib.MATMUL_AUTO, _lib.MATMUL_GEMM, _lib.MATMUL_GEMV, _lib.MATMUL_TWO_PASS)
    assert d["NEMO_STATIC_SCRATCH_BYTES"] == _lib.STATIC_SCRATCH_BYTES == 64 << 20


def test_host_only_calls():
    L = _lib.load()
    assert L.nemo_version().decode().startswith("libnemo")
    dims = _lib.Dims()
    L.nemo_dims_reference(ctypes.byref(dims))
    # the reference's constants, src/webgpu/model.ts:19-28
    assert (dims.hidden, dims.q_heads, dims.kv_heads, dims.head_dim, dims.intermediate, dims.layers, dims.vocab,
            dims.merge_after_layer) == (2048, 24, 8, 128, 6144, 16, 131072, 4)
    assert dims.rms_epsilon == pytest.approx(1e-5) and dims.rope_theta == 1e6
    # the profile stage names of src/webgpu/model.ts:198-211
    names = [L.nemo_profile_stage_name(i).decode() for i in range(L.nemo_profile_stage_count())]
    assert names == ["embedding_norm", "token_merge", "qkv", "rope_attention", "attention_output",
                     "post_attention_norm", "ffn_up_gate", "swiglu", "ffn_down", "post_ffn_norm", "pool"]
    assert L.nemo_profile_stage_name(99) == b""


def test_null_arguments_are_rejected_without_a_device():
    L = _lib.load()
    assert L.nemo_init(0, None) == 1
    assert b"null" in L.nemo_last_error()
    assert L.nemo_plan_destroy(None) == 0 and L.nemo_model_destroy(None) == 0


def test_product_fails_loudly_without_library(tmp_path, monkeypatch):
    """The host package has no CPU fallback: a missing libnemo.so raises."""
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libnemo.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError, match="libnemo.so not found"):
        _lib.load()
