"""CPU oracle for the Nemotron-3-Embed encoder hot path.

TEST INFRASTRUCTURE ONLY. Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline). The product path never calls it.

Two halves:

* the codec (``liboracle.so``, built from ``nemo_oracle.c``): the reference's
  CPU functions for binary16 and the GGML Q4_K / Q6_K / Q4_0 blocks, computed
  in double and stored to float32 exactly as the reference's JavaScript does;
* the float forward pass (numpy, below): the reference's WGSL graph restated
  with float64 arithmetic and binary16 storage at the same points as the
  reference (every activation buffer of src/webgpu/model.ts:83-94 is f16).

Pins — each function is checked against something other than its own formula
(tests/test_oracle_*.py):

=============================  ==============================================
half_to_float                  reference KATs tests/quantization.test.ts:5-9;
                               all 65,536 patterns vs numpy's IEEE binary16
float_to_half                  exact-rational nearest-with-ties-away rule on
                               every f16 midpoint and a dense float32 sample;
                               agrees with numpy RNE off ties
dequant_q4k                    reference KAT tests/quantization.test.ts:11-22;
                               the WGSL per-element decoder
                               (src/webgpu/quant-matmul.ts:38-60) on random
                               blocks; scale/min packing brute-forced over all
                               64x64 values and 8 slots
dequant_q6k                    reference KAT tests/quantization.test.ts:35-42;
                               the WGSL per-element decoder
                               (src/webgpu/quant-matmul.ts:111-127) on random
                               blocks; a scatter encoder round trip
dequant_q40 / quantize_q40     reference KATs tests/quantization.test.ts:24-59
pack_q40_tile32                reference KAT tests/prepacked-format.test.ts
contextual_merged_length       reference KAT tests/model-config.test.ts:5-15
rope_table                     YaRN correction dims (20, 37) at head_dim 128;
                               frequency 1 / (1/16) at the ends of the ramp;
                               |table| == 1
rope                           position 0 is identity; pair norms preserved;
                               two rotations compose (angle addition)
attention                      one key -> that value; equal keys -> mean of
                               values; a dominant key selects its value;
                               stride 3 == dense attention over keys 0,3,6..;
                               key permutation invariance; numpy softmax of a
                               brute-force float64 score matrix
rms_norm                       constant row closed form; scale invariance
swiglu                         silu(0)=0, silu(ln 3)=0.75 ln 3, large-g limit
merge                          constant rows stay constant; BOS row kept;
                               bins partition positions 1..S-1 when T <= S
mean_pool                      unit norm; a single repeated row -> its
                               direction
matmul                         fp64 dot of the reference CPU check
                               (src/main.ts:97-109) on integer-valued inputs
                               where float64 is exact
forward / forward_request      graph wiring (src/webgpu/model.ts:113-138,
                               154-168) by closed forms: zero projections ->
                               pool of the output-normalized merged rows;
                               power-of-two norm weights -> which norm follows
                               which residual add; a value-passthrough layer
                               after the merge -> the normalized stream is
                               merged as it is; RoPE positions restart after
                               the merge; the key set each layer attends
                               under the code's rule and README.md:26's
                               (kv_dense_before_merge), by uniform attention
                               over it; each pin fails on a planted wiring
                               mistake or the other key set
                               (tests/test_oracle_wiring*.py); batch
                               composition invariance
=============================  ==============================================
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def lib() -> ctypes.CDLL:
    """Load liboracle.so, building it with the committed Makefile if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    L = ctypes.CDLL(_LIB_PATH)
    u8p = ctypes.POINTER(ctypes.c_uint8)
    f32p = ctypes.POINTER(ctypes.c_float)
    f64p = ctypes.POINTER(ctypes.c_double)
    L.oracle_half_to_float.restype = ctypes.c_double
    L.oracle_half_to_float.argtypes = [ctypes.c_uint32]
    L.oracle_float_to_half.restype = ctypes.c_uint16
    L.oracle_float_to_half.argtypes = [ctypes.c_float]
    L.oracle_float_to_half_array.argtypes = [f32p, ctypes.c_int64, ctypes.POINTER(ctypes.c_uint16)]
    for name in ("oracle_dequant_q4k", "oracle_dequant_q6k", "oracle_dequant_q40"):
        getattr(L, name).argtypes = [u8p, ctypes.c_int64, f32p]
    L.oracle_q4k_scale_min.argtypes = [u8p, ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    L.oracle_quantize_q40_block.argtypes = [f32p, u8p]
    L.oracle_requantize_to_q40.restype = ctypes.c_int
    L.oracle_requantize_to_q40.argtypes = [u8p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, u8p]
    L.oracle_pack_q40_tile32.argtypes = [u8p, ctypes.c_int64, ctypes.c_int64, u8p]
    L.oracle_contextual_merged_length.restype = ctypes.c_int
    L.oracle_contextual_merged_length.argtypes = [ctypes.c_int]
    L.oracle_matmul_f64.argtypes = [f32p, f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, f64p]
    L.oracle_q4k_matmul_cpu.restype = ctypes.c_double
    L.oracle_q4k_matmul_cpu.argtypes = [u8p, f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, f32p, f64p]
    L.oracle_q4k_matmul_cpu_mt.restype = ctypes.c_double
    L.oracle_q4k_matmul_cpu_mt.argtypes = [u8p, f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                           f32p, f64p]
    _lib = L
    return L


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


# --------------------------------------------------------------------------
# Codec (C restatement; see nemo_oracle.c for the reference citations).
# --------------------------------------------------------------------------

BLOCK_BYTES = {12: 144, 14: 210, 2: 18}
BLOCK_VALUES = {12: 256, 14: 256, 2: 32}
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 2, 12, 14


def half_to_float(bits: int) -> float:
    """src/gguf/quantization.ts:2-9."""
    return lib().oracle_half_to_float(int(bits) & 0xFFFF)


def float_to_half(values) -> np.ndarray:
    """src/math/f16.ts:4-29 (toFloat16Bits): half-away-from-zero rounding."""
    v = np.ascontiguousarray(np.asarray(values, dtype=np.float32).reshape(-1))
    out = np.empty(v.shape, dtype=np.uint16)
    lib().oracle_float_to_half_array(_ptr(v, ctypes.c_float), v.size, _ptr(out, ctypes.c_uint16))
    return out


def dequantize(type_: int, raw, n_values: int | None = None) -> np.ndarray:
    """Dequantize consecutive GGML blocks to float32 (quantization.ts:19-74)."""
    raw = np.ascontiguousarray(np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw.reshape(-1).view(np.uint8))
    bb, bv = BLOCK_BYTES[type_], BLOCK_VALUES[type_]
    if raw.size % bb:
        raise ValueError(f"{raw.size} bytes is not a whole number of {bb}-byte blocks")
    nblocks = raw.size // bb
    out = np.empty(nblocks * bv, dtype=np.float32)
    fn = {12: lib().oracle_dequant_q4k, 14: lib().oracle_dequant_q6k, 2: lib().oracle_dequant_q40}[type_]
    fn(_ptr(raw, ctypes.c_uint8), nblocks, _ptr(out, ctypes.c_float))
    return out if n_values is None else out[:n_values]


def q4k_scale_min(scales: bytes, index: int) -> tuple[int, int]:
    """src/gguf/quantization.ts:11-17."""
    s = np.frombuffer(bytes(scales), dtype=np.uint8).copy()
    a, b = ctypes.c_int(), ctypes.c_int()
    lib().oracle_q4k_scale_min(_ptr(s, ctypes.c_uint8), index, ctypes.byref(a), ctypes.byref(b))
    return a.value, b.value


def quantize_q40_block(values) -> bytes:
    """src/gguf/quantization.ts:77-98."""
    v = np.ascontiguousarray(np.asarray(values, dtype=np.float32).reshape(32))
    out = np.zeros(18, dtype=np.uint8)
    lib().oracle_quantize_q40_block(_ptr(v, ctypes.c_float), _ptr(out, ctypes.c_uint8))
    return out.tobytes()


def requantize_to_q40(raw: bytes, type_: int, k: int, n: int) -> bytes:
    """src/gguf/quantization.ts:101-131."""
    if k % 256:
        raise ValueError(f"K={k} is not divisible by a K-quant block")
    src = np.frombuffer(bytes(raw), dtype=np.uint8).copy()
    expected = n * (k // BLOCK_VALUES[type_]) * BLOCK_BYTES[type_]
    if src.size != expected:
        raise ValueError(f"source has {src.size} bytes; expected {expected}")
    out = np.zeros(n * (k // 32) * 18, dtype=np.uint8)
    rc = lib().oracle_requantize_to_q40(_ptr(src, ctypes.c_uint8), type_, k, n, _ptr(out, ctypes.c_uint8))
    if rc:
        raise ValueError(f"requantize failed ({rc})")
    return out.tobytes()


def pack_q40_tile32(q40: bytes, k: int, n: int) -> bytes:
    """src/prepacked/format.ts:65-99 for one concatenated matrix."""
    src = np.frombuffer(bytes(q40), dtype=np.uint8).copy()
    out = np.zeros(((n + 31) // 32) * (k // 32) * 32 * 20, dtype=np.uint8)
    lib().oracle_pack_q40_tile32(_ptr(src, ctypes.c_uint8), k, n, _ptr(out, ctypes.c_uint8))
    return out.tobytes()


def contextual_merged_length(sequence: int) -> int:
    """src/webgpu/model.ts:30-32."""
    return lib().oracle_contextual_merged_length(int(sequence))


def q4k_matmul_cpu(w_raw: np.ndarray, x: np.ndarray, m: int, n: int, k: int) -> np.ndarray:
    """The reference CPU check (src/main.ts:97-104) for every output element:
    dequantize each Q4_K row, then a scalar float64 dot. Timed as the CPU
    baseline of the Q4_K dequant-matmul."""
    w = np.ascontiguousarray(w_raw.reshape(-1).view(np.uint8))
    xf = np.ascontiguousarray(x.astype(np.float32).reshape(m, k))
    scratch = np.empty(k, dtype=np.float32)
    out = np.empty((m, n), dtype=np.float64)
    lib().oracle_q4k_matmul_cpu(_ptr(w, ctypes.c_uint8), _ptr(xf, ctypes.c_float), m, n, k,
                                _ptr(scratch, ctypes.c_float), _ptr(out, ctypes.c_double))
    return out


def q4k_matmul_cpu_mt(w_raw: np.ndarray, x: np.ndarray, m: int, n: int, k: int, threads: int) -> np.ndarray:
    """q4k_matmul_cpu spread over `threads` OpenMP threads by weight row, each
    output computed by the same loop (same bits): the all-cores CPU baseline."""
    w = np.ascontiguousarray(w_raw.reshape(-1).view(np.uint8))
    xf = np.ascontiguousarray(x.astype(np.float32).reshape(m, k))
    scratch = np.empty(threads * k, dtype=np.float32)
    out = np.empty((m, n), dtype=np.float64)
    lib().oracle_q4k_matmul_cpu_mt(_ptr(w, ctypes.c_uint8), _ptr(xf, ctypes.c_float), m, n, k, int(threads),
                                   _ptr(scratch, ctypes.c_float), _ptr(out, ctypes.c_double))
    return out


# --------------------------------------------------------------------------
# Float forward pass (numpy restatement of src/webgpu/ops.ts + model.ts).
# Storage points round to binary16 with round-to-nearest-even, as the GPU's
# f16() conversion does; arithmetic between them is float64.
# --------------------------------------------------------------------------

def f16(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64).astype(np.float32).astype(np.float16)


@dataclass
class Dims:
    """Model shape. Reference constants: src/webgpu/model.ts:19-28."""
    hidden: int = 2048
    q_heads: int = 24
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 6144
    layers: int = 16
    vocab: int = 131072
    merge_after_layer: int = 4
    rms_epsilon: float = 1e-5
    rope_theta: float = 1_000_000.0
    kv_stride_threshold: int = 2048   # src/webgpu/ops.ts:258
    kv_stride: int = 3
    # 0: the code's rule (src/webgpu/ops.ts:258) in every layer; 1: the rule
    # README.md:26 states, every key in the layers before the merge.
    kv_dense_before_merge: int = 0

    @property
    def qkv_width(self) -> int:
        return (self.q_heads + 2 * self.kv_heads) * self.head_dim


REFERENCE_DIMS = Dims()
CONFIG_DIMS = Dims(q_heads=32, kv_heads=8, head_dim=64, intermediate=8192)

YARN_FACTOR = 16.0
YARN_ORIGINAL_CONTEXT = 16384.0
YARN_BETA_FAST = 32.0
YARN_BETA_SLOW = 1.0


def yarn_correction_range(head_dim: int, theta: float) -> tuple[int, int]:
    """src/webgpu/model.ts:97-99. The reference writes 128 (its head_dim);
    the correction-dimension formula is head_dim * ln(ctx / (beta 2 pi)) /
    (2 ln theta), so other head dims use their own."""
    corr = lambda beta: head_dim * math.log(YARN_ORIGINAL_CONTEXT / (beta * 2 * math.pi)) / (2 * math.log(theta))
    return math.floor(corr(YARN_BETA_FAST)), math.ceil(corr(YARN_BETA_SLOW))


def rope_table(sequence: int, head_dim: int, theta: float = 1e6) -> np.ndarray:
    """src/webgpu/model.ts:95-106: float32 [sequence, head_dim/2, 2] of
    (cos, sin)(position * theta^(-i/(head_dim/2)) * f_i), computed in double."""
    pairs = head_dim // 2
    low, high = yarn_correction_range(head_dim, theta)
    dims = np.arange(pairs, dtype=np.float64)
    ramp = 1 - np.minimum(1, np.maximum(0, (dims - low) / max(0.001, high - low)))
    freq = (1 / YARN_FACTOR) * (1 - ramp) + ramp
    inv = np.array([math.pow(theta, -d / pairs) for d in range(pairs)])
    pos = np.arange(sequence, dtype=np.float64)[:, None]
    angle = pos * inv[None, :] * freq[None, :]
    return np.stack([np.cos(angle), np.sin(angle)], axis=-1).astype(np.float32)


def embedding_lookup(table_type: int, table, ids: np.ndarray, hidden: int) -> np.ndarray:
    """src/webgpu/ops.ts:680-710: rows of a Q6_K (or f16) table, stored f16."""
    ids = np.asarray(ids, dtype=np.int64)
    if table_type == GGML_F16:
        t = np.asarray(table).view(np.float16).reshape(-1, hidden)
        return t[ids].copy()
    if table_type == GGML_Q6_K:
        row_bytes = hidden // 256 * 210
        raw = np.asarray(table).reshape(-1).view(np.uint8)
        rows = np.stack([raw[i * row_bytes:(i + 1) * row_bytes] for i in ids]) if len(ids) else np.zeros((0, row_bytes), np.uint8)
        return f16(dequantize(GGML_Q6_K, rows.reshape(-1)).reshape(len(ids), hidden))
    raise ValueError(f"unsupported embedding type {table_type}")


def rms_norm(x16: np.ndarray, weight: np.ndarray, eps: float, delta16: np.ndarray | None = None):
    """src/webgpu/ops.ts:21-56. Returns (x16 after the residual add, normalized16).
    The sum of squares uses the unrounded v = x + delta; the output scales the
    binary16-rounded x."""
    v = x16.astype(np.float64)
    if delta16 is not None:
        v = v + delta16.astype(np.float64)
    x_new = f16(v)
    inv = 1.0 / np.sqrt((v * v).sum(axis=-1, keepdims=True) / x16.shape[-1] + eps)
    return x_new, f16(x_new.astype(np.float64) * inv * weight.astype(np.float64)[None, :])


def matmul(x16: np.ndarray, w32: np.ndarray) -> np.ndarray:
    """Y = X W^T (src/webgpu/quant-matmul.ts: Y[m,n] = sum_k X[m,k] W[n,k]),
    float64 accumulate over the float32 dequantized weights, stored f16."""
    return f16(x16.astype(np.float64) @ w32.astype(np.float64).T)


def rope(qkv16: np.ndarray, positions: np.ndarray, table: np.ndarray, d: Dims):
    """src/webgpu/ops.ts:168-193: rotate adjacent pairs (2i, 2i+1) of every
    query and key head; q from columns [0, Hq*hd), k from [Hq*hd, +Hkv*hd)."""
    n = qkv16.shape[0]
    hd = d.head_dim
    q = qkv16[:, : d.q_heads * hd].astype(np.float64).reshape(n, d.q_heads, hd // 2, 2)
    k = qkv16[:, d.q_heads * hd:(d.q_heads + d.kv_heads) * hd].astype(np.float64).reshape(n, d.kv_heads, hd // 2, 2)
    cs = table[positions].astype(np.float64)  # [n, pairs, 2]
    c, s = cs[:, None, :, 0], cs[:, None, :, 1]

    def rot(t):
        e, o = t[..., 0], t[..., 1]
        return f16(np.stack([e * c - o * s, e * s + o * c], axis=-1))

    return rot(q).reshape(n, d.q_heads, hd), rot(k).reshape(n, d.kv_heads, hd)


def attention(q16: np.ndarray, k16: np.ndarray, v16: np.ndarray, d: Dims,
              stride_threshold: int = 2048, stride: int = 3) -> np.ndarray:
    """src/webgpu/ops.ts:213-293 (and :295-362) for one request of n valid
    tokens: softmax(q k^T * hd^-1/2 * temperature) v over keys 0, s, 2s, ...
    with s = 3 when n > 2048 else 1; GQA kv head = qh / (Hq / Hkv).
    The reference writes 0.08838834764831845 = 128^-1/2 (its head_dim)."""
    n = q16.shape[0]
    key_stride = stride if n > stride_threshold else 1
    keys = np.arange(0, n, key_stride)
    group = d.q_heads // d.kv_heads
    scale = 1.0 / math.sqrt(d.head_dim)
    qpos = np.arange(n, dtype=np.float64)
    temperature = np.where(qpos >= 16384, np.log(np.floor(qpos / 16384.0) + 1.0) * 0.1 + 1.0, 1.0)
    out = np.empty((n, d.q_heads, d.head_dim), dtype=np.float16)
    for h in range(d.q_heads):
        kvh = h // group
        qh = q16[:, h, :].astype(np.float64)
        kh = k16[keys, kvh, :].astype(np.float64)
        vh = v16[keys, kvh, :].astype(np.float64)
        s = (qh @ kh.T) * scale * temperature[:, None]
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[:, h, :] = f16((p @ vh) / p.sum(axis=1, keepdims=True))
    return out


def swiglu(gu16: np.ndarray, intermediate: int) -> np.ndarray:
    """src/webgpu/ops.ts:74-88: f16(g / (1 + e^-g) * u), g = cols [0, F), u = [F, 2F)."""
    g = gu16[:, :intermediate].astype(np.float64)
    u = gu16[:, intermediate:2 * intermediate].astype(np.float64)
    return f16(g / (1.0 + np.exp(-g)) * u)


def merge_bins(source_length: int, target_length: int) -> list[tuple[int, int]]:
    """src/webgpu/ops.ts:648-654: [start, end) of every output position."""
    bins = []
    for position in range(target_length):
        start, end = 0, 1
        if position > 0 and target_length > 1:
            st, tt = source_length - 1, target_length - 1
            start = 1 + ((position - 1) * st) // tt
            end = 1 + (position * st) // tt
            end = max(end, start + 1)
            end = min(end, source_length)
        bins.append((start, end))
    return bins


def merge(x16: np.ndarray, source_length: int, target_length: int) -> np.ndarray:
    """src/webgpu/ops.ts:629-660 for one request: BOS row kept, adjacent-state
    bin means, stored f16."""
    out = np.empty((target_length, x16.shape[1]), dtype=np.float16)
    for p, (start, end) in enumerate(merge_bins(source_length, target_length)):
        out[p] = f16(x16[start:end].astype(np.float64).mean(axis=0))
    return out


def mean_pool(norm16: np.ndarray, length: int) -> np.ndarray:
    """src/webgpu/ops.ts:596-615: mean over the first `length` rows, then
    times rsqrt(sum of squares) (no epsilon); float32 out."""
    mean = norm16[:length].astype(np.float64).mean(axis=0)
    return (mean / math.sqrt(float((mean * mean).sum()))).astype(np.float32)


@dataclass
class Model:
    """Dequantized weights of one model (float32) plus the raw embedding table.
    Names follow the reference's fused tensors (src/webgpu/model.ts:126-135)."""
    dims: Dims
    embedding_type: int
    embedding: np.ndarray               # raw Q6_K bytes or f16 [vocab, hidden]
    attn_norm: list                     # float32 [hidden] per layer
    ffn_norm: list
    output_norm: np.ndarray
    qkv: list = field(default_factory=list)       # float32 [qkv_width, hidden]
    attn_output: list = field(default_factory=list)
    gate_up: list = field(default_factory=list)   # float32 [2F, hidden]
    down: list = field(default_factory=list)      # float32 [hidden, F]


def forward_request(model: Model, ids: np.ndarray, trace: dict | None = None) -> np.ndarray:
    """src/webgpu/model.ts:146-176 for one request of len(ids) valid tokens
    (the reference's padded rows never reach a valid output, so they are not
    computed). Returns the float32 [hidden] embedding."""
    d = model.dims
    S = len(ids)
    T = contextual_merged_length(S)
    n = S
    x = embedding_lookup(model.embedding_type, model.embedding, ids, d.hidden)
    _, norm = rms_norm(x, model.attn_norm[0], d.rms_epsilon)
    if trace is not None:
        trace["embedding"] = x.copy()
        trace["norm0"] = norm.copy()
    table = rope_table(max(S, 1), d.head_dim, d.rope_theta)
    hd, Hq, Hkv = d.head_dim, d.q_heads, d.kv_heads
    for layer in range(d.layers):
        if layer == d.merge_after_layer:
            x = merge(x, S, T)
            norm = merge(norm, S, T)
            n = T
        qkv = matmul(norm, model.qkv[layer])
        q, k = rope(qkv, np.arange(n), table, d)
        v = qkv[:, (Hq + Hkv) * hd:].reshape(n, Hkv, hd)
        dense = d.kv_dense_before_merge and layer < d.merge_after_layer
        att = attention(q, k, v, d, n if dense else d.kv_stride_threshold, d.kv_stride).reshape(n, Hq * hd)
        delta_o = matmul(att, model.attn_output[layer])
        x, norm = rms_norm(x, model.ffn_norm[layer], d.rms_epsilon, delta_o)
        gate_up = matmul(norm, model.gate_up[layer])
        ffn = swiglu(gate_up, d.intermediate)
        delta = matmul(ffn, model.down[layer])
        nxt = model.attn_norm[layer + 1] if layer + 1 < d.layers else model.output_norm
        x, norm = rms_norm(x, nxt, d.rms_epsilon, delta)
        if trace is not None:
            for key, val in (("qkv", qkv), ("q", q), ("k", k), ("attention", att), ("gate_up", gate_up),
                             ("ffn", ffn), ("delta", delta), ("x", x), ("norm", norm)):
                trace.setdefault(key, []).append(val.copy())
    if d.merge_after_layer == d.layers:
        # Shorter models than the reference's 16 layers may merge after the
        # last layer; the pool always reads the merged normalized stream.
        norm = merge(norm, S, T)
    return mean_pool(norm, T)


def forward(model: Model, ids: np.ndarray, lengths: np.ndarray) -> np.ndarray:
    """EmbeddingPlan.run (src/webgpu/model.ts:146-176): ids [batch * sequence]
    padded after each request, lengths [batch] -> float32 [batch, hidden]."""
    lengths = np.asarray(lengths, dtype=np.int64)
    B = len(lengths)
    S = len(ids) // B
    return np.stack([forward_request(model, np.asarray(ids[b * S:b * S + lengths[b]]), None) for b in range(B)])
