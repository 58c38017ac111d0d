// Non-matmul kernels of the encoder pass (src/webgpu/ops.ts) on the ragged
// packed token layout. Host-side launch helpers; kernels in nemo_ops.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nemo_common.h"

namespace nemo {

// x[t, :] = table row ids[b * padded_seq + p] for packed row t = (b, p).
// table_type kF16 ([vocab, hidden] f16) or kQ6_K (raw GGUF rows).
hipError_t launch_embed(const uint32_t* ids, int padded_seq, const Ragged& rows, int table_type, const void* table,
                        int hidden, int vocab, uint16_t* x, hipStream_t stream);

// normalized = f16(f32(x) * rsqrt(mean(v^2) + eps) * w); with delta != null,
// v = f32(x) + f32(delta) is first stored into x (f16).
hipError_t launch_rmsnorm(uint16_t* x, const uint16_t* delta, const float* w, uint16_t* normalized, int rows,
                          int hidden, float eps, hipStream_t stream);

// The same with delta = f16(sum over s of partials[s][row][:]) (split order).
hipError_t launch_rmsnorm_partials(uint16_t* x, const float* partials, int splits, const float* w,
                                   uint16_t* normalized, int rows, int hidden, float eps, hipStream_t stream);
// The same with f16 partials (kEpiPartial16: each split's fp32 sum rounded
// once), widened and added in split order; splits 2 to 4.
hipError_t launch_rmsnorm_partials16(uint16_t* x, const uint16_t* partials, int splits, const float* w,
                                     uint16_t* normalized, int rows, int hidden, float eps, hipStream_t stream);

// Rotate adjacent pairs of the query and key heads of qkv into q [t, Hq, hd]
// and k [t, Hkv, hd]; position = row index within its request; table =
// [position][pair] (cos, sin) floats. The attention applies the same
// rotation itself; this writes it out.
hipError_t launch_rope(const uint16_t* qkv, int qkv_stride, const Ragged& rows, const float* table, int q_heads,
                       int kv_heads, int head_dim, uint16_t* q, uint16_t* k, hipStream_t stream);

// Bidirectional GQA attention per request on the QKV projection (row t:
// Hq query heads, Hkv key heads, Hkv value heads), queries and keys rotated
// by RoPE with `rope_table`. Without `ks`, each query tile rotates and
// stages the keys and values itself; with `ks` and `vts` (each room for
// kv_heads * keys_cap * head_dim halves, keys_cap >= attention_prep_keys) a
// first pass writes the rotated attended keys and the transposed values
// once, for long requests.
hipError_t launch_attention(const uint16_t* qkv, int qkv_stride, const float* rope_table, const Ragged& rows,
                            int q_heads, int kv_heads, int head_dim, int stride_threshold, int key_stride, uint16_t* out,
                            hipStream_t stream, uint16_t* ks = nullptr, uint16_t* vts = nullptr, int keys_cap = 0);
// Keys the prepared buffers hold for `rows` (each request's attended keys
// rounded up to 32).
int attention_prep_keys(const Ragged& rows, int stride_threshold, int key_stride);
// Keys that one staging round of the attention holds in ~72 KB of LDS (256
// at head_dim 64, 128 at 128). The plan prepares keys when a pass holds a
// request longer than that (whole requests at head_dim 128: 300 tokens 3 %
// faster than staging from the projection, 500 5 %, 16 x 500 4 %, 150
// equal; at head_dim 64, 16 x 150 tokens in one round is 0.8 % faster than
// prepared).
constexpr int attn_round_keys(int head_dim) { return 16384 / head_dim; }

// out[t, :F] = f16(silu(g) * u), g = gu[t, :F], u = gu[t, F:2F].
hipError_t launch_swiglu(const uint16_t* gu, int rows, int f, uint16_t* out, hipStream_t stream);

// Adjacent-state merge of every request from `src` rows to `dst` rows.
hipError_t launch_merge(const uint16_t* in, const Ragged& src, const Ragged& dst, int hidden, uint16_t* out,
                        hipStream_t stream);

// Mean over each request's rows, then L2 normalise; out float [count, hidden].
hipError_t launch_mean_pool(const uint16_t* norm, const Ragged& rows, int hidden, float* out, hipStream_t stream);

}  // namespace nemo
