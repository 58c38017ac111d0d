// Elementwise, attention, merge and pooling kernels of the encoder pass for
// gfx950, on the ragged packed token layout (request b owns rows
// [start[b], start[b+1]); no padding rows exist).
//
// Semantics follow src/webgpu/ops.ts (cited per kernel). Storage is f16 as in
// the reference's buffers; arithmetic is fp32.
#include <algorithm>

#include "nemo_blocks.h"
#include "nemo_common.h"
#include "nemo_ops.h"
#include "nemo_quant.h"

namespace nemo {

__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Block-wide sum over blockDim.x (a multiple of 64, at most 1024) threads.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
  v = warp_sum(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, waves = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float t = lane < waves ? scratch[lane] : 0.f;
  return warp_sum(t);
}

// ---------------------------------------------------------------------------
// Embedding lookup (src/webgpu/ops.ts:680-710).
// ---------------------------------------------------------------------------

__global__ void embed_f16_kernel(const uint32_t* __restrict__ ids, int padded_seq, Ragged rows,
                                 const uint16_t* __restrict__ table, int hidden, int vocab, uint16_t* __restrict__ x) {
  const int t = blockIdx.x;
  const int b = ragged_find(rows, t);
  uint32_t id = ids[(size_t)b * padded_seq + (t - rows.start[b])];
  if (id >= (uint32_t)vocab) id = 0;  // out-of-range ids are rejected on the host; never read past the table
  const u32x4* src = (const u32x4*)(table + (size_t)id * hidden);
  u32x4* dst = (u32x4*)(x + (size_t)t * hidden);
  for (int i = threadIdx.x; i < hidden / 8; i += blockDim.x) dst[i] = src[i];
}

// Q6_K table row: f16(d * scale * (q - 32)) (ops.ts:689-703); thread per
// 32 values (half, quadrant) of one 256-value block of the row.
__global__ void embed_q6k_kernel(const uint32_t* __restrict__ ids, int padded_seq, Ragged rows,
                                 const uint8_t* __restrict__ table, int hidden, int vocab, uint16_t* __restrict__ x) {
  const int t = blockIdx.x;
  const int b = ragged_find(rows, t);
  uint32_t id = ids[(size_t)b * padded_seq + (t - rows.start[b])];
  if (id >= (uint32_t)vocab) id = 0;
  const int blocks = hidden / 256;
  for (int w = threadIdx.x; w < blocks * 8; w += blockDim.x) {
    const int blk = w >> 3, c = w & 7, half = c >> 2, quadrant = c & 3;
    const uint8_t* p = table + ((size_t)id * blocks + blk) * 210;
    const float d = h2f((uint16_t)(p[208] | (p[209] << 8)));
    uint16_t* o = x + (size_t)t * hidden + blk * 256 + 128 * half + 32 * quadrant;
    for (int lane = 0; lane < 32; lane += 2) {
      uint32_t packed = 0;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int l = lane + e;
        const uint32_t low = p[64 * half + l + 32 * (quadrant & 1)];
        const uint32_t lowq = quadrant >= 2 ? (low >> 4) : (low & 15u);
        const uint32_t high = (p[128 + 32 * half + l] >> (2 * quadrant)) & 3u;
        const int scale = (int8_t)p[192 + 8 * half + (l >> 4) + 2 * quadrant];
        packed |= (uint32_t)f2h((d * (float)scale) * (float)((int)(lowq | (high << 4)) - 32)) << (16 * e);
      }
      *(uint32_t*)(o + lane) = packed;
    }
  }
}

hipError_t launch_embed(const uint32_t* ids, int padded_seq, const Ragged& rows, int table_type, const void* table,
                        int hidden, int vocab, uint16_t* x, hipStream_t stream) {
  const int total = rows.start[rows.count];
  if (total <= 0) return hipSuccess;
  if (table_type == kF16)
    embed_f16_kernel<<<total, 256, 0, stream>>>(ids, padded_seq, rows, (const uint16_t*)table, hidden, vocab, x);
  else if (table_type == kQ6_K)
    embed_q6k_kernel<<<total, 64, 0, stream>>>(ids, padded_seq, rows, (const uint8_t*)table, hidden, vocab, x);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Residual add + RMSNorm (src/webgpu/ops.ts:21-56). One workgroup per row,
// 8 values (16 bytes) per thread and pass. The residual delta is either an
// f16 row or the fp32 split-K partial sums of the producing GEMM, summed in
// split order and rounded to f16 (the reference's delta buffer is f16).
// ---------------------------------------------------------------------------

// DELTA = 0: normalize x; -1: x += f16 delta first; S >= 1: x += the sum of
// S fp32 K-split partials first (all 2 S loads issued before the first add,
// added in split order); kAnySplits: the same for a run-time count.
constexpr int kAnySplits = 1000;

// H16: the partials are f16 (kEpiPartial16), widened to fp32 before the sum.
template <int DELTA, bool H16 = false>
__global__ __launch_bounds__(256) void rmsnorm_kernel(uint16_t* __restrict__ x, const void* __restrict__ delta,
                                                      int splits, int rows, const float* __restrict__ w,
                                                      uint16_t* __restrict__ out, int hidden, float eps) {
  __shared__ float scratch[16];
  const size_t base = (size_t)blockIdx.x * hidden;
  float sum = 0.f;
  for (int c = threadIdx.x * 8; c < hidden; c += blockDim.x * 8) {
    half8v xv = *(const half8v*)(x + base + c);
    if constexpr (DELTA != 0) {
      float dv[8];
      if constexpr (DELTA > 0 && H16) {
        const uint16_t* p = (const uint16_t*)delta + base + c;
        const size_t slice = (size_t)rows * hidden;
        half8v ph[DELTA];
#pragma unroll
        for (int s = 0; s < DELTA; ++s) ph[s] = *(const half8v*)(p + s * slice);
        float a[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = (float)ph[0][i];
#pragma unroll
        for (int s = 1; s < DELTA; ++s)
#pragma unroll
          for (int i = 0; i < 8; ++i) a[i] += (float)ph[s][i];
#pragma unroll
        for (int i = 0; i < 8; ++i) dv[i] = (float)(half_t)a[i];
      } else if constexpr (DELTA > 0) {
        const float* p = (const float*)delta + base + c;
        const size_t slice = (size_t)rows * hidden;
        float4v a, b;
        if constexpr (DELTA == kAnySplits) {
          a = *(const float4v*)p, b = *(const float4v*)(p + 4);
          for (int s = 1; s < splits; ++s) {
            a += *(const float4v*)(p + s * slice);
            b += *(const float4v*)(p + s * slice + 4);
          }
        } else {
          float4v pa[DELTA], pb[DELTA];
#pragma unroll
          for (int s = 0; s < DELTA; ++s) {
            pa[s] = *(const float4v*)(p + s * slice);
            pb[s] = *(const float4v*)(p + s * slice + 4);
          }
          a = pa[0], b = pb[0];
#pragma unroll
          for (int s = 1; s < DELTA; ++s) a += pa[s], b += pb[s];
        }
        const float raw[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) dv[i] = (float)(half_t)raw[i];
      } else {
        const half8v d16 = *(const half8v*)((const uint16_t*)delta + base + c);
#pragma unroll
        for (int i = 0; i < 8; ++i) dv[i] = (float)d16[i];
      }
      half8v stored;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = (float)xv[i] + dv[i];
        sum += v * v;  // the unrounded sum, as ops.ts:39-40
        stored[i] = (half_t)v;
      }
      *(half8v*)(x + base + c) = stored;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) sum += (float)xv[i] * (float)xv[i];
    }
  }
  const float total = block_sum(sum, scratch);
  const float inv = 1.0f / sqrtf(total / (float)hidden + eps);
  for (int c = threadIdx.x * 8; c < hidden; c += blockDim.x * 8) {
    const half8v xv = *(const half8v*)(x + base + c);
    const float4v w0 = *(const float4v*)(w + c), w1 = *(const float4v*)(w + c + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    half8v o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (half_t)(((float)xv[i] * inv) * wv[i]);
    *(half8v*)(out + base + c) = o;
  }
}

hipError_t launch_rmsnorm(uint16_t* x, const uint16_t* delta, const float* w, uint16_t* normalized, int rows,
                          int hidden, float eps, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  if (delta)
    rmsnorm_kernel<-1><<<rows, 256, 0, stream>>>(x, delta, 1, rows, w, normalized, hidden, eps);
  else
    rmsnorm_kernel<0><<<rows, 256, 0, stream>>>(x, nullptr, 1, rows, w, normalized, hidden, eps);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_partials(uint16_t* x, const float* partials, int splits, const float* w,
                                   uint16_t* normalized, int rows, int hidden, float eps, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  if (splits < 1) return hipErrorInvalidValue;
#define NEMO_NORM(S) rmsnorm_kernel<S><<<rows, 256, 0, stream>>>(x, partials, splits, rows, w, normalized, hidden, eps)
  switch (splits) {
    case 1: NEMO_NORM(1); break;
    case 2: NEMO_NORM(2); break;
    case 3: NEMO_NORM(3); break;
    case 4: NEMO_NORM(4); break;
    case 6: NEMO_NORM(6); break;
    case 8: NEMO_NORM(8); break;
    case 12: NEMO_NORM(12); break;
    case 16: NEMO_NORM(16); break;
    default: NEMO_NORM(kAnySplits); break;
  }
#undef NEMO_NORM
  return hipGetLastError();
}

hipError_t launch_rmsnorm_partials16(uint16_t* x, const uint16_t* partials, int splits, const float* w,
                                     uint16_t* normalized, int rows, int hidden, float eps, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
#define NEMO_NORM16(S) \
  rmsnorm_kernel<S, true><<<rows, 256, 0, stream>>>(x, partials, splits, rows, w, normalized, hidden, eps)
  switch (splits) {
    case 2: NEMO_NORM16(2); break;
    case 3: NEMO_NORM16(3); break;
    case 4: NEMO_NORM16(4); break;
    default: return hipErrorInvalidValue;
  }
#undef NEMO_NORM16
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Pairwise RoPE (src/webgpu/ops.ts:168-193): (e, o) -> (e c - o s, e s + o c)
// with (c, s) = table[position][pair], on 8 consecutive values of a head (4
// pairs) at a time. The attention kernel applies it as it loads queries and
// keys from the QKV projection; rope_kernel writes the rotated heads out
// (one workgroup per token) for inspection of the stage.
// ---------------------------------------------------------------------------

// v = values 2p0 .. 2p0 + 7 of a head; (a, b) = the table's (c, s) of its 4
// pairs (table row + 2 p0, 8 floats).
__device__ __forceinline__ half8v rope8(half8v v, float4v a, float4v b) {
  const float c[4] = {a[0], a[2], b[0], b[2]}, sn[4] = {a[1], a[3], b[1], b[3]};
  half8v r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float e = (float)v[2 * j], o = (float)v[2 * j + 1];
    r[2 * j] = (half_t)(e * c[j] - o * sn[j]);
    r[2 * j + 1] = (half_t)(e * sn[j] + o * c[j]);
  }
  return r;
}
__device__ __forceinline__ half8v rope8(half8v v, const float* __restrict__ cs) {
  return rope8(v, *(const float4v*)cs, *(const float4v*)(cs + 4));
}

__global__ __launch_bounds__(256) void rope_kernel(const uint16_t* __restrict__ qkv, int qkv_stride, Ragged rows,
                                                   const float* __restrict__ table, int q_heads, int kv_heads,
                                                   int head_dim, uint16_t* __restrict__ q, uint16_t* __restrict__ k) {
  const int t = blockIdx.x;
  const int b = ragged_find(rows, t);
  const int pos = t - rows.start[b];
  const int chunks = head_dim / 8, total = (q_heads + kv_heads) * chunks;
  const float* trow = table + (size_t)pos * head_dim;
  for (int i = threadIdx.x; i < total; i += blockDim.x) {
    const int head = i / chunks, d = 8 * (i - head * chunks);
    const half8v r = rope8(*(const half8v*)(qkv + (size_t)t * qkv_stride + head * head_dim + d), trow + d);
    if (head < q_heads)
      *(half8v*)(q + ((size_t)t * q_heads + head) * head_dim + d) = r;
    else
      *(half8v*)(k + ((size_t)t * kv_heads + (head - q_heads)) * head_dim + d) = r;
  }
}

hipError_t launch_rope(const uint16_t* qkv, int qkv_stride, const Ragged& rows, const float* table, int q_heads,
                       int kv_heads, int head_dim, uint16_t* q, uint16_t* k, hipStream_t stream) {
  const int total = rows.start[rows.count];
  if (total <= 0) return hipSuccess;
  if (head_dim % 8) return hipErrorInvalidValue;
  rope_kernel<<<total, 256, 0, stream>>>(qkv, qkv_stride, rows, table, q_heads, kv_heads, head_dim, q, k);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Bidirectional GQA flash attention on MFMA (src/webgpu/ops.ts:213-293,
// 295-362), reading queries, keys and values from the QKV projection [t,
// (Hq + 2 Hkv) hd] and rotating queries and keys (RoPE, position = row
// within the request) as it loads them. For request b with n valid rows,
// query i attends keys
// 0, s, 2s, ... < n (s = key_stride if n > stride_threshold, else 1) with
// scores q.k * head_dim^-1/2 * temperature(i), temperature = 1 + 0.1
// ln(floor(i / 16384) + 1) for i >= 16384 (ops.ts:241); online softmax in
// fp32, output f16.
//
// Workgroup = one request, one KV head, 32 queries; wave w handles query
// head kv_head * group + w, so the staged K/V tiles serve the whole GQA
// group. Scores are computed transposed, S^T = K Q^T (32 keys x 32 queries
// per v_mfma_f32_32x32x16_f16), so lane l always holds query l%32: the
// softmax max/sum are per-lane scalars (one cross-half exchange), and the
// rescale of the output accumulators is a per-lane multiply. The output is
// accumulated transposed too, O^T = V^T P^T, with V staged transposed in LDS
// and P fed from the score registers: the MFMA's k index is mapped to the
// keys a lane holds (the key order of a sum is free; A and B agree on it).
// ---------------------------------------------------------------------------

constexpr int kAttnQ = 32, kAttnKeys = 32;

__device__ __forceinline__ int attn_keys(int n, int stride_threshold, int key_stride_long) {
  const int s = n > stride_threshold ? key_stride_long : 1;
  return (n + s - 1) / s;
}

// Long requests: one pass per layer writes each request's attended keys,
// rotated, as K_s [kv head][key][hd] and its values transposed as
// V^T_s [kv head][hd][key] (keys of request b from 32 * (sum over earlier
// requests of ceil(keys / 32)), zero past the last key). The attention's
// query tiles (157 of them at 5000 tokens) then stage both with 16-byte
// loads and stores instead of rotating every key again and transposing V
// with 2-byte LDS stores. Workgroup = 32 keys of one kv head.
template <int HD>
__global__ __launch_bounds__(256) void attention_prep_kernel(const uint16_t* __restrict__ qkv, int qkv_stride,
                                                             const float* __restrict__ table, Ragged rows,
                                                             int q_heads, int kv_heads, int stride_threshold,
                                                             int key_stride_long, int keys_cap,
                                                             uint16_t* __restrict__ ks, uint16_t* __restrict__ vts) {
  __shared__ __attribute__((aligned(16))) half_t sv[kAttnKeys * (HD + 8)];
  int b = 0, blk = blockIdx.x;
  for (; b < rows.count; ++b) {
    const int blocks = (attn_keys(rows.start[b + 1] - rows.start[b], stride_threshold, key_stride_long) + 31) / 32;
    if (blk < blocks) break;
    blk -= blocks;
  }
  if (b >= rows.count) return;
  const int row0 = rows.start[b], n = rows.start[b + 1] - row0;
  const int key_stride = n > stride_threshold ? key_stride_long : 1;
  const int n_keys = (n + key_stride - 1) / key_stride;
  const int kvh = blockIdx.y, g0 = kAttnKeys * blockIdx.x;  // first key of this block in the buffers
  const uint16_t* kbase = qkv + (q_heads + kvh) * HD;
  const uint16_t* vbase = qkv + (q_heads + kv_heads + kvh) * HD;
  for (int i = threadIdx.x; i < kAttnKeys * HD / 8; i += blockDim.x) {
    const int j = i / (HD / 8), c = (i % (HD / 8)) * 8, key = kAttnKeys * blk + j;
    half8v kv = {}, vv = {};
    if (key < n_keys) {
      const int kpos = key * key_stride;
      const size_t trow = (size_t)(row0 + kpos) * qkv_stride;
      kv = rope8(*(const half8v*)(kbase + trow + c), table + (size_t)kpos * HD + c);
      vv = *(const half8v*)(vbase + trow + c);
    }
    *(half8v*)(ks + ((size_t)kvh * keys_cap + g0 + j) * HD + c) = kv;
    *(half8v*)&sv[j * (HD + 8) + c] = vv;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < HD * kAttnKeys / 8; i += blockDim.x) {
    const int d = i / (kAttnKeys / 8), k0 = (i % (kAttnKeys / 8)) * 8;
    half8v col;
#pragma unroll
    for (int r = 0; r < 8; ++r) col[r] = sv[(k0 + r) * (HD + 8) + d];
    *(half8v*)(vts + ((size_t)kvh * HD + d) * keys_cap + g0 + k0) = col;
  }
}

// Fewest threads per block that the prepared path's staging supports.
constexpr int attn_prep_min_threads(int hd) { return hd == 128 ? 128 : 64; }

template <int HD, bool PREP>
__global__ __launch_bounds__(512) void attention_kernel(const uint16_t* __restrict__ qkv, int qkv_stride,
                                                        const float* __restrict__ table, Ragged rows, int q_heads,
                                                        int kv_heads, int stride_threshold, int key_stride_long,
                                                        const uint16_t* __restrict__ ks,
                                                        const uint16_t* __restrict__ vts, int keys_cap, int sb_keys,
                                                        uint16_t* __restrict__ out) {
  constexpr int KP = HD + 8;  // padded K row (halves)
  constexpr int DC = HD / 16; // 16-wide d chunks of the score MFMAs
  constexpr int DB = HD / 32; // 32-wide d blocks of the output
  // sb_keys (a multiple of 32) keys are staged per round: sK [sb_keys][KP],
  // sVt [HD][VP].
  extern __shared__ __attribute__((aligned(16))) uint8_t attn_lds[];
  const int VP = sb_keys + 8;
  half_t* sK = (half_t*)attn_lds;
  half_t* sVt = sK + sb_keys * KP;
  int b = 0, tile = blockIdx.x, koff = 0;  // koff: the request's first key in K_s / V^T_s
  for (; b < rows.count; ++b) {
    const int n = rows.start[b + 1] - rows.start[b];
    const int tiles = (n + kAttnQ - 1) / kAttnQ;
    if (tile < tiles) break;
    tile -= tiles;
    koff += kAttnKeys * ((attn_keys(n, stride_threshold, key_stride_long) + kAttnKeys - 1) / kAttnKeys);
  }
  if (b >= rows.count) return;
  const int row0 = rows.start[b];
  const int n = rows.start[b + 1] - row0;
  const int kvh = blockIdx.y;
  const int group = q_heads / kv_heads;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, hl = lane >> 5;
  const int h = kvh * group + wave;
  const int qi = tile * kAttnQ + (lane & 31);
  const int key_stride = n > stride_threshold ? key_stride_long : 1;
  const int n_keys = (n + key_stride - 1) / key_stride;
  const float temperature = qi >= 16384 ? logf(floorf((float)qi / 16384.0f) + 1.0f) * 0.1f + 1.0f : 1.0f;
  const float scale2 = (1.0f / sqrtf((float)HD)) * temperature * 1.4426950408889634f;

  half8v qf[DC];
  {
    const int qpos = min(qi, n - 1);
    const uint16_t* qp = qkv + (size_t)(row0 + qpos) * qkv_stride + h * HD + 8 * hl;
    const float* cs = table + (size_t)qpos * HD + 8 * hl;
#pragma unroll
    for (int c = 0; c < DC; ++c) qf[c] = rope8(*(const half8v*)(qp + 16 * c), cs + 16 * c);
  }
  const uint16_t* kbase = qkv + (q_heads + kvh) * HD;
  const uint16_t* vbase = qkv + (q_heads + kv_heads + kvh) * HD;
  float16v o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  // m: the query's reference maximum (log2 units, scaled); lsum: the sum of
  // this half's probabilities (the two halves' are added at the end).
  float m = -INFINITY, lsum = 0.f;

  // One block of kAttnKeys staged keys from key kb of cK [keys][KP] and
  // cV [HD][vp]; keys at or past `staged` are masked.
  //
  // Probabilities are taken against a reference maximum m that is raised
  // only when a query's block maximum exceeds it by more than 2^8 (a wave
  // vote): p = 2^(s - m) <= 256 then, exact enough in f16 and far from
  // overflow in the fp32 sums, and the common block needs no cross-lane
  // exchange, no rescale of the accumulators and no 2^(m - m') of its own.
  // The result is the softmax all the same: numerator and denominator share
  // the reference.
  auto block = [&](const half_t* cK, const half_t* cV, int vp, int kb, int staged) {
    // S^T block: lane holds query l%32, key kb + 8(r/4) + 4hl + r%4.
    float16v s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const half8v a = *(const half8v*)&cK[(kb + (lane & 31)) * KP + 16 * c + 8 * hl];
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[c], s, 0, 0, 0);
    }
    if (kb + kAttnKeys > staged) {  // the request's last keys: mask past its end
      asm volatile("");  // keeps this rare path a branch (not computed and selected every block)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (kb + 8 * (r >> 2) + 4 * hl + (r & 3) >= staged) s[r] = -INFINITY;
    }
    float bm = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) bm = fmaxf(bm, s[r]);
    bm *= scale2;  // scale2 > 0: the maximum of the scaled scores
    if (__builtin_amdgcn_ballot_w64(bm > m + 8.0f)) {
      asm volatile("");
      const float mn = fmaxf(m, fmaxf(bm, __shfl_xor(bm, 32, 64)));
      const float alpha = __builtin_amdgcn_exp2f(m - mn);
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      m = mn;
    }
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      // v_exp_f32 itself: results below 2^-126 (flushed) add nothing to the sums
      p[r] = __builtin_amdgcn_exp2f(fmaf(s[r], scale2, -m));
      lsum += p[r];
    }
    // O^T += V^T P^T over two 16-key chunks: MFMA k slot 8hl + e of chunk c2
    // is key 16c2 + 8(e/4) + 4hl + e%4 = score register 8c2 + e.
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
      const half8v pb = to_half8(p + 8 * c2);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const half_t* vr = &cV[(32 * db + (lane & 31)) * vp + kb + 16 * c2 + 4 * hl];
        const half4v v0 = *(const half4v*)vr;
        const half4v v1 = *(const half4v*)(vr + 8);
        const half8v a = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb, o[db], 0, 0, 0);
      }
    }
  };
  if constexpr (PREP) {
    // Rounds of kAttnKeys keys from K_s / V^T_s (zero-padded to whole
    // rounds), double-buffered in LDS: each thread's 16-byte chunks of
    // round r + 2 are loaded into registers while round r is computed and
    // stored after it, so one barrier per round remains and a round's loads
    // have a whole round to land.
    constexpr int RK = kAttnKeys, VPR = RK + 8;
    constexpr int KCH = RK * HD / 8, VCH = HD * (RK / 8);  // chunks of a round's K rows and V^T rows
    constexpr int U = KCH / attn_prep_min_threads(HD);      // slots per thread at the smallest block
    static_assert(KCH == VCH && KCH % attn_prep_min_threads(HD) == 0, "K and V^T chunks share the slots");
    constexpr int STAGE = RK * KP + HD * VPR;               // halves per LDS stage
    const int rounds = (n_keys + RK - 1) / RK;
    const uint16_t* kp = ks + ((size_t)kvh * keys_cap + koff) * HD;
    const uint16_t* vp0 = vts + (size_t)kvh * HD * keys_cap + koff;
    half8v kr[U], vr[U];
    auto load = [&](int r) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = threadIdx.x + u * blockDim.x;
        if (i < KCH) {
          kr[u] = *(const half8v*)(kp + (size_t)r * RK * HD + 8 * i);
          const int d = i / (RK / 8), k0 = (i % (RK / 8)) * 8;
          vr[u] = *(const half8v*)(vp0 + (size_t)d * keys_cap + r * RK + k0);
        }
      }
    };
    auto store = [&](int stage) {
      half_t* dK = sK + stage * STAGE;
      half_t* dV = dK + RK * KP;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = threadIdx.x + u * blockDim.x;
        if (i < KCH) {
          *(half8v*)&dK[(i / (HD / 8)) * KP + (i % (HD / 8)) * 8] = kr[u];
          *(half8v*)&dV[(i / (RK / 8)) * VPR + (i % (RK / 8)) * 8] = vr[u];
        }
      }
    };
    load(0);
    store(0);
    if (rounds > 1) load(1);
    __syncthreads();
    for (int r = 0; r < rounds; ++r) {
      const half_t* cK = sK + (r & 1) * STAGE;
      block(cK, cK + RK * KP, VPR, 0, min(RK, n_keys - r * RK));
      if (r + 1 < rounds) {
        store((r + 1) & 1);
        if (r + 2 < rounds) load(r + 2);
      }
      __syncthreads();
    }
  } else {
    for (int sb = 0; sb < n_keys; sb += sb_keys) {
      const int staged = min(sb_keys, n_keys - sb);
      __syncthreads();
      // 16-byte chunks of the staged keys (rows past `staged` up to the
      // next multiple of 32 are zero), in batches of 4 per thread with every
      // load of a batch issued before the first is used.
      const int chunks = (staged + 31) / 32 * 32 * HD / 8;
      for (int i0 = threadIdx.x; i0 < chunks; i0 += 4 * blockDim.x) {
        half8v kr[4], vr[4];
        float4v ca[4], cb[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = i0 + u * blockDim.x, j = i / (HD / 8), c = (i % (HD / 8)) * 8;
          kr[u] = half8v{};
          vr[u] = half8v{};
          ca[u] = cb[u] = float4v{0.f, 0.f, 0.f, 0.f};
          if (i < chunks && j < staged) {
            const int kpos = (sb + j) * key_stride;
            const size_t trow = (size_t)(row0 + kpos) * qkv_stride;
            kr[u] = *(const half8v*)(kbase + trow + c);
            vr[u] = *(const half8v*)(vbase + trow + c);
            const float* cs = table + (size_t)kpos * HD + c;
            ca[u] = *(const float4v*)cs;
            cb[u] = *(const float4v*)(cs + 4);
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = i0 + u * blockDim.x, j = i / (HD / 8), c = (i % (HD / 8)) * 8;
          if (i < chunks) {
            *(half8v*)&sK[j * KP + c] = rope8(kr[u], ca[u], cb[u]);
#pragma unroll
            for (int e = 0; e < 8; ++e) sVt[(c + e) * VP + j] = vr[u][e];
          }
        }
      }
      __syncthreads();
      for (int kb = 0; kb < staged; kb += kAttnKeys) block(sK, sVt, VP, kb, staged);
    }
  }
  lsum += __shfl_xor(lsum, 32, 64);  // the two halves' keys (same references)
  if (qi >= n) return;
  const float inv = 1.0f / lsum;
  uint16_t* op = out + ((size_t)(row0 + qi) * q_heads + h) * HD;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // registers 4j..4j+3 hold d = 32db + 8j + 4hl + 0..3 (contiguous)
      const half4v hv = {(half_t)(o[db][4 * j] * inv), (half_t)(o[db][4 * j + 1] * inv),
                         (half_t)(o[db][4 * j + 2] * inv), (half_t)(o[db][4 * j + 3] * inv)};
      *(half4v*)(op + 32 * db + 8 * j + 4 * hl) = hv;
    }
}

int attention_prep_keys(const Ragged& rows, int stride_threshold, int key_stride) {
  int keys = 0;
  for (int b = 0; b < rows.count; ++b) {
    const int n = rows.start[b + 1] - rows.start[b];
    const int s = n > stride_threshold ? key_stride : 1;
    keys += kAttnKeys * (((n + s - 1) / s + kAttnKeys - 1) / kAttnKeys);
  }
  return keys;
}

hipError_t launch_attention(const uint16_t* qkv, int qkv_stride, const float* rope_table, const Ragged& rows,
                            int q_heads, int kv_heads, int head_dim, int stride_threshold, int key_stride, uint16_t* out,
                            hipStream_t stream, uint16_t* ks, uint16_t* vts, int keys_cap) {
  int tiles = 0;
  for (int b = 0; b < rows.count; ++b) tiles += (rows.start[b + 1] - rows.start[b] + kAttnQ - 1) / kAttnQ;
  if (tiles == 0) return hipSuccess;
  const int group = q_heads / kv_heads;
  if (group < 1 || group > 8 || q_heads % kv_heads) return hipErrorInvalidValue;
  if (head_dim != 64 && head_dim != 128) return hipErrorInvalidValue;
  // The prepared path's register slots cover a round with 64 threads per
  // 16 dims of the head (one wave at head_dim 64, two at 128); smaller
  // blocks stage from the projection instead.
  const bool prep = ks != nullptr && 64 * group >= attn_prep_min_threads(head_dim);
  if (prep) {
    const int keys = attention_prep_keys(rows, stride_threshold, key_stride);
    if (!vts || keys > keys_cap) return hipErrorInvalidValue;
    dim3 pgrid(keys / kAttnKeys, kv_heads);
    if (head_dim == 64)
      attention_prep_kernel<64><<<pgrid, 256, 0, stream>>>(qkv, qkv_stride, rope_table, rows, q_heads, kv_heads,
                                                           stride_threshold, key_stride, keys_cap, ks, vts);
    else
      attention_prep_kernel<128><<<pgrid, 256, 0, stream>>>(qkv, qkv_stride, rope_table, rows, q_heads, kv_heads,
                                                            stride_threshold, key_stride, keys_cap, ks, vts);
  }
  dim3 grid(tiles, kv_heads);
  // Keys staged per round: every key of the pass's longest request when
  // they fit in ~72 KB of LDS and short requests only (one round of loads
  // and barriers instead of one per 32 keys); 32 for the prepared path, in
  // two LDS stages.
  int longest_keys = 0;
  for (int b = 0; b < rows.count; ++b) {
    const int n = rows.start[b + 1] - rows.start[b];
    const int s = n > stride_threshold ? key_stride : 1;
    longest_keys = std::max(longest_keys, (n + s - 1) / s);
  }
  const int cap = attn_round_keys(head_dim);
  const int sb = prep ? kAttnKeys : std::min(cap, (longest_keys + kAttnKeys - 1) / kAttnKeys * kAttnKeys);
  const int lds = (prep ? 2 : 1) * 2 * (sb * (head_dim + 8) + head_dim * (sb + 8));  // prepared: two stages
#define NEMO_ATTN(HD, P)                                                                                           \
  attention_kernel<HD, P><<<grid, 64 * group, lds, stream>>>(qkv, qkv_stride, rope_table, rows, q_heads, kv_heads, \
                                                             stride_threshold, key_stride, ks, vts, keys_cap, sb, out)
  auto attr = [&](const void* kernel) {
    static bool configured[4] = {false, false, false, false};  // one attribute call per instantiation
    const int slot = (head_dim == 64 ? 0 : 2) + (prep ? 1 : 0);
    if (!configured[slot]) {
      (void)hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 2 * (cap * (head_dim + 8) + head_dim * (cap + 8)));
      configured[slot] = true;
    }
  };
  if (head_dim == 64) {
    if (prep) { attr((const void*)attention_kernel<64, true>); NEMO_ATTN(64, true); }
    else { attr((const void*)attention_kernel<64, false>); NEMO_ATTN(64, false); }
  } else {
    if (prep) { attr((const void*)attention_kernel<128, true>); NEMO_ATTN(128, true); }
    else { attr((const void*)attention_kernel<128, false>); NEMO_ATTN(128, false); }
  }
#undef NEMO_ATTN
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// SwiGLU (src/webgpu/ops.ts:74-88).
// ---------------------------------------------------------------------------

__global__ void swiglu_kernel(const uint16_t* __restrict__ gu, int rows, int f, uint16_t* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  const int64_t total = (int64_t)rows * f;
  if (i >= total) return;
  const int64_t r = i / f, c = i - r * f;
  const half8v g = *(const half8v*)(gu + r * 2 * f + c);
  const half8v u = *(const half8v*)(gu + r * 2 * f + f + c);
  half8v o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float gv = (float)g[e];
    o[e] = (half_t)(gv / (1.0f + expf(-gv)) * (float)u[e]);
  }
  *(half8v*)(out + i) = o;
}

hipError_t launch_swiglu(const uint16_t* gu, int rows, int f, uint16_t* out, hipStream_t stream) {
  const int64_t vec = (int64_t)rows * f / 8;
  if (vec <= 0) return hipSuccess;
  swiglu_kernel<<<(unsigned)((vec + 255) / 256), 256, 0, stream>>>(gu, rows, f, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Adjacent-state token merge (src/webgpu/ops.ts:629-660): output position 0
// is source row 0 (BOS); position p > 0 averages source rows [start, end) with
// start = 1 + (p-1)(S-1)/(T-1), end = max(1 + p(S-1)/(T-1), start+1) min S.
// One workgroup per output row.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void merge_kernel(const uint16_t* __restrict__ in, Ragged src, Ragged dst,
                                                    int hidden, uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int b = ragged_find(dst, t);
  const int p = t - dst.start[b];
  const int S = src.start[b + 1] - src.start[b];
  const int T = dst.start[b + 1] - dst.start[b];
  int start = 0, end = 1;
  if (p > 0 && T > 1) {
    const int st = S - 1, tt = T - 1;
    start = 1 + (int)(((int64_t)(p - 1) * st) / tt);
    end = 1 + (int)(((int64_t)p * st) / tt);
    end = max(end, start + 1);
    end = min(end, S);
  }
  const float inv = 1.0f / (float)(end - start);
  for (int c = threadIdx.x * 8; c < hidden; c += blockDim.x * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int r = start; r < end; ++r) {
      const half8v v = *(const half8v*)(in + (size_t)(src.start[b] + r) * hidden + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += (float)v[e];
    }
    half8v o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (half_t)(acc[e] * inv);
    *(half8v*)(out + (size_t)t * hidden + c) = o;
  }
}

hipError_t launch_merge(const uint16_t* in, const Ragged& src, const Ragged& dst, int hidden, uint16_t* out,
                        hipStream_t stream) {
  const int total = dst.start[dst.count];
  if (total <= 0) return hipSuccess;
  merge_kernel<<<total, 256, 0, stream>>>(in, src, dst, hidden, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Mean pool + L2 normalise (src/webgpu/ops.ts:596-615), in two kernels so a
// long request is read by many CUs:
//  * mean_pool_sum_kernel, grid (hidden / 64, batch): a workgroup owns 64
//    columns of one request; thread (g, p) sums 8 columns (16-byte loads) of
//    rows p, p + 32, ... in order, and the 32 row phases are added in phase
//    order: a fixed order that depends only on the request's length. Writes
//    the means.
//  * l2_normalize_kernel, one workgroup per request: scales the means to unit
//    length (no epsilon, as the reference).
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void mean_pool_sum_kernel(const uint16_t* __restrict__ norm, Ragged rows,
                                                            int hidden, float* __restrict__ out) {
  __shared__ float part[32][64];
  const int b = blockIdx.y, c0 = blockIdx.x * 64;
  const int r0 = rows.start[b], n = rows.start[b + 1] - r0;
  const int g = threadIdx.x & 7, p = threadIdx.x >> 3;
  float total[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int r = p; r < n; r += 32) {
    const half8v v = *(const half8v*)(norm + (size_t)(r0 + r) * hidden + c0 + 8 * g);
#pragma unroll
    for (int e = 0; e < 8; ++e) total[e] += (float)v[e];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) part[p][8 * g + e] = total[e];
  __syncthreads();
  if (threadIdx.x < 64) {
    float sum = part[0][threadIdx.x];
    for (int q = 1; q < 32; ++q) sum += part[q][threadIdx.x];
    out[(size_t)b * hidden + c0 + threadIdx.x] = sum / (float)n;
  }
}

__global__ __launch_bounds__(256) void l2_normalize_kernel(float* __restrict__ out, int hidden) {
  __shared__ float scratch[16];
  float* v = out + (size_t)blockIdx.x * hidden;
  float sq = 0.f;
  for (int c = threadIdx.x; c < hidden; c += blockDim.x) sq += v[c] * v[c];
  const float inv = 1.0f / sqrtf(block_sum(sq, scratch));
  for (int c = threadIdx.x; c < hidden; c += blockDim.x) v[c] *= inv;
}

hipError_t launch_mean_pool(const uint16_t* norm, const Ragged& rows, int hidden, float* out, hipStream_t stream) {
  if (rows.count <= 0) return hipSuccess;
  if (hidden % 64) return hipErrorInvalidValue;
  mean_pool_sum_kernel<<<dim3(hidden / 64, rows.count), 256, 0, stream>>>(norm, rows, hidden, out);
  l2_normalize_kernel<<<rows.count, 256, 0, stream>>>(out, hidden);
  return hipGetLastError();
}

}  // namespace nemo
