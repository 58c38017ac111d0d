// Elementwise, attention, merge and pooling kernels of the encoder pass for
// gfx950, on the ragged packed token layout (request b owns rows
// [start[b], start[b+1]); no padding rows exist).
//
// Semantics follow src/webgpu/ops.ts (cited per kernel). Storage is f16 as in
// the reference's buffers; arithmetic is fp32.
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
// 8 values (16 bytes) per thread and pass.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void rmsnorm_kernel(uint16_t* __restrict__ x, const uint16_t* __restrict__ delta,
                                                      const float* __restrict__ w, uint16_t* __restrict__ out,
                                                      int hidden, float eps) {
  __shared__ float scratch[16];
  const size_t base = (size_t)blockIdx.x * hidden;
  float sum = 0.f;
  for (int c = threadIdx.x * 8; c < hidden; c += blockDim.x * 8) {
    half8v xv = *(const half8v*)(x + base + c);
    if (delta) {
      const half8v dv = *(const half8v*)(delta + base + c);
      half8v stored;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = (float)xv[i] + (float)dv[i];
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
  rmsnorm_kernel<<<rows, 256, 0, stream>>>(x, delta, w, normalized, hidden, eps);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Pairwise RoPE (src/webgpu/ops.ts:168-193): (e, o) -> (e c - o s, e s + o c)
// with (c, s) = table[position][pair]. One workgroup per token.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void rope_kernel(const uint16_t* __restrict__ qkv, int qkv_stride, Ragged rows,
                                                   const float* __restrict__ table, int q_heads, int kv_heads,
                                                   int head_dim, uint16_t* __restrict__ q, uint16_t* __restrict__ k) {
  const int t = blockIdx.x;
  const int b = ragged_find(rows, t);
  const int pos = t - rows.start[b];
  const int pairs = head_dim / 2;
  const int total = (q_heads + kv_heads) * pairs;
  const float* trow = table + (size_t)pos * pairs * 2;
  for (int i = threadIdx.x; i < total; i += blockDim.x) {
    const int head = i / pairs, pair = i - head * pairs;
    const uint32_t in = *(const uint32_t*)(qkv + (size_t)t * qkv_stride + head * head_dim + 2 * pair);
    const float e = h2f((uint16_t)(in & 0xffffu)), o = h2f((uint16_t)(in >> 16));
    const float c = trow[2 * pair], s = trow[2 * pair + 1];
    const uint32_t outv = (uint32_t)f2h(e * c - o * s) | ((uint32_t)f2h(e * s + o * c) << 16);
    if (head < q_heads)
      *(uint32_t*)(q + ((size_t)t * q_heads + head) * head_dim + 2 * pair) = outv;
    else
      *(uint32_t*)(k + ((size_t)t * kv_heads + (head - q_heads)) * head_dim + 2 * pair) = outv;
  }
}

hipError_t launch_rope(const uint16_t* qkv, int qkv_stride, const Ragged& rows, const float* table, int q_heads,
                       int kv_heads, int head_dim, uint16_t* q, uint16_t* k, hipStream_t stream) {
  const int total = rows.start[rows.count];
  if (total <= 0) return hipSuccess;
  rope_kernel<<<total, 256, 0, stream>>>(qkv, qkv_stride, rows, table, q_heads, kv_heads, head_dim, q, k);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Bidirectional GQA attention (src/webgpu/ops.ts:213-293, 295-362).
// For request b with n valid rows, query i attends keys 0, s, 2s, ... < n
// (s = key_stride if n > stride_threshold, else 1) with scores
// q.k * head_dim^-1/2 * temperature(i), temperature = 1 + 0.1 ln(floor(i /
// 16384) + 1) for i >= 16384 (ops.ts:241). Online softmax in fp32.
// Workgroup = 64 queries of one request and head; 4 lanes per query, each
// holding a quarter of the head dimension. Keys/values staged in LDS tiles.
// ---------------------------------------------------------------------------

constexpr int kAttnQ = 64, kAttnKeys = 64;

template <int HD>
__global__ __launch_bounds__(256) void attention_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                        const uint16_t* __restrict__ v_base, int v_stride,
                                                        Ragged rows, int q_heads, int kv_heads, int stride_threshold,
                                                        int key_stride_long, uint16_t* __restrict__ out) {
  constexpr int QD = HD / 4;
  __shared__ __attribute__((aligned(16))) half_t sK[kAttnKeys * HD];
  __shared__ __attribute__((aligned(16))) half_t sV[kAttnKeys * HD];
  // Locate (request, query tile) of this workgroup.
  int b = 0, tile = blockIdx.x;
  for (; b < rows.count; ++b) {
    const int n = rows.start[b + 1] - rows.start[b];
    const int tiles = (n + kAttnQ - 1) / kAttnQ;
    if (tile < tiles) break;
    tile -= tiles;
  }
  if (b >= rows.count) return;
  const int row0 = rows.start[b];
  const int n = rows.start[b + 1] - row0;
  const int h = blockIdx.y;
  const int kvh = h / (q_heads / kv_heads);
  const int qi = tile * kAttnQ + (threadIdx.x >> 2);
  const int part = threadIdx.x & 3;
  const int key_stride = n > stride_threshold ? key_stride_long : 1;
  const float temperature = qi >= 16384 ? logf(floorf((float)qi / 16384.0f) + 1.0f) * 0.1f + 1.0f : 1.0f;
  const float scale = (1.0f / sqrtf((float)HD)) * temperature;

  float qv[QD], acc[QD];
  {
    const int qrow = min(qi, n - 1);
    const uint16_t* qp = q + ((size_t)(row0 + qrow) * q_heads + h) * HD + part * QD;
#pragma unroll
    for (int i = 0; i < QD; i += 8) {
      const half8v hv = *(const half8v*)(qp + i);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qv[i + e] = (float)hv[e];
        acc[i + e] = 0.f;
      }
    }
  }
  float mx = -INFINITY, den = 0.f;
  const int n_keys = (n + key_stride - 1) / key_stride;
  for (int kb = 0; kb < n_keys; kb += kAttnKeys) {
    __syncthreads();
    // Stage up to 64 sampled keys and values: 8 halves per thread and pass.
    for (int i = threadIdx.x; i < kAttnKeys * HD / 8; i += blockDim.x) {
      const int j = i / (HD / 8), c = (i % (HD / 8)) * 8;
      const int kj = kb + j;
      u32x4 kv4 = {0u, 0u, 0u, 0u}, vv4 = {0u, 0u, 0u, 0u};
      if (kj < n_keys) {
        const int trow = row0 + kj * key_stride;
        kv4 = *(const u32x4*)(k + ((size_t)trow * kv_heads + kvh) * HD + c);
        vv4 = *(const u32x4*)(v_base + (size_t)trow * v_stride + kvh * HD + c);
      }
      *(u32x4*)&sK[j * HD + c] = kv4;
      *(u32x4*)&sV[j * HD + c] = vv4;
    }
    __syncthreads();
    const int jn = min(kAttnKeys, n_keys - kb);
    for (int j = 0; j < jn; ++j) {
      const half_t* kr = &sK[j * HD + part * QD];
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < QD; i += 8) {
        const half8v kh = *(const half8v*)(kr + i);
#pragma unroll
        for (int e = 0; e < 8; ++e) s = fmaf(qv[i + e], (float)kh[e], s);
      }
      s += __shfl_xor(s, 1, 64);
      s += __shfl_xor(s, 2, 64);
      s *= scale;
      const float mnew = fmaxf(mx, s);
      const float alpha = expf(mx - mnew);
      const float p = expf(s - mnew);
      den = den * alpha + p;
      mx = mnew;
      const half_t* vr = &sV[j * HD + part * QD];
#pragma unroll
      for (int i = 0; i < QD; i += 8) {
        const half8v vh = *(const half8v*)(vr + i);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[i + e] = fmaf(p, (float)vh[e], acc[i + e] * alpha);
      }
    }
  }
  if (qi >= n) return;
  const float inv = 1.0f / den;
  uint16_t* op = out + ((size_t)(row0 + qi) * q_heads + h) * HD + part * QD;
#pragma unroll
  for (int i = 0; i < QD; i += 8) {
    half8v o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (half_t)(acc[i + e] * inv);
    *(half8v*)(op + i) = o;
  }
}

hipError_t launch_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v_base, int v_stride,
                            const Ragged& rows, int q_heads, int kv_heads, int head_dim, int stride_threshold,
                            int key_stride, uint16_t* out, hipStream_t stream) {
  int tiles = 0;
  for (int b = 0; b < rows.count; ++b) tiles += (rows.start[b + 1] - rows.start[b] + kAttnQ - 1) / kAttnQ;
  if (tiles == 0) return hipSuccess;
  dim3 grid(tiles, q_heads);
  if (head_dim == 64)
    attention_kernel<64><<<grid, 256, 0, stream>>>(q, k, v_base, v_stride, rows, q_heads, kv_heads, stride_threshold,
                                                   key_stride, out);
  else if (head_dim == 128)
    attention_kernel<128><<<grid, 256, 0, stream>>>(q, k, v_base, v_stride, rows, q_heads, kv_heads, stride_threshold,
                                                    key_stride, out);
  else
    return hipErrorInvalidValue;
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
// Mean pool + L2 normalise (src/webgpu/ops.ts:596-615). One workgroup per
// request.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void mean_pool_kernel(const uint16_t* __restrict__ norm, Ragged rows, int hidden,
                                                        float* __restrict__ out) {
  __shared__ float scratch[16];
  const int b = blockIdx.x;
  const int r0 = rows.start[b], n = rows.start[b + 1] - r0;
  float sq = 0.f;
  for (int d = threadIdx.x; d < hidden; d += blockDim.x) {
    float total = 0.f;
    for (int p = 0; p < n; ++p) total += h2f(norm[(size_t)(r0 + p) * hidden + d]);
    const float mean = total / (float)n;
    out[(size_t)b * hidden + d] = mean;
    sq += mean * mean;
  }
  const float inv = 1.0f / sqrtf(block_sum(sq, scratch));
  for (int d = threadIdx.x; d < hidden; d += blockDim.x) out[(size_t)b * hidden + d] *= inv;
}

hipError_t launch_mean_pool(const uint16_t* norm, const Ragged& rows, int hidden, float* out, hipStream_t stream) {
  if (rows.count <= 0) return hipSuccess;
  mean_pool_kernel<<<rows.count, 256, 0, stream>>>(norm, rows, hidden, out);
  return hipGetLastError();
}

}  // namespace nemo
