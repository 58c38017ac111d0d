// Quantized-weight kernels for gfx950: GGML Q4_K / Q6_K / Q4_0 block
// decoding, the fused dequant + MFMA GEMM (batched tokens) and the split-K
// wavefront GEMV (m <= 16).
//
// Decoding follows src/gguf/quantization.ts:11-74 (and the WGSL decoders of
// src/webgpu/quant-matmul.ts:37-154). Every decoded weight is formed in fp32
// exactly as the reference's JavaScript forms it: d*sc and dmin*m are exact
// products of an 11-bit and a 6-bit significand, d*sc*q is exact (<= 21
// bits), so one fmaf(d*sc, q, -dmin*m) rounds the exact value once - the
// same single rounding as the JS double expression stored to Float32Array.
// Q6_K: d*scale*(q-32) has <= 23 significant bits and is exact in fp32.
// The GEMM feeds MFMA with f16(RNE(that fp32 value)), as the WGSL tiles do.
#include "nemo_common.h"
#include "nemo_quant.h"

namespace nemo {

// ---------------------------------------------------------------------------
// Block field helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t byte_of(const u32x4& v, int i) {
  const uint32_t w = (i < 4) ? v.x : (i < 8) ? v.y : (i < 12) ? v.z : v.w;
  return (w >> (8 * (i & 3))) & 0xffu;
}

// Scale and min of sub-block j (0..7) from the 12 packed bytes that follow
// d and dmin (src/gguf/quantization.ts:11-17). `hdr` is the block's first 16
// bytes, so scale byte i is byte 4 + i of hdr.
__device__ __forceinline__ void q4k_scale_min(const u32x4& hdr, int j, uint32_t& sc, uint32_t& m) {
  if (j < 4) {
    sc = byte_of(hdr, 4 + j) & 63u;
    m = byte_of(hdr, 8 + j) & 63u;
  } else {
    sc = (byte_of(hdr, 8 + j) & 15u) | ((byte_of(hdr, j) >> 6) << 4);
    m = (byte_of(hdr, 8 + j) >> 4) | ((byte_of(hdr, 4 + j) >> 6) << 4);
  }
}

// fp32 factors of group g (sub-blocks 2g, 2g+1): w = fmaf(dsc, q, ndm).
__device__ __forceinline__ void q4k_group_factors(const u32x4& hdr, int g, float& dsc0, float& ndm0,
                                                  float& dsc1, float& ndm1) {
  const float d = h2f((uint16_t)(hdr.x & 0xffffu));
  const float dmin = h2f((uint16_t)(hdr.x >> 16));
  uint32_t sc, m;
  q4k_scale_min(hdr, 2 * g, sc, m);
  dsc0 = d * (float)sc;
  ndm0 = -(dmin * (float)m);
  q4k_scale_min(hdr, 2 * g + 1, sc, m);
  dsc1 = d * (float)sc;
  ndm1 = -(dmin * (float)m);
}

// Four packed bytes (one value per byte) -> four fp32 values scale*b + bias.
__device__ __forceinline__ void bytes4_fma(uint32_t w, float scale, float bias, float* out) {
  out[0] = fmaf(scale, (float)(w & 0xffu), bias);
  out[1] = fmaf(scale, (float)((w >> 8) & 0xffu), bias);
  out[2] = fmaf(scale, (float)((w >> 16) & 0xffu), bias);
  out[3] = fmaf(scale, (float)(w >> 24), bias);
}

__device__ __forceinline__ half8v to_half8(const float* v) {
  half8v h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = (half_t)v[i];
  return h;
}

// ---------------------------------------------------------------------------
// W tile loaders. A loader fetches, for one weight row and one 64-column
// chunk starting at k0, the bytes of "part" p (0/1) and later expands them to
// 32 f16 values: lo[16] for columns k0+16p..k0+16p+15 and hi[16] for columns
// k0+32+16p..k0+32+16p+15.
// ---------------------------------------------------------------------------

struct Q4KFetch {
  u32x4 hdr;
  u32x4 q;
  int g;
};

__device__ __forceinline__ Q4KFetch q4k_fetch(const QWeight& w, size_t row_bytes, int row, int k0, int p) {
  const uint8_t* blk = w.blocks + (size_t)row * row_bytes + (size_t)(k0 >> 8) * 144;
  Q4KFetch f;
  f.g = (k0 >> 6) & 3;
  f.hdr = *(const u32x4*)blk;
  f.q = *(const u32x4*)(blk + 16 + 32 * f.g + 16 * p);
  return f;
}

__device__ __forceinline__ void q4k_expand(const Q4KFetch& f, half8v* lo, half8v* hi) {
  float dsc0, ndm0, dsc1, ndm1;
  q4k_group_factors(f.hdr, f.g, dsc0, ndm0, dsc1, ndm1);
  const uint32_t words[4] = {f.q.x, f.q.y, f.q.z, f.q.w};
  float vl[16], vh[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bytes4_fma(words[i] & 0x0f0f0f0fu, dsc0, ndm0, vl + 4 * i);
    bytes4_fma((words[i] >> 4) & 0x0f0f0f0fu, dsc1, ndm1, vh + 4 * i);
  }
  lo[0] = to_half8(vl);
  lo[1] = to_half8(vl + 8);
  hi[0] = to_half8(vh);
  hi[1] = to_half8(vh + 8);
}

struct Q6KFetch {
  u32x4 qla, qlb, qh;
  uint32_t scw;
  uint16_t d;
  int qp, p;
};

// Q6_K split layout: record = ql[128] qh[64] scales[16], d separate. Chunk
// c = (k0 / 64) % 4 covers half c/2, quadrants 2(c%2) and 2(c%2)+1
// (src/gguf/quantization.ts:53-71).
__device__ __forceinline__ Q6KFetch q6k_fetch(const QWeight& w, size_t row_bytes, int row, int k0, int p) {
  const int blk = k0 >> 8;
  const uint8_t* rec = w.blocks + (size_t)row * row_bytes + (size_t)blk * 208;
  const int c = (k0 >> 6) & 3, half = c >> 1;
  Q6KFetch f;
  f.qp = c & 1;
  f.p = p;
  f.qla = *(const u32x4*)(rec + 64 * half + 16 * p);
  f.qlb = *(const u32x4*)(rec + 64 * half + 32 + 16 * p);
  f.qh = *(const u32x4*)(rec + 128 + 32 * half + 16 * p);
  f.scw = *(const uint32_t*)(rec + 192 + 8 * half + 4 * f.qp);
  f.d = w.d[(size_t)row * (w.k >> 8) + blk];
  return f;
}

__device__ __forceinline__ void q6k_expand(const Q6KFetch& f, half8v* lo, half8v* hi) {
  const float d = h2f(f.d);
  // scale of quadrant 2qp for lanes 16p..16p+15 is scales[8h + p + 4qp]
  // (byte p of scw); quadrant 2qp+1 uses scales[8h + p + 4qp + 2].
  const float dsc0 = d * (float)(int8_t)((f.scw >> (8 * f.p)) & 0xffu);
  const float dsc1 = d * (float)(int8_t)((f.scw >> (8 * (f.p + 2))) & 0xffu);
  const int s0 = 4 * f.qp, s1 = 4 * f.qp + 2;
  const uint32_t la[4] = {f.qla.x, f.qla.y, f.qla.z, f.qla.w};
  const uint32_t lb[4] = {f.qlb.x, f.qlb.y, f.qlb.z, f.qlb.w};
  const uint32_t hh[4] = {f.qh.x, f.qh.y, f.qh.z, f.qh.w};
  float vl[16], vh[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t q0 = ((la[i] >> s0) & 0x0f0f0f0fu) | (((hh[i] >> s0) & 0x03030303u) << 4);
    const uint32_t q1 = ((lb[i] >> s0) & 0x0f0f0f0fu) | (((hh[i] >> s1) & 0x03030303u) << 4);
    bytes4_fma(q0, dsc0, -32.0f * dsc0, vl + 4 * i);
    bytes4_fma(q1, dsc1, -32.0f * dsc1, vh + 4 * i);
  }
  lo[0] = to_half8(vl);
  lo[1] = to_half8(vl + 8);
  hi[0] = to_half8(vh);
  hi[1] = to_half8(vh + 8);
}

// ---------------------------------------------------------------------------
// Fused dequant + MFMA GEMM.  Y[M,N] = X[M,K] * W[N,K]^T.
// Tile 128 x 128 x 64, 256 threads = 4 waves in a 2 x 2 grid, each wave a
// 64 x 64 block of four v_mfma_f32_32x32x16_f16 accumulators. W is decoded
// once per workgroup into LDS and shared by all 128 rows of the M tile.
// Global loads of step k+1 are issued before the MFMAs of step k.
// ---------------------------------------------------------------------------

constexpr int kBM = 128, kBN = 128, kBK = 64, kLdsK = kBK + 8;  // 144-byte LDS rows

template <int TYPE>
__global__ __launch_bounds__(256, 2) void gemm_q_kernel(const uint16_t* __restrict__ x, int ldx, QWeight w,
                                                        uint16_t* __restrict__ y, int ldy, int M) {
  __shared__ __attribute__((aligned(16))) half_t sA[kBM * kLdsK];
  __shared__ __attribute__((aligned(16))) half_t sB[kBN * kLdsK];
  const int N = w.n, K = w.k;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const size_t row_bytes = qweight_row_bytes(TYPE, K);

  // X loader: 4 passes of 32 rows; 8 threads cover one row's 64 columns.
  const int xr = tid >> 3, xc = (tid & 7) * 8;
  const uint16_t* xrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = min(m0 + i * 32 + xr, M - 1);
    xrow[i] = x + (size_t)r * ldx + xc;
  }
  // W loader: 2 threads per weight row.
  const int wr = tid >> 1, wp = tid & 1;
  const int wrow = min(n0 + wr, N - 1);

  u32x4 xa[4];
  Q4KFetch f4;
  Q6KFetch f6;
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) xa[i] = *(const u32x4*)(xrow[i] + k0);
    if constexpr (TYPE == kQ4_K) f4 = q4k_fetch(w, row_bytes, wrow, k0, wp);
    else f6 = q6k_fetch(w, row_bytes, wrow, k0, wp);
  };

  float16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  fetch(0);
  for (int k0 = 0; k0 < K; k0 += kBK) {
    half8v lo[2], hi[2];
    if constexpr (TYPE == kQ4_K) q4k_expand(f4, lo, hi);
    else q6k_expand(f6, lo, hi);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) *(u32x4*)&sA[(i * 32 + xr) * kLdsK + xc] = xa[i];
    half_t* brow = &sB[wr * kLdsK];
    *(half8v*)(brow + 16 * wp) = lo[0];
    *(half8v*)(brow + 16 * wp + 8) = lo[1];
    *(half8v*)(brow + 32 + 16 * wp) = hi[0];
    *(half8v*)(brow + 32 + 16 * wp + 8) = hi[1];
    __syncthreads();
    if (k0 + kBK < K) fetch(k0 + kBK);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int kk = ks * 16 + (lane >> 5) * 8;
      half8v af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = *(const half8v*)&sA[(wm * 64 + i * 32 + (lane & 31)) * kLdsK + kk];
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = *(const half8v*)&sB[(wn * 64 + j * 32 + (lane & 31)) * kLdsK + kk];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }

  // D layout of a 32x32 MFMA block: lane l, register r -> row
  // 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < M) y[(size_t)row * ldy + col] = f2h(acc[i][j][r]);
      }
    }
}

hipError_t launch_gemm(const uint16_t* x, int ldx, const QWeight& w, uint16_t* y, int ldy, int m, hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  dim3 grid((w.n + kBN - 1) / kBN, (m + kBM - 1) / kBM);
  if (w.type == kQ4_K) gemm_q_kernel<kQ4_K><<<grid, 256, 0, stream>>>(x, ldx, w, y, ldy, m);
  else if (w.type == kQ6_K) gemm_q_kernel<kQ6_K><<<grid, 256, 0, stream>>>(x, ldx, w, y, ldy, m);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Split-K GEMV for m <= 16 using v_mfma_f32_16x16x32_f16: a wave owns 16
// weight rows and one K slice; lane l works on row n0 + l%16 and the 8-column
// slice 8*(l/16) of each 32-column MFMA step. Each lane decodes its own
// weights straight into the B fragment (no LDS). Partials of the K slices are
// summed in a fixed order by gemv_reduce_kernel (deterministic).
// ---------------------------------------------------------------------------

constexpr int kGemvWaves = 4;

__device__ __forceinline__ void gemv_q4k_group(const QWeight& w, size_t row_bytes, int row, int k0, int kq,
                                               const u32x4& hdr, half8v& lo, half8v& hi) {
  const uint8_t* blk = w.blocks + (size_t)row * row_bytes + (size_t)(k0 >> 8) * 144;
  const int g = (k0 >> 6) & 3;
  const u32x2 q = *(const u32x2*)(blk + 16 + 32 * g + 8 * kq);
  float dsc0, ndm0, dsc1, ndm1;
  q4k_group_factors(hdr, g, dsc0, ndm0, dsc1, ndm1);
  float vl[8], vh[8];
  bytes4_fma(q.x & 0x0f0f0f0fu, dsc0, ndm0, vl);
  bytes4_fma(q.y & 0x0f0f0f0fu, dsc0, ndm0, vl + 4);
  bytes4_fma((q.x >> 4) & 0x0f0f0f0fu, dsc1, ndm1, vh);
  bytes4_fma((q.y >> 4) & 0x0f0f0f0fu, dsc1, ndm1, vh + 4);
  lo = to_half8(vl);
  hi = to_half8(vh);
}

__device__ __forceinline__ void gemv_q6k_group(const QWeight& w, size_t row_bytes, int row, int k0, int kq,
                                               half8v& lo, half8v& hi) {
  const int blk = k0 >> 8;
  const uint8_t* rec = w.blocks + (size_t)row * row_bytes + (size_t)blk * 208;
  const int c = (k0 >> 6) & 3, half = c >> 1, qp = c & 1;
  const u32x2 qla = *(const u32x2*)(rec + 64 * half + 8 * kq);
  const u32x2 qlb = *(const u32x2*)(rec + 64 * half + 32 + 8 * kq);
  const u32x2 qh = *(const u32x2*)(rec + 128 + 32 * half + 8 * kq);
  const int8_t* sc = (const int8_t*)(rec + 192 + 8 * half);
  const float d = h2f(w.d[(size_t)row * (w.k >> 8) + blk]);
  const float dsc0 = d * (float)sc[(kq >> 1) + 4 * qp];
  const float dsc1 = d * (float)sc[(kq >> 1) + 4 * qp + 2];
  const int s0 = 4 * qp, s1 = 4 * qp + 2;
  float vl[8], vh[8];
  const uint32_t la[2] = {qla.x, qla.y}, lb[2] = {qlb.x, qlb.y}, hh[2] = {qh.x, qh.y};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t q0 = ((la[i] >> s0) & 0x0f0f0f0fu) | (((hh[i] >> s0) & 0x03030303u) << 4);
    const uint32_t q1 = ((lb[i] >> s0) & 0x0f0f0f0fu) | (((hh[i] >> s1) & 0x03030303u) << 4);
    bytes4_fma(q0, dsc0, -32.0f * dsc0, vl + 4 * i);
    bytes4_fma(q1, dsc1, -32.0f * dsc1, vh + 4 * i);
  }
  lo = to_half8(vl);
  hi = to_half8(vh);
}

template <int TYPE>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_q_kernel(const uint16_t* __restrict__ x, int ldx, QWeight w,
                                                                 int M, int kchunk, float* __restrict__ partials,
                                                                 uint16_t* __restrict__ y, int ldy) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int N = w.n;
  const int n0 = (blockIdx.x * kGemvWaves + wave) * 16;
  if (n0 >= N) return;
  const int kbeg = blockIdx.y * kchunk, kend = min(w.k, kbeg + kchunk);
  const int c = lane & 15, kq = lane >> 4;
  const int row = min(n0 + c, N - 1);
  const size_t row_bytes = qweight_row_bytes(TYPE, w.k);
  const uint16_t* xr = x + (size_t)min(c, M - 1) * ldx + 8 * kq;
  float4v acc = {0.f, 0.f, 0.f, 0.f};
  for (int kb = kbeg; kb < kend; kb += 256) {
    u32x4 hdr;
    if constexpr (TYPE == kQ4_K) hdr = *(const u32x4*)(w.blocks + (size_t)row * row_bytes + (size_t)(kb >> 8) * 144);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int k0 = kb + 64 * g;
      half8v blo, bhi;
      if constexpr (TYPE == kQ4_K) gemv_q4k_group(w, row_bytes, row, k0, kq, hdr, blo, bhi);
      else gemv_q6k_group(w, row_bytes, row, k0, kq, blo, bhi);
      const half8v alo = *(const half8v*)(xr + k0);
      const half8v ahi = *(const half8v*)(xr + k0 + 32);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, blo, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bhi, acc, 0, 0, 0);
    }
  }
  // D layout of a 16x16 MFMA block: lane l, register i -> row 4*(l/16) + i,
  // column l%16.
  const int col = n0 + c;
  if (col >= N) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * kq + i;
    if (m >= M) continue;
    if (gridDim.y == 1) y[(size_t)m * ldy + col] = f2h(acc[i]);
    else partials[((size_t)blockIdx.y * M + m) * N + col] = acc[i];
  }
}

__global__ void gemv_reduce_kernel(const float* __restrict__ partials, int splits, int M, int N,
                                   uint16_t* __restrict__ y, int ldy) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * N) return;
  float s = 0.f;
  for (int i = 0; i < splits; ++i) s += partials[(size_t)i * M * N + idx];
  y[(size_t)(idx / N) * ldy + (idx % N)] = f2h(s);
}

static int gemv_splits(const QWeight& w) {
  // Enough waves to keep every SIMD streaming: target >= 4096 waves.
  const int col_waves = (w.n + 15) / 16;
  const int blocks = w.k / 256;
  int splits = 1;
  while (splits < blocks && col_waves * splits < 4096 && blocks % (splits * 2) == 0) splits *= 2;
  return splits;
}

size_t gemv_partials_floats(const QWeight& w, int m) {
  const int s = gemv_splits(w);
  return s > 1 ? (size_t)s * m * w.n : 0;
}

hipError_t launch_gemv(const uint16_t* x, int ldx, const QWeight& w, uint16_t* y, int ldy, int m, float* partials,
                       hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  if (m > 16) return hipErrorInvalidValue;
  const int splits = gemv_splits(w);
  const int kchunk = w.k / splits;
  if (splits > 1 && partials == nullptr) return hipErrorInvalidValue;
  dim3 grid((w.n + 16 * kGemvWaves - 1) / (16 * kGemvWaves), splits);
  if (w.type == kQ4_K)
    gemv_q_kernel<kQ4_K><<<grid, 64 * kGemvWaves, 0, stream>>>(x, ldx, w, m, kchunk, partials, y, ldy);
  else if (w.type == kQ6_K)
    gemv_q_kernel<kQ6_K><<<grid, 64 * kGemvWaves, 0, stream>>>(x, ldx, w, m, kchunk, partials, y, ldy);
  else
    return hipErrorInvalidValue;
  if (splits > 1) {
    const int total = m * w.n;
    gemv_reduce_kernel<<<(total + 255) / 256, 256, 0, stream>>>(partials, splits, m, w.n, y, ldy);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Standalone decoding.
// ---------------------------------------------------------------------------

// Q4_K raw: 8 threads per 144-byte block; thread c decodes nibble bytes
// [16(c%2), +16) of group c/2: 16 low-nibble and 16 high-nibble values.
__global__ void dequant_q4k_kernel(const uint8_t* __restrict__ raw, int64_t n_blocks, float* __restrict__ out32,
                                   uint16_t* __restrict__ out16) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = t >> 3;
  if (b >= n_blocks) return;
  const int c = (int)(t & 7), g = c >> 1, h = c & 1;
  const uint8_t* blk = raw + b * 144;
  const u32x4 hdr = *(const u32x4*)blk;
  const u32x4 q = *(const u32x4*)(blk + 16 + 32 * g + 16 * h);
  float dsc0, ndm0, dsc1, ndm1;
  q4k_group_factors(hdr, g, dsc0, ndm0, dsc1, ndm1);
  const uint32_t words[4] = {q.x, q.y, q.z, q.w};
  float vl[16], vh[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bytes4_fma(words[i] & 0x0f0f0f0fu, dsc0, ndm0, vl + 4 * i);
    bytes4_fma((words[i] >> 4) & 0x0f0f0f0fu, dsc1, ndm1, vh + 4 * i);
  }
  const int64_t lo = b * 256 + 64 * g + 16 * h, hi = lo + 32;
  if (out32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *(float4v*)(out32 + lo + 4 * i) = float4v{vl[4 * i], vl[4 * i + 1], vl[4 * i + 2], vl[4 * i + 3]};
      *(float4v*)(out32 + hi + 4 * i) = float4v{vh[4 * i], vh[4 * i + 1], vh[4 * i + 2], vh[4 * i + 3]};
    }
  }
  if (out16) {
    *(half8v*)(out16 + lo) = to_half8(vl);
    *(half8v*)(out16 + lo + 8) = to_half8(vl + 8);
    *(half8v*)(out16 + hi) = to_half8(vh);
    *(half8v*)(out16 + hi + 8) = to_half8(vh + 8);
  }
}

// Blocks whose size is not a multiple of 16 bytes (Q6_K 210, Q4_0 18) are
// staged: a workgroup copies a span of whole blocks, which starts 16-byte
// aligned, from HBM into LDS with 16-byte loads, then decodes from LDS.
constexpr int kQ6Span = 32;   // 32 * 210 = 6720 bytes = 420 * 16
constexpr int kQ40Span = 64;  // 64 * 18 = 1152 bytes = 72 * 16

__device__ __forceinline__ void stage_span(const uint8_t* __restrict__ src, int bytes, uint8_t* lds) {
  const int vec = bytes >> 4;
  for (int i = threadIdx.x; i < vec; i += blockDim.x) ((u32x4*)lds)[i] = ((const u32x4*)src)[i];
  // Block sizes are even, so the tail is whole 16-bit words.
  for (int i = (vec << 3) + threadIdx.x; i < (bytes >> 1); i += blockDim.x)
    ((uint16_t*)lds)[i] = ((const uint16_t*)src)[i];
  __syncthreads();
}

// Q6_K raw: thread t decodes 32 values (half c/4, quadrant c%4, lanes 0..31)
// of block t/8 of the span (src/gguf/quantization.ts:53-71).
__global__ __launch_bounds__(256) void dequant_q6k_kernel(const uint8_t* __restrict__ raw, int64_t n_blocks,
                                                          float* __restrict__ out32, uint16_t* __restrict__ out16) {
  __shared__ __attribute__((aligned(16))) uint8_t span[kQ6Span * 210];
  const int64_t b0 = (int64_t)blockIdx.x * kQ6Span;
  const int nb = (int)min((int64_t)kQ6Span, n_blocks - b0);
  stage_span(raw + b0 * 210, nb * 210, span);
  const int bl = threadIdx.x >> 3, c = threadIdx.x & 7;
  if (bl >= nb) return;
  const uint8_t* blk = span + bl * 210;
  const int half = c >> 2, quadrant = c & 3;
  const float d = h2f((uint16_t)(blk[208] | (blk[209] << 8)));
  float v[32];
#pragma unroll
  for (int lane = 0; lane < 32; ++lane) {
    const uint32_t low = blk[64 * half + lane + 32 * (quadrant & 1)];
    const uint32_t lowq = quadrant >= 2 ? (low >> 4) : (low & 15u);
    const uint32_t high = (blk[128 + 32 * half + lane] >> (2 * quadrant)) & 3u;
    const int scale = (int8_t)blk[192 + 8 * half + (lane >> 4) + 2 * quadrant];
    v[lane] = (d * (float)scale) * (float)((int)(lowq | (high << 4)) - 32);
  }
  const int64_t o = (b0 + bl) * 256 + 128 * half + 32 * quadrant;
  if (out32) {
#pragma unroll
    for (int i = 0; i < 8; ++i) *(float4v*)(out32 + o + 4 * i) = float4v{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
  }
  if (out16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *(half8v*)(out16 + o + 8 * i) = to_half8(v + 8 * i);
  }
}

// Q4_0 raw (src/gguf/quantization.ts:40-44): thread t decodes 8 values of
// block t/4: part p<2 -> low nibbles of bytes 2+8p.., p>=2 -> high nibbles.
__global__ __launch_bounds__(256) void dequant_q40_kernel(const uint8_t* __restrict__ raw, int64_t n_blocks,
                                                          float* __restrict__ out32, uint16_t* __restrict__ out16) {
  __shared__ __attribute__((aligned(16))) uint8_t span[kQ40Span * 18];
  const int64_t b0 = (int64_t)blockIdx.x * kQ40Span;
  const int nb = (int)min((int64_t)kQ40Span, n_blocks - b0);
  stage_span(raw + b0 * 18, nb * 18, span);
  const int bl = threadIdx.x >> 2, p = threadIdx.x & 3;
  if (bl >= nb) return;
  const uint8_t* blk = span + bl * 18;
  const float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t byte = blk[2 + 8 * (p & 1) + i];
    const uint32_t q = p >= 2 ? (byte >> 4) : (byte & 15u);
    v[i] = d * (float)((int)q - 8);
  }
  const int64_t o = (b0 + bl) * 32 + 8 * p;
  if (out32) {
    *(float4v*)(out32 + o) = float4v{v[0], v[1], v[2], v[3]};
    *(float4v*)(out32 + o + 4) = float4v{v[4], v[5], v[6], v[7]};
  }
  if (out16) *(half8v*)(out16 + o) = to_half8(v);
}

hipError_t launch_dequant_raw(int type, const uint8_t* raw, int64_t n_blocks, float* out32, uint16_t* out16,
                              hipStream_t stream) {
  if (n_blocks <= 0) return hipSuccess;
  if (type == kQ4_K) {
    const int64_t threads = n_blocks * 8;
    dequant_q4k_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(raw, n_blocks, out32, out16);
  } else if (type == kQ6_K) {
    dequant_q6k_kernel<<<(unsigned)((n_blocks + kQ6Span - 1) / kQ6Span), 256, 0, stream>>>(raw, n_blocks, out32, out16);
  } else if (type == kQ4_0) {
    dequant_q40_kernel<<<(unsigned)((n_blocks + kQ40Span - 1) / kQ40Span), 256, 0, stream>>>(raw, n_blocks, out32, out16);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Q6_K split layout -> float32: thread per (block, 32 values).
__global__ void dequant_q6k_split_kernel(QWeight w, float* __restrict__ out32) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nb = (int64_t)w.n * (w.k >> 8);
  const int64_t b = t >> 3;
  if (b >= nb) return;
  const int c = (int)(t & 7), half = c >> 2, quadrant = c & 3;
  const uint8_t* rec = w.blocks + b * 208;
  const float d = h2f(w.d[b]);
#pragma unroll 4
  for (int lane = 0; lane < 32; ++lane) {
    const uint32_t low = rec[64 * half + lane + 32 * (quadrant & 1)];
    const uint32_t lowq = quadrant >= 2 ? (low >> 4) : (low & 15u);
    const uint32_t high = (rec[128 + 32 * half + lane] >> (2 * quadrant)) & 3u;
    const int scale = (int8_t)rec[192 + 8 * half + (lane >> 4) + 2 * quadrant];
    out32[b * 256 + 128 * half + 32 * quadrant + lane] = (d * (float)scale) * (float)((int)(lowq | (high << 4)) - 32);
  }
}

hipError_t launch_dequant_weight(const QWeight& w, float* out32, hipStream_t stream) {
  const int64_t nb = (int64_t)w.n * (w.k / 256);
  if (w.type == kQ4_K) return launch_dequant_raw(kQ4_K, w.blocks, nb, out32, nullptr, stream);
  if (w.type != kQ6_K) return hipErrorInvalidValue;
  const int64_t threads = nb * 8;
  dequant_q6k_split_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(w, out32);
  return hipGetLastError();
}

}  // namespace nemo
