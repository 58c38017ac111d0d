// Quantized-weight kernels for gfx950 besides the GEMM: the split-K
// wavefront GEMV (m <= 16), GGML Q4_K / Q6_K / Q4_0 block decoding to
// float32/f16 (bit-exact with src/gguf/quantization.ts:19-74), and the
// fixed-order reduction of split-K partial sums.
#include "nemo_blocks.h"
#include "nemo_common.h"
#include "nemo_quant.h"

namespace nemo {

// ---------------------------------------------------------------------------
// Split-K GEMV for m <= 16 using v_mfma_f32_16x16x32_f16: a wave owns 16
// weight rows and one K slice; lane l works on row n0 + l%16 and the 8-column
// slice 8*(l/16) of each 32-column MFMA step. Each lane decodes its own
// weights straight into the B fragment (no LDS). Partials of the K slices are
// summed in a fixed order by reduce_partials_kernel (deterministic).
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
    if (partials == nullptr) y[(size_t)m * ldy + col] = f2h(acc[i]);
    else partials[((size_t)blockIdx.y * M + m) * N + col] = acc[i];
  }
}

__global__ void reduce_partials_kernel(const float* __restrict__ partials, int splits, int M, int N,
                                       uint16_t* __restrict__ y, int ldy) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  float s = 0.f;
  for (int i = 0; i < splits; ++i) s += partials[(size_t)i * M * N + idx];
  y[(size_t)(idx / N) * ldy + (idx % N)] = f2h(s);
}

hipError_t launch_reduce_partials(const float* partials, int splits, int m, int n, uint16_t* y, int ldy,
                                  hipStream_t stream) {
  const int64_t total = (int64_t)m * n;
  if (total <= 0) return hipSuccess;
  reduce_partials_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(partials, splits, m, n, y, ldy);
  return hipGetLastError();
}

// SwiGLU over split-K partials of the gate/up projection, whose rows are
// interleaved per 128-row group (64 gate rows, then the matching 64 up rows):
// feature f reads columns 128 (f / 64) + f % 64 (g) and that + 64 (u). Same
// arithmetic as the GEMM's SwiGLU epilogue (src/webgpu/ops.ts:85-87 on the
// f16-rounded g and u).
__global__ void reduce_swiglu_kernel(const float* __restrict__ partials, int splits, int M, int N,
                                     uint16_t* __restrict__ y, int ldy) {
  const int F = N / 2;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)M * F) return;
  const int m = (int)(idx / F), f = (int)(idx % F);
  const int gc = 128 * (f >> 6) + (f & 63);
  float gs = 0.f, us = 0.f;
  for (int i = 0; i < splits; ++i) {
    const float* row = partials + ((size_t)i * M + m) * N;
    gs += row[gc];
    us += row[gc + 64];
  }
  const float g = (float)(half_t)gs;
  const float u = (float)(half_t)us;
  y[(size_t)m * ldy + f] = f2h(g / (1.0f + expf(-g)) * u);
}

int gemv_splits(const QWeight& w) {
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
  float* p = splits > 1 ? partials : nullptr;
  if (w.type == kQ4_K)
    gemv_q_kernel<kQ4_K><<<grid, 64 * kGemvWaves, 0, stream>>>(x, ldx, w, m, kchunk, p, y, ldy);
  else if (w.type == kQ6_K)
    gemv_q_kernel<kQ6_K><<<grid, 64 * kGemvWaves, 0, stream>>>(x, ldx, w, m, kchunk, p, y, ldy);
  else
    return hipErrorInvalidValue;
  if (splits > 1) return launch_reduce_partials(partials, splits, m, w.n, y, ldy, stream);
  return hipGetLastError();
}

hipError_t launch_gemv_ex(const uint16_t* x, int ldx, const QWeight& w, int m, int epilogue, void* out, int ldo,
                          float* partials, hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  if (m > 16 || (w.type != kQ4_K && w.type != kQ6_K)) return hipErrorInvalidValue;
  if (epilogue == kEpiStore) return launch_gemv(x, ldx, w, (uint16_t*)out, ldo, m, partials, stream);
  const int splits = gemv_splits(w);
  const int kchunk = w.k / splits;
  dim3 grid((w.n + 16 * kGemvWaves - 1) / (16 * kGemvWaves), splits);
  // kEpiPartial: the caller's buffer receives [splits][m][n] fp32 sums;
  // kEpiSwiGLU: sums go to `partials`, then the SwiGLU reduction.
  float* p = epilogue == kEpiPartial ? (float*)out : partials;
  if (p == nullptr || (epilogue == kEpiPartial && ldo != w.n)) return hipErrorInvalidValue;
  if (epilogue == kEpiSwiGLU && w.n % 128) return hipErrorInvalidValue;
  if (w.type == kQ4_K)
    gemv_q_kernel<kQ4_K><<<grid, 64 * kGemvWaves, 0, stream>>>(x, ldx, w, m, kchunk, p, nullptr, 0);
  else
    gemv_q_kernel<kQ6_K><<<grid, 64 * kGemvWaves, 0, stream>>>(x, ldx, w, m, kchunk, p, nullptr, 0);
  if (epilogue == kEpiSwiGLU) {
    const int64_t total = (int64_t)m * (w.n / 2);
    reduce_swiglu_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(p, splits, m, w.n, (uint16_t*)out, ldo);
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
