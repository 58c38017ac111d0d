// Quantized-weight kernels for gfx950 besides the GEMM: the split-K
// wavefront GEMV (m <= 160), GGML Q4_K / Q6_K / Q4_0 block decoding to
// float32/f16 (bit-exact with src/gguf/quantization.ts:19-74), and the
// fixed-order reduction of split-K partial sums.
#include <algorithm>
#include <type_traits>

#include "nemo_blocks.h"
#include "nemo_common.h"
#include "nemo_quant.h"

namespace nemo {

// ---------------------------------------------------------------------------
// GEMV for m <= 160 on v_mfma_f32_16x16x32_f16. A workgroup of 8 waves owns
// 16 T weight rows (T = 1, 2 or 4 tiles of 16) and 8 consecutive 256-value
// blocks of K: wave w takes block 8 * blockIdx.y + w of all T tiles. A wave
// issues all of its weight loads before their first use (one memory round
// trip per wave) and decodes them once into MFMA fragments that serve every
// group of 16 tokens in turn (the next group's X loads in flight meanwhile);
// each X fragment feeds the MFMAs of the T tiles, and the 8 waves' sums are
// added in LDS in wave order (deterministic). A token's arithmetic does not
// depend on how many groups share the launch. For T >= 2 the first
// T/2 tiles are consecutive rows of the first half of a 128-row group and
// the last T/2 the rows 64 later, so with the gate/up rows interleaved per
// 128-row group a workgroup holds gate and up rows of the same features and
// SwiGLU completes in it. K beyond 2048 splits over blockIdx.y into fp32
// partials that the consumer sums in split order.
//
// MFMA operands: lane l supplies A = X[token l%16][8 consecutive k] and
// B = W[row l%16][the same 8 k]. Lane group kq = l/16 owns four runs of 16
// consecutive k in every block (the bytes it loads), two MFMAs per run.
//
// X reaches the MFMAs through LDS: a wave reads its 16 x 256 slice of X
// with 8 loads of 1 KB (two whole 512-byte rows each, so every load reads 8
// full cache lines; loading the fragments straight from global memory
// touches 16 or more lines per load), writes it to LDS and reads its
// fragments back with ds_read_b128. Row t's 16-byte chunk s sits in slot
// s ^ t of the row, which spreads the 16 rows a fragment read touches over
// distinct banks. The slice is the wave's own; its region later holds the
// wave's sums for the cross-wave reduction.
// ---------------------------------------------------------------------------

constexpr int kGvWaves = 8;
constexpr int kGvXSlice = 16 * 256 * 2;  // LDS bytes of a wave's X slice

// Q4_K: the lane group loads nibble bytes [16kq, +16) (group kq/2) and
// [64 + 16kq, +16) (group 2 + kq/2); runs: 0 = first chunk's low nibbles,
// 1 = its high nibbles, 2 / 3 = the same for the second chunk.
__device__ __forceinline__ int gv_q4k_run_k(int kq, int r) {
  return 64 * ((kq >> 1) + 2 * (r >> 1)) + 16 * (kq & 1) + 32 * (r & 1);
}
// Q6_K: half h = kq/2 and quadrants Qa = kq & 1 (low nibbles of ql bytes
// [64h + 32Qa, +32)) and Qa + 2 (their high nibbles); run r: quadrant
// Qa + 2 (r >> 1), lanes 16 (r & 1) .. +16.
__device__ __forceinline__ int gv_q6k_run_k(int kq, int r) {
  return 128 * (kq >> 1) + 32 * ((kq & 1) + 2 * (r >> 1)) + 16 * (r & 1);
}

struct GvQ4K {
  u32x4 hdr, qa, qb;
  __device__ __forceinline__ void load(const QWeight& w, size_t row_bytes, int row, int blk, int kq) {
    const uint8_t* p = w.blocks + (size_t)row * row_bytes + (size_t)blk * 144;
    hdr = *(const u32x4*)p;
    qa = *(const u32x4*)(p + 16 + 16 * kq);
    qb = *(const u32x4*)(p + 80 + 16 * kq);
  }
  // The same bytes from the tiled copy (launch_tile_q4k): row 16 tile + c.
  __device__ __forceinline__ void load_tiled(const QWeight& w, int tile, int c, int blk, int kq) {
    const uint8_t* base = w.gv + ((size_t)tile * (w.k >> 8) + blk) * 2304;
    hdr = *(const u32x4*)(base + 16 * c);
    qa = *(const u32x4*)(base + 256 + 16 * (16 * kq + c));
    qb = *(const u32x4*)(base + 1280 + 16 * (16 * kq + c));
  }
  // The 16 values of run r as two f16 fragments (k order).
  __device__ __forceinline__ void run(int kq, int r, half8v& f0, half8v& f1) const {
    float dsc0, ndm0, dsc1, ndm1;
    q4k_group_factors(hdr, (kq >> 1) + 2 * (r >> 1), dsc0, ndm0, dsc1, ndm1);
    const u32x4 q = (r >> 1) ? qb : qa;
    const int sh = 4 * (r & 1);
    const float dsc = (r & 1) ? dsc1 : dsc0, ndm = (r & 1) ? ndm1 : ndm0;
    const uint32_t words[4] = {q.x, q.y, q.z, q.w};
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) nibbles4_fma((words[i] >> sh) & 0x0f0f0f0fu, dsc, ndm, v + 4 * i);
    f0 = to_half8(v);
    f1 = to_half8(v + 8);
  }
};

struct GvQ6K {
  u32x4 ql0, ql1, qh0, qh1, sc;
  uint16_t d;
  __device__ __forceinline__ void load(const QWeight& w, size_t row_bytes, int row, int blk, int kq) {
    const uint8_t* rec = w.blocks + (size_t)row * row_bytes + (size_t)blk * 208;
    const int h = kq >> 1, qa = kq & 1;
    ql0 = *(const u32x4*)(rec + 64 * h + 32 * qa);
    ql1 = *(const u32x4*)(rec + 64 * h + 32 * qa + 16);
    qh0 = *(const u32x4*)(rec + 128 + 32 * h);
    qh1 = *(const u32x4*)(rec + 128 + 32 * h + 16);
    sc = *(const u32x4*)(rec + 192);
    d = w.d[(size_t)row * (w.k >> 8) + blk];
  }
  // From the tiled copy (launch_tile_gemv): 3360 bytes per 16-row tile and
  // block: ql first halves [kq][row], ql second halves, qh first halves
  // [half][row], qh second halves, the 16 scale bytes [row], d [row].
  __device__ __forceinline__ void load_tiled(const QWeight& w, int tile, int c, int blk, int kq) {
    const uint8_t* base = w.gv + ((size_t)tile * (w.k >> 8) + blk) * 3360;
    const int h = kq >> 1;
    ql0 = *(const u32x4*)(base + 16 * (16 * kq + c));
    ql1 = *(const u32x4*)(base + 1024 + 16 * (16 * kq + c));
    qh0 = *(const u32x4*)(base + 2048 + 16 * (16 * h + c));
    qh1 = *(const u32x4*)(base + 2560 + 16 * (16 * h + c));
    sc = *(const u32x4*)(base + 3072 + 16 * c);
    d = *(const uint16_t*)(base + 3328 + 2 * c);
  }
  __device__ __forceinline__ void run(int kq, int r, half8v& f0, half8v& f1) const {
    const int h = kq >> 1, Q = (kq & 1) + 2 * (r >> 1), jh = r & 1;
    const u32x4 ql = jh ? ql1 : ql0, qh = jh ? qh1 : qh0;
    // scale of (half h, lanes 16 jh.., quadrant Q) is scales[8h + jh + 2Q]
    const int sb = 8 * h + jh + 2 * Q;
    const uint32_t sw = sb < 4 ? sc.x : sb < 8 ? sc.y : sb < 12 ? sc.z : sc.w;
    const float dsc = h2f(d) * (float)(int8_t)((sw >> (8 * (sb & 3))) & 0xffu);
    const int ls = 4 * (r >> 1), hs = 2 * Q;
    const uint32_t lw[4] = {ql.x, ql.y, ql.z, ql.w}, hw[4] = {qh.x, qh.y, qh.z, qh.w};
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q = ((lw[i] >> ls) & 0x0f0f0f0fu) | (((hw[i] >> hs) & 0x03030303u) << 4);
      bytes4_fma(opaque(q), dsc, -32.0f * dsc, v + 4 * i);
    }
    f0 = to_half8(v);
    f1 = to_half8(v + 8);
  }
};

// Q4_0 (split layout): lane group kq owns values [64kq, +64) of the
// 256-value block, i.e. the Q4_0 blocks 2kq and 2kq + 1; run r = block
// 2kq + r/2, low (r even) or high (r odd) nibbles.
__device__ __forceinline__ int gv_q40_run_k(int kq, int r) { return 64 * kq + 16 * r; }

struct GvQ40 {
  u32x4 q0, q1;
  uint16_t d0, d1;
  __device__ __forceinline__ void load(const QWeight& w, size_t row_bytes, int row, int blk, int kq) {
    const int b = 8 * blk + 2 * kq;
    const uint8_t* p = w.blocks + (size_t)row * row_bytes + (size_t)b * 16;
    q0 = *(const u32x4*)p;
    q1 = *(const u32x4*)(p + 16);
    const uint16_t* d = w.d + (size_t)row * (w.k >> 5) + b;
    d0 = d[0];
    d1 = d[1];
  }
  // From the tiled copy (launch_tile_gemv): 2304 bytes per 16-row tile and
  // 256 values: first blocks of the pairs [kq][row], second blocks, the two
  // scales [kq][row].
  __device__ __forceinline__ void load_tiled(const QWeight& w, int tile, int c, int blk, int kq) {
    const uint8_t* base = w.gv + ((size_t)tile * (w.k >> 8) + blk) * 2304;
    q0 = *(const u32x4*)(base + 16 * (16 * kq + c));
    q1 = *(const u32x4*)(base + 1024 + 16 * (16 * kq + c));
    const uint32_t dd = *(const uint32_t*)(base + 2048 + 4 * (16 * kq + c));
    d0 = (uint16_t)(dd & 0xffffu);
    d1 = (uint16_t)(dd >> 16);
  }
  __device__ __forceinline__ void run(int kq, int r, half8v& f0, half8v& f1) const {
    const u32x4 q = (r >> 1) ? q1 : q0;
    const float d = h2f((r >> 1) ? d1 : d0);
    const int sh = 4 * (r & 1);
    const uint32_t words[4] = {q.x, q.y, q.z, q.w};
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) nibbles4_fma((words[i] >> sh) & 0x0f0f0f0fu, d, -8.0f * d, v + 4 * i);
    f0 = to_half8(v);
    f1 = to_half8(v + 8);
  }
};

enum GvMode { kGvStore = 0, kGvPartial = 1, kGvSwiGLU = 2 };

template <int TYPE, int MODE, int kGvTiles, bool TILED = false, int NG = 1>
__global__ __launch_bounds__(64 * kGvWaves) void gemv_kernel(const uint16_t* __restrict__ x, int ldx, QWeight w, int M,
                                                             void* __restrict__ out, int ldo) {
  using Raw = typename std::conditional<TYPE == kQ4_K, GvQ4K,
                                        typename std::conditional<TYPE == kQ6_K, GvQ6K, GvQ40>::type>::type;
  // T >= 2: P = T / 2 tiles of a 128-row group's first half and the P tiles
  // 64 rows later, G workgroups per group; T = 1 (not SwiGLU): 16 rows.
  // NG groups of 16 tokens (M <= 16 NG) share each decoded weight fragment.
  static_assert(kGvTiles >= 2 || MODE != kGvSwiGLU, "SwiGLU pairs gate and up tiles");
  constexpr int P = kGvTiles >= 2 ? kGvTiles / 2 : 1, G = kGvTiles >= 2 ? 4 / P : 8;
  static_assert(kGvWaves * 64 * 16 <= kGvXSlice, "a round's sums of a wave fit in its X region");
  __shared__ __attribute__((aligned(16))) uint8_t smem[kGvWaves * kGvXSlice];
  // wave index in a scalar register: the block and tile addresses below are
  // then uniform and the loads take scalar bases with 32-bit lane offsets
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = lane >> 4, c = lane & 15;
  const int N = w.n, nblocks = w.k >> 8;
  const int n0 = kGvTiles >= 2 ? 128 * (blockIdx.x / G) + 16 * P * (blockIdx.x % G) : 16 * blockIdx.x;
  const int blk = kGvWaves * blockIdx.y + wave;
  const size_t row_bytes = qweight_row_bytes(TYPE, w.k);
  uint8_t* sx = smem + wave * kGvXSlice;

  float4v acc[NG][kGvTiles];
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int t = 0; t < kGvTiles; ++t) acc[g][t] = float4v{0.f, 0.f, 0.f, 0.f};
  if (blk < nblocks) {
    // Load i of token group g: rows 2i, 2i + 1 of its 16 x 256 slice; lane l
    // takes slot l & 31 of row 2i + l / 32 (chunk (l & 31) ^ row).
    // Registers, then LDS: the compiler orders the wave's own LDS write and
    // reads.
    half8v xs[8];
    const uint8_t* xb = (const uint8_t*)(x + 256 * blk);  // uniform base, 32-bit lane offsets
    auto load_x = [&](int g) {
      const int t0 = lane >> 5, s = lane & 31;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int t = 2 * i + t0;
        xs[i] = *(const half8v*)(xb + 2u * (uint32_t)(min(16 * g + t, M - 1) * ldx + 8 * (s ^ t)));
      }
    };
    load_x(0);
    Raw raw[kGvTiles];
#pragma unroll
    for (int t = 0; t < kGvTiles; ++t) {
      if constexpr (TILED)  // N % 16 == 0: every tile's rows exist
        raw[t].load_tiled(w, (n0 + 16 * (t % P) + 64 * (t / P)) >> 4, c, blk, kq);
      else
        raw[t].load(w, row_bytes, min(n0 + 16 * (t % P) + 64 * (t / P) + c, N - 1), blk, kq);
    }
    half8v wf[kGvTiles][8];  // decoded fragments: run r -> 2r, 2r + 1
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
      for (int i = 0; i < 8; ++i) *(half8v*)(sx + 1024 * i + 16 * lane) = xs[i];
      if (g + 1 < NG) load_x(g + 1);
      half8v xa[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k = TYPE == kQ4_K ? gv_q4k_run_k(kq, r) : TYPE == kQ6_K ? gv_q6k_run_k(kq, r) : gv_q40_run_k(kq, r);
        xa[2 * r] = *(const half8v*)(sx + 512 * c + 16 * ((k >> 3) ^ c));
        xa[2 * r + 1] = *(const half8v*)(sx + 512 * c + 16 * (((k >> 3) + 1) ^ c));
      }
      // Tile by tile: the weight loads return in issue order, so the first
      // tile's decode and MFMAs start while the later tiles' bytes arrive.
#pragma unroll
      for (int t = 0; t < kGvTiles; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (g == 0) raw[t].run(kq, r, wf[t][2 * r], wf[t][2 * r + 1]);
          acc[g][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[2 * r], wf[t][2 * r], acc[g][t], 0, 0, 0);
          acc[g][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[2 * r + 1], wf[t][2 * r + 1], acc[g][t], 0, 0, 0);
        }
    }
  }
  // The 8 waves' sums are added in LDS in rounds of GR token groups (8 tile
  // sums of 1 KB per wave, in the wave's X region: its fragment reads came
  // first), each (tile, group) by one wave.
  constexpr int GR = kGvWaves / kGvTiles, ROUNDS = (NG + GR - 1) / GR;
  float4v* red = (float4v*)smem;  // round's sums: [wave][group - GR r][tile][lane] at wave * kGvXSlice
  // D layout: lane l, register i -> token 16 g + 4 (l / 16) + i, row l % 16 of the tile.
  auto tile_sum = [&](int pair) {
    float4v s = red[pair * 64 + lane];
#pragma unroll
    for (int v = 1; v < kGvWaves; ++v) s += red[v * (kGvXSlice / 16) + pair * 64 + lane];
    return s;
  };
#pragma unroll
  for (int r = 0; r < ROUNDS; ++r) {
    if (r > 0) __syncthreads();  // the previous round's sums have been read
#pragma unroll
    for (int gg = 0; gg < GR; ++gg)
      if (GR * r + gg < NG)
#pragma unroll
        for (int t = 0; t < kGvTiles; ++t)
          red[(wave * kGvXSlice / 16) + (gg * kGvTiles + t) * 64 + lane] = acc[min(GR * r + gg, NG - 1)][t];
    __syncthreads();
    if constexpr (MODE == kGvSwiGLU) {
      // wave -> gate tile wave % P (and its up tile) of group GR r + wave / P
      const int tp = wave % P, gg = wave / P, g = GR * r + gg;
      const int f = 64 * (blockIdx.x / G) + 16 * P * (blockIdx.x % G) + 16 * tp + c;
      if (gg < GR && g < NG && n0 + 16 * tp + c + 64 < N) {
        const float4v gs = tile_sum(gg * kGvTiles + tp), us = tile_sum(gg * kGvTiles + tp + P);
        uint16_t* y = (uint16_t*)out;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 16 * g + 4 * kq + i;
          if (m >= M) continue;
          const float gv = (float)(half_t)gs[i], uv = (float)(half_t)us[i];
          y[(size_t)m * ldo + f] = f2h(gv / (1.0f + expf(-gv)) * uv);
        }
      }
    } else {
      // wave -> tile wave % T of group GR r + wave / T
      const int t = wave % kGvTiles, g = GR * r + wave / kGvTiles;
      const int row = n0 + 16 * (t % P) + 64 * (t / P) + c;
      if (g < NG && row < N) {
        const float4v s = tile_sum(wave);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 16 * g + 4 * kq + i;
          if (m >= M) continue;
          if constexpr (MODE == kGvStore)
            ((uint16_t*)out)[(size_t)m * ldo + row] = f2h(s[i]);
          else
            ((float*)out)[((size_t)blockIdx.y * M + m) * N + row] = s[i];
        }
      }
    }
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

hipError_t launch_reduce_swiglu(const float* partials, int splits, int m, int n, uint16_t* y, int ldy,
                                hipStream_t stream) {
  const int64_t total = (int64_t)m * (n / 2);
  if (total <= 0) return hipSuccess;
  if (n % 128) return hipErrorInvalidValue;
  reduce_swiglu_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(partials, splits, m, n, y, ldy);
  return hipGetLastError();
}

int gemv_splits(const QWeight& w) {
  // One workgroup row covers 8 blocks (2048 values) of K.
  return ((w.k >> 8) + kGvWaves - 1) / kGvWaves;
}

size_t gemv_partials_floats(const QWeight& w, int m) {
  const int s = gemv_splits(w);
  return s > 1 ? (size_t)s * m * w.n : 0;
}

// One launch over NG >= ceil(m / 16) token groups (1, 2, 3, 4, 6, 8 or 10;
// groups past m are clamped loads whose sums are not stored).
template <int TYPE, int MODE, int T, bool TILED>
static void launch_gemv_groups(dim3 grid, const uint16_t* x, int ldx, const QWeight& w, int m, void* out, int ldo,
                               hipStream_t stream) {
  const int ng = (m + 15) / 16;
  if (ng == 1)
    gemv_kernel<TYPE, MODE, T, TILED, 1><<<grid, 64 * kGvWaves, 0, stream>>>(x, ldx, w, m, out, ldo);
  else if (ng == 2)
    gemv_kernel<TYPE, MODE, T, TILED, 2><<<grid, 64 * kGvWaves, 0, stream>>>(x, ldx, w, m, out, ldo);
  else if constexpr (T <= 2) {
    if (ng == 3)
      gemv_kernel<TYPE, MODE, T, TILED, 3><<<grid, 64 * kGvWaves, 0, stream>>>(x, ldx, w, m, out, ldo);
    else if (ng == 4)
      gemv_kernel<TYPE, MODE, T, TILED, 4><<<grid, 64 * kGvWaves, 0, stream>>>(x, ldx, w, m, out, ldo);
    else if (ng <= 6)
      gemv_kernel<TYPE, MODE, T, TILED, 6><<<grid, 64 * kGvWaves, 0, stream>>>(x, ldx, w, m, out, ldo);
    else if (ng <= 8)
      gemv_kernel<TYPE, MODE, T, TILED, 8><<<grid, 64 * kGvWaves, 0, stream>>>(x, ldx, w, m, out, ldo);
    else
      gemv_kernel<TYPE, MODE, T, TILED, 10><<<grid, 64 * kGvWaves, 0, stream>>>(x, ldx, w, m, out, ldo);
  }
}

template <int TYPE, int MODE>
static void launch_gemv_kernel(const uint16_t* x, int ldx, const QWeight& w, int m, void* out, int ldo,
                               hipStream_t stream) {
  const int groups = (w.n + 127) / 128, splits = gemv_splits(w);
  if (w.gv && w.n % 16 == 0) {
    // Tiled weights: 2 tiles per wave when that gives every CU a workgroup
    // (or for SwiGLU), else 1 (measured on Q4_K: 16384 x 2048 7.7 us on 2
    // tiles, 7.9 on 4; 2048 x 2048 3.7 us on 1 against 4.5 untiled).
    if (MODE == kGvSwiGLU || 4 * groups * splits >= 256) {
      launch_gemv_groups<TYPE, MODE, 2, true>(dim3(4 * groups, splits), x, ldx, w, m, out, ldo, stream);
    } else {
      if constexpr (MODE != kGvSwiGLU)
        launch_gemv_groups<TYPE, MODE, 1, true>(dim3(8 * groups, splits), x, ldx, w, m, out, ldo, stream);
    }
    return;
  }
  // 4 tiles per wave (X fragments reused 4 times) once that alone gives
  // every CU a workgroup and m <= 32 (more token groups of 4 tiles
  // outgrow the registers); else 2 when that does (or for
  // SwiGLU, whose gate and up tiles pair up); else 1, which spreads a small
  // matrix over the most CUs (2048 x 2048: 128 workgroups, 1.2x faster than
  // 64 of 2 tiles). A row's arithmetic is the same in every configuration.
  if (2 * groups * splits >= 256 && m <= 32) {
    launch_gemv_groups<TYPE, MODE, 4, false>(dim3(2 * groups, splits), x, ldx, w, m, out, ldo, stream);
  } else if (MODE == kGvSwiGLU || 4 * groups * splits >= 256) {
    launch_gemv_groups<TYPE, MODE, 2, false>(dim3(4 * groups, splits), x, ldx, w, m, out, ldo, stream);
  } else {
    if constexpr (MODE != kGvSwiGLU)
      launch_gemv_groups<TYPE, MODE, 1, false>(dim3(8 * groups, splits), x, ldx, w, m, out, ldo, stream);
  }
}

// Tiled copies for the GEMV (one thread per piece of row r, 256-value block
// b; layouts at the load_tiled functions above).
__global__ void tile_q4k_kernel(const uint8_t* __restrict__ src, int n, int nblocks, uint8_t* __restrict__ dst) {
  // piece p: 0 the header, 1-4 the first 64 nibble bytes, 5-8 the last 64
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)n * nblocks * 9) return;
  const int p = (int)(i % 9);
  const int64_t rb = i / 9;
  const int b = (int)(rb % nblocks), r = (int)(rb / nblocks), c = r & 15;
  const u32x4 v = *(const u32x4*)(src + ((size_t)r * nblocks + b) * 144 + 16 * p);
  uint8_t* base = dst + ((size_t)(r >> 4) * nblocks + b) * 2304;
  uint8_t* o = p == 0 ? base + 16 * c : p <= 4 ? base + 256 + 16 * (16 * (p - 1) + c) : base + 1280 + 16 * (16 * (p - 5) + c);
  *(u32x4*)o = v;
}

__global__ void tile_q6k_kernel(const uint8_t* __restrict__ rec, const uint16_t* __restrict__ dsrc, int n,
                                int nblocks, uint8_t* __restrict__ dst) {
  // piece p: 0-7 ql (16 bytes each), 8-11 qh, 12 the scales, 13 d
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)n * nblocks * 14) return;
  const int p = (int)(i % 14);
  const int64_t rb = i / 14;
  const int b = (int)(rb % nblocks), r = (int)(rb / nblocks), c = r & 15;
  const uint8_t* src = rec + ((size_t)r * nblocks + b) * 208;
  uint8_t* base = dst + ((size_t)(r >> 4) * nblocks + b) * 3360;
  if (p == 13) {
    *(uint16_t*)(base + 3328 + 2 * c) = dsrc[(size_t)r * nblocks + b];
    return;
  }
  const u32x4 v = *(const u32x4*)(src + 16 * p);
  uint8_t* o;
  if (p < 8) {  // ql bytes 16p: kq = p / 2 (h = kq / 2, qa = kq % 2), second half when p is odd
    o = base + (p & 1) * 1024 + 16 * (16 * (p >> 1) + c);
  } else if (p < 12) {  // qh bytes 128 + 16 (p - 8): half (p - 8) / 2, second half when p is odd
    o = base + 2048 + (p & 1) * 512 + 16 * (16 * ((p - 8) >> 1) + c);
  } else {
    o = base + 3072 + 16 * c;
  }
  *(u32x4*)o = v;
}

__global__ void tile_q40_kernel(const uint8_t* __restrict__ nib, const uint16_t* __restrict__ dsrc, int n,
                                int nblocks, uint8_t* __restrict__ dst) {
  // piece p of a 256-value block: 0-7 the eight 16-byte nibble blocks, 8-11 the scale pairs
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)n * nblocks * 12) return;
  const int p = (int)(i % 12);
  const int64_t rb = i / 12;
  const int b = (int)(rb % nblocks), r = (int)(rb / nblocks), c = r & 15;
  uint8_t* base = dst + ((size_t)(r >> 4) * nblocks + b) * 2304;
  if (p < 8) {  // Q4_0 block 8b + p: pair kq = p / 2, second of the pair when p is odd
    const u32x4 v = *(const u32x4*)(nib + ((size_t)r * nblocks * 8 + 8 * b + p) * 16);
    *(u32x4*)(base + (p & 1) * 1024 + 16 * (16 * (p >> 1) + c)) = v;
  } else {
    const int kq = p - 8;
    const uint16_t* d = dsrc + (size_t)r * nblocks * 8 + 8 * b + 2 * kq;
    *(uint32_t*)(base + 2048 + 4 * (16 * kq + c)) = (uint32_t)d[0] | ((uint32_t)d[1] << 16);
  }
}

size_t gemv_tile_bytes(const QWeight& w) {
  if (w.n <= 0 || w.n % 16 || w.k <= 0 || w.k % 256) return 0;
  const size_t tiles = (size_t)(w.n / 16) * (w.k / 256);
  return w.type == kQ4_K ? tiles * 2304 : w.type == kQ6_K ? tiles * 3360 : w.type == kQ4_0 ? tiles * 2304 : 0;
}

hipError_t launch_tile_gemv(const QWeight& w, uint8_t* out, hipStream_t stream) {
  if (!gemv_tile_bytes(w)) return hipErrorInvalidValue;
  const int nb = w.k / 256;
  const int64_t rows_blocks = (int64_t)w.n * nb;
  if (w.type == kQ4_K) {
    tile_q4k_kernel<<<(unsigned)((rows_blocks * 9 + 255) / 256), 256, 0, stream>>>(w.blocks, w.n, nb, out);
  } else if (w.type == kQ6_K) {
    if (!w.d) return hipErrorInvalidValue;
    tile_q6k_kernel<<<(unsigned)((rows_blocks * 14 + 255) / 256), 256, 0, stream>>>(w.blocks, w.d, w.n, nb, out);
  } else {
    if (!w.d) return hipErrorInvalidValue;
    tile_q40_kernel<<<(unsigned)((rows_blocks * 12 + 255) / 256), 256, 0, stream>>>(w.blocks, w.d, w.n, nb, out);
  }
  return hipGetLastError();
}

template <int MODE>
static void launch_gemv_typed(const uint16_t* x, int ldx, const QWeight& w, int m, void* out, int ldo,
                              hipStream_t stream) {
  if (w.type == kQ4_K) launch_gemv_kernel<kQ4_K, MODE>(x, ldx, w, m, out, ldo, stream);
  else if (w.type == kQ6_K) launch_gemv_kernel<kQ6_K, MODE>(x, ldx, w, m, out, ldo, stream);
  else launch_gemv_kernel<kQ4_0, MODE>(x, ldx, w, m, out, ldo, stream);
}

hipError_t launch_gemv_ex(const uint16_t* x, int ldx, const QWeight& w, int m, int epilogue, void* out, int ldo,
                          float* partials, hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  if (m > kGemvMaxM || (w.type != kQ4_K && w.type != kQ6_K && w.type != kQ4_0)) return hipErrorInvalidValue;
  if (epilogue == kEpiSwiGLU && w.n % 128) return hipErrorInvalidValue;
  // The kernel addresses X with 32-bit byte offsets.
  if (ldx < w.k || 2 * ((int64_t)(m - 1) * ldx + w.k) > INT32_MAX) return hipErrorInvalidValue;
  const int splits = gemv_splits(w);
  if (epilogue == kEpiPartial) {
    // [splits][m][n] fp32 sums into `out` (row stride n)
    if (ldo != w.n || out == nullptr) return hipErrorInvalidValue;
    launch_gemv_typed<kGvPartial>(x, ldx, w, m, out, ldo, stream);
    return hipGetLastError();
  }
  if (splits == 1) {
    if (epilogue == kEpiStore) launch_gemv_typed<kGvStore>(x, ldx, w, m, out, ldo, stream);
    else launch_gemv_typed<kGvSwiGLU>(x, ldx, w, m, out, ldo, stream);
    return hipGetLastError();
  }
  if (partials == nullptr) return hipErrorInvalidValue;
  launch_gemv_typed<kGvPartial>(x, ldx, w, m, partials, w.n, stream);
  if (epilogue == kEpiStore) return launch_reduce_partials(partials, splits, m, w.n, (uint16_t*)out, ldo, stream);
  return launch_reduce_swiglu(partials, splits, m, w.n, (uint16_t*)out, ldo, stream);
}

hipError_t launch_gemv(const uint16_t* x, int ldx, const QWeight& w, uint16_t* y, int ldy, int m, float* partials,
                       hipStream_t stream) {
  return launch_gemv_ex(x, ldx, w, m, kEpiStore, y, ldy, partials, stream);
}

// ---------------------------------------------------------------------------
// Standalone decoding.
// ---------------------------------------------------------------------------

template <bool NT>
__global__ __launch_bounds__(256) void dequant_q4k_kernel(const uint8_t* __restrict__ raw, int64_t n_blocks,
                                                          float* __restrict__ out32, uint16_t* __restrict__ out16) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = t >> 3;
  if (b >= n_blocks) return;
  q4k_block_part<NT>(raw + b * 144, (int)(t & 7), b * 256, out32, out16);
}

// Two matrices in one launch: blocks [0, n0) of raw0 to out0, then the n1 of
// raw1 to out1 (f16, row-major; small expansions are latency-bound alone).
__global__ __launch_bounds__(256) void expand_q4k_pair_kernel(const uint8_t* __restrict__ raw0, int64_t n0,
                                                              uint16_t* __restrict__ out0,
                                                              const uint8_t* __restrict__ raw1, int64_t n1,
                                                              uint16_t* __restrict__ out1) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t b = t >> 3;
  if (b < n0) {
    q4k_block_part<false>(raw0 + b * 144, (int)(t & 7), b * 256, nullptr, out0);
  } else if ((b -= n0) < n1) {
    q4k_block_part<false>(raw1 + b * 144, (int)(t & 7), b * 256, nullptr, out1);
  }
}

hipError_t launch_expand_q4k_pair(const uint8_t* blocks0, int64_t n0, uint16_t* out0, const uint8_t* blocks1,
                                  int64_t n1, uint16_t* out1, hipStream_t stream) {
  if (n0 + n1 <= 0) return hipSuccess;
  expand_q4k_pair_kernel<<<(unsigned)(((n0 + n1) * 8 + 255) / 256), 256, 0, stream>>>(blocks0, n0, out0, blocks1, n1,
                                                                                        out1);
  return hipGetLastError();
}

hipError_t launch_expand_q4k(const uint8_t* blocks, int64_t n_blocks, uint16_t* out16, hipStream_t stream) {
  if (n_blocks <= 0) return hipSuccess;
  dequant_q4k_kernel<false><<<(unsigned)((n_blocks * 8 + 255) / 256), 256, 0, stream>>>(blocks, n_blocks, nullptr,
                                                                                        out16);
  return hipGetLastError();
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
    dequant_q4k_kernel<true><<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(raw, n_blocks, out32, out16);
  } else if (type == kQ6_K) {
    dequant_q6k_kernel<<<(unsigned)((n_blocks + kQ6Span - 1) / kQ6Span), 256, 0, stream>>>(raw, n_blocks, out32, out16);
  } else if (type == kQ4_0) {
    dequant_q40_kernel<<<(unsigned)((n_blocks + kQ40Span - 1) / kQ40Span), 256, 0, stream>>>(raw, n_blocks, out32, out16);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Q6_K split layout -> f16, row-major (the two-pass GEMM's first pass):
// 8 threads per 256-value block, thread c writing chunks c + 8 i of 8
// values, so 8 neighbouring lanes fill 128 contiguous bytes per store. Value
// 64 i + 8 c + j is (half h = i / 2, quadrant Q = 2 (i % 2) + c / 4, lane
// l = 8 (c % 4) + j) (src/gguf/quantization.ts:53-71): its low bits are the
// low (Q < 2) or high nibble of ql[64 h + 8 c + j], its high bits bits 2Q of
// qh[32 h + 8 (c % 4) + j], its scale sc[8 h + (c % 4) / 2 + 2 Q].
__global__ __launch_bounds__(256) void expand_q6k_kernel(QWeight w, uint16_t* __restrict__ out16) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = t >> 3;
  if (b >= (int64_t)w.n * (w.k >> 8)) return;
  q6k_block_part(w.blocks + b * 208, w.d[b], (int)(t & 7), out16 + b * 256);
}

hipError_t launch_expand_q6k(const QWeight& w, uint16_t* out16, hipStream_t stream) {
  const int64_t threads = (int64_t)w.n * (w.k / 256) * 8;
  if (threads <= 0) return hipSuccess;
  expand_q6k_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(w, out16);
  return hipGetLastError();
}

SidePart side_part_range(const SidePart& p, int64_t first, int64_t count) {
  SidePart r = p;
  first = std::max<int64_t>(0, std::min(first, p.nblocks));
  r.nblocks = std::max<int64_t>(0, std::min(count, p.nblocks - first));
  r.blocks = p.blocks + first * (p.type == kQ4_K ? 144 : 208);
  if (p.d) r.d = p.d + first;
  r.out = p.out + first * 256;
  return r;
}

SidePart side_part_of(const QWeight& w, uint16_t* out) {
  SidePart e;
  if (w.k % 256 || (w.type != kQ4_K && w.type != kQ6_K) || (w.type == kQ6_K && !w.d)) return e;
  e.type = w.type;
  e.blocks = w.blocks;
  e.d = w.d;
  e.nblocks = (int64_t)w.n * (w.k / 256);
  e.out = out;
  return e;
}

__global__ __launch_bounds__(256) void side_expand_kernel(SideExpand e) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if ((t >> 3) < e.nblocks) side_expand_part(e, t >> 3, (int)(t & 7));
}

hipError_t launch_side_expand(const SideExpand& e, hipStream_t stream) {
  if (e.count == 0 || e.nblocks <= 0) return hipSuccess;
  side_expand_kernel<<<(unsigned)((e.nblocks * 8 + 255) / 256), 256, 0, stream>>>(e);
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

// Q4_0 split layout: thread per 32-value block.
__global__ void dequant_q40_split_kernel(QWeight w, int64_t n_blocks, float* __restrict__ out32) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const u32x4 q = *(const u32x4*)(w.blocks + b * 16);
  const float d = h2f(w.d[b]);
  const uint32_t words[4] = {q.x, q.y, q.z, q.w};
  float v[32];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bytes4_fma(words[i] & 0x0f0f0f0fu, d, -8.0f * d, v + 4 * i);
    bytes4_fma((words[i] >> 4) & 0x0f0f0f0fu, d, -8.0f * d, v + 16 + 4 * i);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) *(float4v*)(out32 + b * 32 + 4 * i) = float4v{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
}

hipError_t launch_dequant_weight(const QWeight& w, float* out32, hipStream_t stream) {
  const int64_t nb = (int64_t)w.n * (w.k / 256);
  if (w.type == kQ4_K) return launch_dequant_raw(kQ4_K, w.blocks, nb, out32, nullptr, stream);
  if (w.type == kQ4_0) {
    const int64_t n40 = (int64_t)w.n * (w.k / 32);
    dequant_q40_split_kernel<<<(unsigned)((n40 + 255) / 256), 256, 0, stream>>>(w, n40, out32);
    return hipGetLastError();
  }
  if (w.type != kQ6_K) return hipErrorInvalidValue;
  const int64_t threads = nb * 8;
  dequant_q6k_split_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(w, out32);
  return hipGetLastError();
}

}  // namespace nemo
