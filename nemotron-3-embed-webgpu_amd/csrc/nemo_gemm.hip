// Dequant + MFMA GEMM for gfx950: Y[M, N] = X[M, K] * W[N, K]^T with W in
// Q4_K (GGUF blocks) or Q6_K (split layout), X f16, fp32 accumulate.
//
// Three kernels share the decode, the epilogues and the split-K contract:
//  * gemm_kernel<BM>: BM x 128 x 64 tiles (BM 128 or 256), 4 waves, both
//    operands staged in LDS through registers, W decoded in the kernel.
//  * gemm_big_kernel: 256 x 256 x 64 tiles, 8 waves of 64 x 128, X copied
//    global -> LDS directly, W decoded in the kernel (Q4_K, large problems).
//  * expand_kernel + gemm_f16_kernel (two-pass): W expanded to f16 once per
//    call, then 256 x 256 x 64 tiles with both operands copied global -> LDS.
// Every wave owns whole 128-column groups, so the gate/up projection finishes
// SwiGLU in registers: the plan stores gate_up with rows interleaved per
// 128-row group (64 gate rows, then the matching 64 up rows), and a lane
// holds g and u of the same (token, feature) in column blocks j and j+2.
//
// Split-K: blockIdx.z selects a contiguous K range; partial sums are written
// as fp32 and summed in a fixed order by the consumer (deterministic). The
// split count depends only on the weight's shape, never on M, and every row's
// K order is the same in every kernel (sequential 16-column MFMA steps on the
// same f16 operands), so all paths give identical bits and a
// token's result does not depend on how many other tokens share the batch.
#include <algorithm>
#include <mutex>
#include <type_traits>
#include <unordered_map>
#include <vector>

#include "nemo_blocks.h"
#include "nemo_common.h"
#include "nemo_quant.h"

namespace nemo {

constexpr int kBK = 64, kLdsK = kBK + 8;

template <int TYPE>
struct WFetch;
template <>
struct WFetch<kQ4_K> {
  Q4KFetch f;
  __device__ __forceinline__ void load(const QWeight& w, size_t rb, int row, int k0, int p) {
    f = q4k_fetch(w, rb, row, k0, p);
  }
  __device__ __forceinline__ void expand(half8v* lo, half8v* hi) const { q4k_expand(f, lo, hi); }
};
template <>
struct WFetch<kQ6_K> {
  Q6KFetch f;
  __device__ __forceinline__ void load(const QWeight& w, size_t rb, int row, int k0, int p) {
    f = q6k_fetch(w, rb, row, k0, p);
  }
  __device__ __forceinline__ void expand(half8v* lo, half8v* hi) const { q6k_expand(f, lo, hi); }
};

template <>
struct WFetch<kQ4_0> {
  Q40Fetch f;
  __device__ __forceinline__ void load(const QWeight& w, size_t rb, int row, int k0, int p) {
    f = q40_fetch(w, rb, row, k0, p);
  }
  __device__ __forceinline__ void expand(half8v* lo, half8v* hi) const { q40_expand(f, lo, hi); }
};

// Epilogue for a wave owning MI x 4 blocks of 32 x 32 starting at (rbase0,
// cbase): lane l, register r of block (i, j) is row rbase0 + 32i + 8(r/4) +
// 4(l/32) + r%4, column cbase + 32j + l%32. `split`: the K split whose fp32
// partials kEpiPartial writes.
template <int EPI, int MI>
__device__ __forceinline__ void gemm_epilogue(const float16v (&acc)[MI][4], int rbase0, int cbase, int lane, int M,
                                              int N, void* out, int ldo, int split) {
  const int rbase = rbase0 + 4 * (lane >> 5);
  if constexpr (EPI == kEpiSwiGLU) {
    // Columns j*32 + l%32 (j = 0, 1) of this wave's 128 are gate features
    // cbase/2 + j*32 + l%32; columns 64 + j*32 + l%32 are their up rows.
    // SwiGLU as src/webgpu/ops.ts:85-87 on the f16-rounded gate/up values.
    uint16_t* y = (uint16_t*)out;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int col = (cbase >> 1) + j * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = rbase + i * 32 + 8 * (r >> 2) + (r & 3);
          if (row < M) {
            const float g = (float)(half_t)acc[i][j][r];
            const float u = (float)(half_t)acc[i][j + 2][r];
            y[(size_t)row * ldo + col] = f2h(g / (1.0f + expf(-g)) * u);
          }
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = cbase + j * 32 + (lane & 31);
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = rbase + i * 32 + 8 * (r >> 2) + (r & 3);
          if (row >= M) continue;
          if constexpr (EPI == kEpiStore)
            ((uint16_t*)out)[(size_t)row * ldo + col] = f2h(acc[i][j][r]);
          else if constexpr (EPI == kEpiPartial16)
            ((uint16_t*)out)[((size_t)split * M + row) * ldo + col] = f2h(acc[i][j][r]);
          else
            ((float*)out)[((size_t)split * M + row) * ldo + col] = acc[i][j][r];
        }
      }
  }
}

// The same epilogue for a wave owning MI16 x 8 blocks of 16 x 16 starting at
// (rbase0, cbase): lane l, register r of block (i, j) is row rbase0 + 16i +
// 4(l/16) + r, column cbase + 16j + l%16. For kEpiSwiGLU blocks j < 4 are the
// gate features cbase/2 + 16j + l%16 and blocks j + 4 their up rows.
template <int EPI, int MI16>
__device__ __forceinline__ void gemm_epilogue16(const float4v (&acc)[MI16][8], int rbase0, int cbase, int lane, int M,
                                                int N, void* out, int ldo, int split) {
  const int rbase = rbase0 + 4 * (lane >> 4);
  if constexpr (EPI == kEpiSwiGLU) {
    uint16_t* y = (uint16_t*)out;
#pragma unroll
    for (int i = 0; i < MI16; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = (cbase >> 1) + j * 16 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rbase + i * 16 + r;
          if (row < M) {
            const float g = (float)(half_t)acc[i][j][r];
            const float u = (float)(half_t)acc[i][j + 4][r];
            y[(size_t)row * ldo + col] = f2h(g / (1.0f + expf(-g)) * u);
          }
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < MI16; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int col = cbase + j * 16 + (lane & 15);
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rbase + i * 16 + r;
          if (row >= M) continue;
          if constexpr (EPI == kEpiStore)
            ((uint16_t*)out)[(size_t)row * ldo + col] = f2h(acc[i][j][r]);
          else if constexpr (EPI == kEpiPartial16)
            ((uint16_t*)out)[((size_t)split * M + row) * ldo + col] = f2h(acc[i][j][r]);
          else
            ((float*)out)[((size_t)split * M + row) * ldo + col] = acc[i][j][r];
        }
      }
  }
}

// ---------------------------------------------------------------------------
// LDS-staged tiles: BM x 128 x 64 (BM = 128 or 256), 4 waves along M, each
// BM/4 x 128. Per K step every thread loads its share of X (8 threads per
// row, 16 bytes each: coalesced 128-byte row segments) and the raw weight
// bytes of its half row into registers; after the barrier it decodes, stores
// both tiles to LDS (rows padded to 72 halves so fragment reads of 32
// consecutive rows hit distinct banks), and the loads of the next step are
// issued before the MFMAs of this one.
// ---------------------------------------------------------------------------

template <int TYPE, int BM, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const uint16_t* __restrict__ x, int ldx, QWeight w, int M,
                                                   int kchunk, void* __restrict__ out, int ldo) {
  constexpr int BN = 128, WM = BM / 4, MI = WM / 32, XP = BM / 32;
  __shared__ __attribute__((aligned(16))) half_t sA[BM * kLdsK];
  __shared__ __attribute__((aligned(16))) half_t sB[BN * kLdsK];
  const int N = w.n;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int kbeg = blockIdx.z * kchunk, kend = kbeg + kchunk;
  const size_t row_bytes = qweight_row_bytes(TYPE, w.k);

  const int xr = tid >> 3, xc = (tid & 7) * 8;
  const uint16_t* xrow[XP];
#pragma unroll
  for (int i = 0; i < XP; ++i) xrow[i] = x + (size_t)min(m0 + i * 32 + xr, M - 1) * ldx + xc;
  const int wr = tid >> 1, wp = tid & 1;
  const int wrow = min(n0 + wr, N - 1);

  u32x4 xa[XP];
  WFetch<TYPE> wf;
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < XP; ++i) xa[i] = *(const u32x4*)(xrow[i] + k0);
    wf.load(w, row_bytes, wrow, k0, wp);
  };

  float16v acc[MI][4];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  fetch(kbeg);
  for (int k0 = kbeg; k0 < kend; k0 += kBK) {
    half8v lo[2], hi[2];
    wf.expand(lo, hi);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < XP; ++i) *(u32x4*)&sA[(i * 32 + xr) * kLdsK + xc] = xa[i];
    half_t* brow = &sB[wr * kLdsK];
    *(half8v*)(brow + 16 * wp) = lo[0];
    *(half8v*)(brow + 16 * wp + 8) = lo[1];
    *(half8v*)(brow + 32 + 16 * wp) = hi[0];
    *(half8v*)(brow + 32 + 16 * wp + 8) = hi[1];
    __syncthreads();
    if (k0 + kBK < kend) fetch(k0 + kBK);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int kk = ks * 16 + (lane >> 5) * 8;
      half8v af[MI], bf[4];
#pragma unroll
      for (int i = 0; i < MI; ++i) af[i] = *(const half8v*)&sA[(wave * WM + i * 32 + (lane & 31)) * kLdsK + kk];
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = *(const half8v*)&sB[(j * 32 + (lane & 31)) * kLdsK + kk];
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }
  gemm_epilogue<EPI, MI>(acc, m0 + wave * WM, n0, lane, M, N, out, ldo, blockIdx.z);
}

// ---------------------------------------------------------------------------
// Mid-size batches: 64 x 128 x 64 tiles, 4 waves (2 along M x 2 along N) of
// 32 rows x 64 columns. Wave (wm, wn) owns column blocks wn and wn + 2 of
// 32, so the gate and up rows of the same features (64 apart in the
// interleaved gate/up layout) meet in one wave for the SwiGLU epilogue. With
// few workgroups per CU a step is bound by memory latency, which the
// 1-step-ahead loads of gemm_kernel expose every step; here the raw X and W
// bytes of the next kMidDepth - 1 steps are in flight in registers while a
// step decodes into LDS (double-buffered, one barrier per step) and runs its
// MFMAs. The MFMA sequence per output element is the one above.
// ---------------------------------------------------------------------------

constexpr int kMidDepth = 4, kMidBM = 64;

template <int TYPE, int EPI>
// (x is not __restrict__: a restrict read-only pointer's loads may move across
// the compiler fences below.)
__global__ __launch_bounds__(256) void gemm_mid_kernel(const uint16_t* x, int ldx, QWeight w, int M,
                                                       int kchunk, void* __restrict__ out, int ldo, int ntx, int nty,
                                                       int ntiles, SideExpand side) {
  constexpr int BM = kMidBM, BN = 128, D = kMidDepth;
  static_assert(D % 2 == 0, "the LDS buffer of step s + u is u % 2");
  __shared__ __attribute__((aligned(16))) half_t sA[2][BM * kLdsK];
  __shared__ __attribute__((aligned(16))) half_t sB[2][BN * kLdsK];
  // One-dimensional grid: workgroup i < ntiles computes tile (i % ntx,
  // i / ntx % nty) of K split i / (ntx nty); the workgroups past the tiles
  // do `side` (as gemm_f16_kernel's).
  const int tile = blockIdx.x;
  if (tile >= ntiles) {
    const int nside = gridDim.x - ntiles;
    for (int64_t b = (int64_t)(tile - ntiles) * 32 + (threadIdx.x >> 3); b < side.nblocks; b += (int64_t)nside * 32)
      side_expand_part(side, b, (int)(threadIdx.x & 7));
    return;
  }
  const int bx = tile % ntx, by = tile / ntx % nty, bz = tile / (ntx * nty);
  const int N = w.n;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = by * BM, n0 = bx * BN;
  const int kbeg = bz * kchunk;
  const int nsteps = kchunk / kBK;
  const size_t row_bytes = qweight_row_bytes(TYPE, w.k);

  // X: 4 threads per row, 32 bytes each; W: 2 threads per weight row.
  const int xr = tid >> 2, xc = (tid & 3) * 16;
  const uint16_t* xrow = x + (size_t)min(m0 + xr, M - 1) * ldx + xc;
  const int wr = tid >> 1, wp = tid & 1;
  const int wrow = min(n0 + wr, N - 1);

  u32x4 xa[D][2];
  WFetch<TYPE> wf[D];
  auto kat = [&](int s) { return kbeg + min(s, nsteps - 1) * kBK; };
  auto fetch = [&](int slot, int k0) {
    xa[slot][0] = *(const u32x4*)(xrow + k0);
    xa[slot][1] = *(const u32x4*)(xrow + k0 + 8);
    wf[slot].load(w, row_bytes, wrow, k0, wp);
  };

  float16v acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;

  // Loads are issued in step order, which the waits count on: neither the
  // optimizer (memory clobber) nor the scheduler may move them across steps.
  auto fence = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
#pragma unroll
  for (int i = 0; i < D - 1; ++i) {
    fetch(i, kat(i));
    fence();
  }
  for (int s = 0; s < nsteps; s += D) {  // nsteps is a multiple of D (host check)
#pragma unroll
    for (int u = 0; u < D; ++u) {
      // Each step's decode stays in its step: hoisted into an earlier one it
      // would wait there for loads that are meant to still be in flight.
      fence();
      half8v lo[2], hi[2];
      wf[u].expand(lo, hi);
      half_t* arow = &sA[u & 1][xr * kLdsK + xc];
      *(u32x4*)arow = xa[u][0];
      *(u32x4*)(arow + 8) = xa[u][1];
      half_t* brow = &sB[u & 1][wr * kLdsK];
      *(half8v*)(brow + 16 * wp) = lo[0];
      *(half8v*)(brow + 16 * wp + 8) = lo[1];
      *(half8v*)(brow + 32 + 16 * wp) = hi[0];
      *(half8v*)(brow + 32 + 16 * wp + 8) = hi[1];
      fence();
      fetch((u + D - 1) % D, kat(s + u + D - 1));
      fence();
      __syncthreads();
      const half_t* as = sA[u & 1];
      const half_t* bs = sB[u & 1];
#pragma unroll
      for (int ks = 0; ks < kBK / 16; ++ks) {
        const int kk = ks * 16 + (lane >> 5) * 8;
        const half8v af = *(const half8v*)&as[(wm * 32 + (lane & 31)) * kLdsK + kk];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const half8v bf = *(const half8v*)&bs[((wn + 2 * j) * 32 + (lane & 31)) * kLdsK + kk];
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[j], 0, 0, 0);
        }
      }
    }
  }

  // lane l, register r: row 32 wm + 8 (r / 4) + 4 (l / 32) + r % 4, column
  // 32 (wn + 2 j) + l % 32 of the tile (gemm_epilogue's layout).
  const int rbase = m0 + wm * 32 + 4 * (lane >> 5);
  if constexpr (EPI == kEpiSwiGLU) {
    const int col = (n0 >> 1) + 32 * wn + (lane & 31);
    uint16_t* y = (uint16_t*)out;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = rbase + 8 * (r >> 2) + (r & 3);
      if (row < M) {
        const float g = (float)(half_t)acc[0][r];
        const float u = (float)(half_t)acc[1][r];
        y[(size_t)row * ldo + col] = f2h(g / (1.0f + expf(-g)) * u);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + 32 * (wn + 2 * j) + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = rbase + 8 * (r >> 2) + (r & 3);
        if (row >= M) continue;
        if constexpr (EPI == kEpiStore)
          ((uint16_t*)out)[(size_t)row * ldo + col] = f2h(acc[j][r]);
        else if constexpr (EPI == kEpiPartial16)
          ((uint16_t*)out)[((size_t)bz * M + row) * ldo + col] = f2h(acc[j][r]);
        else
          ((float*)out)[((size_t)bz * M + row) * ldo + col] = acc[j][r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Large tiles: 256 x 256 x 64, 8 waves (4 along M x 2 along N), each 64 x 128,
// two waves per SIMD so one wave's decode overlaps the other's MFMAs.
//  * X: each K step's 256 x 64 tile is copied HBM/L2 -> LDS by
//    global_load_lds_dwordx4 (no registers, no VALU): one wave instruction
//    moves 8 whole 128-byte row segments (8 lanes per row). In LDS a row is 8
//    slots of 16 bytes; logical chunk c of row r sits in slot c ^ f(r), f(r)
//    = (r & 7) ^ ((r >> 3) & 1), so A-fragment reads (32 rows, one chunk) hit
//    distinct banks for 32- or 64-bank LDS.
//  * W: two threads per weight row decode it into a padded LDS tile. Raw
//    bytes use two register sets; the set for step s+3 is loaded right after
//    the barrier that closes step s.
// X and W tiles are double-buffered: the copy of step k+2 and the decode of
// step k+1 run under the MFMAs of step k, and every global access has a
// whole step to land before the vmcnt(0) that precedes the step's barrier.
// LDS: 2 x 32 KB (X) + 2 x 36 KB (W) = 138 KB, dynamic.
// ---------------------------------------------------------------------------

constexpr int kBigBM = 256, kBigBN = 256;
constexpr int kBigXStage = kBigBM * kBK * 2;    // bytes
constexpr int kBigWStage = kBigBN * kLdsK * 2;  // bytes
constexpr int kBigLds = 2 * kBigXStage + 2 * kBigWStage;

__device__ __forceinline__ int xswz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

typedef __attribute__((address_space(3))) void lds_void;

template <int TYPE, int EPI>
__global__ __launch_bounds__(512) void gemm_big_kernel(const uint16_t* __restrict__ x, int ldx, QWeight w, int M,
                                                       int kchunk, void* __restrict__ out, int ldo) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* sX = smem;                             // [2][256 rows][128 B]
  half_t* sW = (half_t*)(smem + 2 * kBigXStage);  // [2][256][72]
  constexpr int MI = 2;
  const int N = w.n;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const int m0 = blockIdx.y * kBigBM, n0 = blockIdx.x * kBigBN;
  const int kbeg = blockIdx.z * kchunk;
  const int nsteps = kchunk / kBK;
  const size_t row_bytes = qweight_row_bytes(TYPE, w.k);

  // X copy: wave w moves rows [32w, 32w + 32) in 4 instructions of 8 rows;
  // lane l -> row R + l/8, slot l%8, which holds logical chunk
  // (l%8) ^ f(row).
  const uint16_t* xsrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 32 * wave + 8 * i + (lane >> 3);
    const int c = (lane & 7) ^ xswz(r);
    xsrc[i] = x + (size_t)min(m0 + r, M - 1) * ldx + 8 * c;
  }
  auto copy_x = [&](int stage, int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(xsrc[i] + k0),
                                       (lds_void*)(sX + stage * kBigXStage + (32 * wave + 8 * i) * 128), 16, 0, 0);
  };

  // W decode: 2 threads per weight row.
  const int wr = tid >> 1, wp = tid & 1;
  const int wrow = min(n0 + wr, N - 1);
  WFetch<TYPE> ra, rb;  // raw bytes of even / odd steps
  auto store_w = [&](const WFetch<TYPE>& f, int stage) {
    half8v lo[2], hi[2];
    f.expand(lo, hi);
    half_t* brow = sW + stage * (kBigBN * kLdsK) + wr * kLdsK;
    *(half8v*)(brow + 16 * wp) = lo[0];
    *(half8v*)(brow + 16 * wp + 8) = lo[1];
    *(half8v*)(brow + 32 + 16 * wp) = hi[0];
    *(half8v*)(brow + 32 + 16 * wp + 8) = hi[1];
  };

  float16v acc[MI][4];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  auto mfma_step = [&](int stage) {
    const uint8_t* xs = sX + stage * kBigXStage;
    const half_t* ws = sW + stage * (kBigBN * kLdsK);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int c = 2 * ks + (lane >> 5);
      half8v af[MI], bf[4];
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int r = wm * 64 + i * 32 + (lane & 31);
        af[i] = *(const half8v*)(xs + r * 128 + 16 * (c ^ xswz(r)));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = *(const half8v*)(ws + (wn * 128 + j * 32 + (lane & 31)) * kLdsK + 8 * c);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  // One MFMA pair, then some of the decode's VALU work and LDS traffic.
  auto interleave = [] {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
    }
  };

  auto kat = [&](int s) { return kbeg + min(s, nsteps - 1) * kBK; };
  copy_x(0, kat(0));
  ra.load(w, row_bytes, wrow, kat(0), wp);
  copy_x(1, kat(1));
  rb.load(w, row_bytes, wrow, kat(1), wp);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  store_w(ra, 0);
  ra.load(w, row_bytes, wrow, kat(2), wp);
  __syncthreads();
  for (int s = 0; s < nsteps; s += 2) {
    // even step s: stage 0 holds X(s), W(s); rb holds raw(s+1); ra is
    // receiving raw(s+2).
    mfma_step(0);
    store_w(rb, 1);
    interleave();
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    copy_x(0, kat(s + 2));
    rb.load(w, row_bytes, wrow, kat(s + 3), wp);
    // odd step s+1: stage 1 holds X(s+1), W(s+1); ra holds raw(s+2).
    mfma_step(1);
    store_w(ra, 0);
    interleave();
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    copy_x(1, kat(s + 3));
    ra.load(w, row_bytes, wrow, kat(s + 4), wp);
  }
  // The last (clamped, unused) copies must land before the workgroup's LDS
  // is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  gemm_epilogue<EPI, MI>(acc, m0 + wm * 64, n0 + wn * 128, lane, M, N, out, ldo, blockIdx.z);
}

// ---------------------------------------------------------------------------
// Two-pass path for large batches. A bandwidth-bound pre-pass expands W to an
// f16 [n][k] matrix with the same decoders the fused kernels use (identical
// f16 values), then gemm_f16_kernel runs 256 x BN x 64 tiles (BN 256 or 128)
// with both operands copied global -> LDS by global_load_lds_dwordx4 into the
// swizzled layout described above, 4 x BN/128 waves of 64 x 128. Each wave
// issues the same MFMA sequence per output element as the fused kernels
// (16-column steps in K order), so the two paths give bit-identical results.
// ---------------------------------------------------------------------------

template <int TYPE>
__global__ __launch_bounds__(256) void expand_kernel(QWeight w, uint16_t* __restrict__ out) {
  // Thread t: row t / (k/32), 64-column chunk (t % (k/32)) / 2, part t % 2.
  const int per_row = w.k >> 5;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)w.n * per_row) return;
  const int row = (int)(t / per_row), i = (int)(t % per_row);
  const int k0 = 64 * (i >> 1), p = i & 1;
  WFetch<TYPE> f;
  f.load(w, qweight_row_bytes(TYPE, w.k), row, k0, p);
  half8v lo[2], hi[2];
  f.expand(lo, hi);
  uint16_t* dst = out + (size_t)row * w.k + k0 + 16 * p;
  *(half8v*)dst = lo[0];
  *(half8v*)(dst + 8) = lo[1];
  *(half8v*)(dst + 32) = hi[0];
  *(half8v*)(dst + 40) = hi[1];
}

// gemm_f16_kernel<EPI, BN, WM, MI>: BM x BN x 64 tiles, BM = 32 MI WM, with
// WM waves along M (32 MI rows each) x BN/128 along N (128 columns each).
// LDS: two stages of the BM x 64 X tile and the BN x 64 W tile (128 bytes
// per row). Configurations: 256 x 256 (8 waves of 64 x 128), 256 x 128 (4
// waves of 64 x 128), 192 x 256 (4 waves of 96 x 128), 384 x 256 (8 waves of
// 96 x 128), 192 x 128 (2 waves of 96 x 128), 128 x 256 (8 waves of 32 x 128)
// and 128 x 128 (4 waves of 32 x 128): the tile grid is chosen per
// problem by counting rounds of 256 workgroups, and every configuration
// issues the same MFMA sequence per output element.
constexpr int f16_lds_bytes(int bm, int bn) { return 2 * bm * 128 + 2 * bn * 128; }

// Tile (column bx, row by, K split bz) of workgroup i < ntiles = ntx nty ntz.
// gw == 0: (i % ntx, i / ntx % nty, i / (ntx nty)), the order a 3-D grid
// dispatches. gw > 0: workgroups go to the 8 XCDs round robin (i on XCD
// i % 8), each with its own L2, so XCD x takes a contiguous run of tiles,
// [x q + min(x, r), + q + (x < r)) for ntiles = 8 q + r, in an order that
// keeps a run compact: K split outermost, then groups of gw column tiles
// taken row by row. The XCDs then share fewer operand panels.
__host__ __device__ inline void f16_tile_coords(int i, int ntx, int nty, int ntiles, int gw, int& bx, int& by,
                                                int& bz) {
  if (gw > 0) {
    const int q = ntiles >> 3, r = ntiles & 7, x = i & 7;
    i = x * q + (x < r ? x : r) + (i >> 3);
  }
  const int per = ntx * nty;
  bz = i / per;
  const int t = i - bz * per;
  if (gw > 0) {
    const int g = t / (gw * nty), c0 = g * gw, w = ntx - c0 < gw ? ntx - c0 : gw, u = t - g * gw * nty;
    by = u / w;
    bx = c0 + u % w;
  } else {
    bx = t % ntx;
    by = t / ntx;
  }
}

// The grid is one-dimensional: workgroup i < ntiles computes the tile that
// f16_tile_coords gives it; the workgroups past the tiles do `side`, another
// matrix's expansion, on the CUs the tiles leave idle (dispatched after the
// tiles, so they never delay one).
//
// K16: 16 x 16 x 32 MFMAs (each wave's MI 32-row blocks as 2 MI 16-row
// blocks, 8 column blocks of 16) instead of 32 x 32 x 16. Every output sums
// the same f16 products in the same k order, and the two forms give
// bit-identical results (the fused kernels use 32 x 32 x 16). In the 16 x
// 150 encoder pass the 16 x 16 form runs the 4- and 8-wave tiles whose waves
// hold 64 or 96 rows 4-9 % faster (gate/up 256 x 256 137.0 -> 124.5 us, 384 x
// 256 103.4 -> 99.2, down 256 x 256 61.6 -> 57.5); with 32-row waves
// (128 x 256) and on the 2-wave 192 x 128 tile it gains nothing or loses up
// to 1.3 %, and they keep 32 x 32.
template <int EPI, int BN, int WM, int MI, bool K16>
__global__ __launch_bounds__(WM * BN / 128 * 64) void gemm_f16_kernel(const uint16_t* __restrict__ x, int ldx,
                                                                     const uint16_t* __restrict__ wt, int N, int K,
                                                                     int M, int kchunk, void* __restrict__ out,
                                                                     int ldo, int ntx, int nty, int ntiles, int gw,
                                                                     SideExpand side) {
  constexpr int WAVES = WM * BN / 128, BM = 32 * MI * WM;
  const int tile = blockIdx.x;
  if (tile >= ntiles) {
    constexpr int kPer = WAVES * 64 / 8;  // blocks per workgroup and round, 8 threads each
    const int nside = gridDim.x - ntiles;
    for (int64_t b = (int64_t)(tile - ntiles) * kPer + (threadIdx.x >> 3); b < side.nblocks; b += (int64_t)nside * kPer)
      side_expand_part(side, b, (int)(threadIdx.x & 7));
    return;
  }
  int bx, by, bz;
  f16_tile_coords(tile, ntx, nty, ntiles, gw, bx, by, bz);
  constexpr int XI = BM / 8 / WAVES, WI = BN / 8 / WAVES;  // copy instructions per wave and stage
  static_assert(XI * 8 * WAVES == BM && WI * 8 * WAVES == BN, "copies must cover the tiles");
  constexpr int XSTAGE = BM * 128, WSTAGE = BN * 128;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* sX = smem;               // [2][BM rows][128 B]
  uint8_t* sW = smem + 2 * XSTAGE;  // [2][BN rows][128 B]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int m0 = by * BM, n0 = bx * BN;
  const int kbeg = bz * kchunk;
  const int nsteps = kchunk / kBK;

  // Each copy instruction moves 8 whole rows: lane l -> row R + l/8, slot
  // l%8 holding logical chunk (l%8) ^ f(row). Wave w copies X rows
  // [8 XI w, +8 XI) and W rows [8 WI w, +8 WI). Addresses are the tile's
  // first row (uniform) plus 32-bit element offsets (at most BM ldx and
  // BN K), half the registers of per-lane pointers.
  const uint16_t* xtile = x + (size_t)m0 * ldx;
  const uint16_t* wtile = wt + (size_t)n0 * K;
  int xoff[XI], woff[WI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int r = 8 * XI * wave + 8 * i + (lane >> 3);
    xoff[i] = (min(m0 + r, M - 1) - m0) * ldx + 8 * ((lane & 7) ^ xswz(r));
  }
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int r = 8 * WI * wave + 8 * i + (lane >> 3);
    woff[i] = (min(n0 + r, N - 1) - n0) * K + 8 * ((lane & 7) ^ xswz(r));
  }
  auto copy = [&](int stage, int k0) {
    const uint16_t* xk = xtile + k0;
    const uint16_t* wk = wtile + k0;
#pragma unroll
    for (int i = 0; i < XI; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(xk + xoff[i]),
                                       (lds_void*)(sX + stage * XSTAGE + (8 * XI * wave + 8 * i) * 128), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < WI; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(wk + woff[i]),
                                       (lds_void*)(sW + stage * WSTAGE + (8 * WI * wave + 8 * i) * 128), 16, 0, 0);
  };

  // Accumulators: MI x 4 blocks of 32 x 32, or 2 MI x 8 blocks of 16 x 16.
  constexpr int AI = K16 ? 2 * MI : MI, AJ = K16 ? 8 : 4;
  using Acc = std::conditional_t<K16, float4v, float16v>;
  Acc acc[AI][AJ];
#pragma unroll
  for (int i = 0; i < AI; ++i)
#pragma unroll
    for (int j = 0; j < AJ; ++j) acc[i][j] = Acc{};

  auto mfma_step = [&](int stage) {
    const uint8_t* xs = sX + stage * XSTAGE;
    const uint8_t* ws = sW + stage * WSTAGE;
    if constexpr (K16) {
      // Two k steps of 32: lane l holds k 8(l/16) .. +7 of row or column l%16.
      // Beside the 192 accumulator registers of the 384 x 256 tile's waves
      // the B fragments go 2 at a time, each group's reads and MFMAs kept
      // together (without the scheduling barrier, or with all 8 B fragments
      // live, the compiler spills; reading A in two halves instead fits too
      // but reads B twice, 6.5 % slower).
      constexpr int JG = (WM == 4 && MI == 3) ? 2 : 4;  // B fragments at a time
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        // Rows 16 i + l%16 share the swizzle of row l%16: one lane offset per
        // operand and k step, the blocks at constant offsets of 2 KB.
        const int c = 4 * ks + (lane >> 4), sw = 16 * (c ^ xswz(lane & 15));
        const uint8_t* xa = xs + (wm * 32 * MI + (lane & 15)) * 128 + sw;
        const uint8_t* wb = ws + (wn * 128 + (lane & 15)) * 128 + sw;
        half8v af[AI];
#pragma unroll
        for (int i = 0; i < AI; ++i) af[i] = *(const half8v*)(xa + i * 2048);
#pragma unroll
        for (int jg = 0; jg < 8 / JG; ++jg) {
          half8v bf[JG];
#pragma unroll
          for (int j = 0; j < JG; ++j) bf[j] = *(const half8v*)(wb + (JG * jg + j) * 2048);
#pragma unroll
          for (int i = 0; i < AI; ++i)
#pragma unroll
            for (int j = 0; j < JG; ++j)
              acc[i][JG * jg + j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][JG * jg + j], 0, 0, 0);
          if constexpr (JG == 2) __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else {
      // Four k steps of 16: lane l holds k 8(l/32) .. +7 of row or column l%32
      // (row blocks at constant offsets of 4 KB from one lane offset).
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int c = 2 * ks + (lane >> 5), sw = 16 * (c ^ xswz(lane & 31));
        const uint8_t* xa = xs + (wm * 32 * MI + (lane & 31)) * 128 + sw;
        const uint8_t* wb = ws + (wn * 128 + (lane & 31)) * 128 + sw;
        half8v af[MI], bf[4];
#pragma unroll
        for (int i = 0; i < MI; ++i) af[i] = *(const half8v*)(xa + i * 4096);
#pragma unroll
        for (int j = 0; j < 4; ++j) bf[j] = *(const half8v*)(wb + j * 4096);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
      }
    }
  };

  // The copies of step s+2 are issued right after the barrier that frees
  // their stage and have the whole of step s+1 to land. Loads complete in
  // order: vmcnt(XI + WI) leaves the newer stage's copies in flight.
  auto kat = [&](int s) { return kbeg + min(s, nsteps - 1) * kBK; };
  copy(0, kat(0));
  copy(1, kat(1));
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(XI + WI));
  __syncthreads();
  for (int s = 0; s < nsteps; s += 2) {
    mfma_step(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    copy(0, kat(s + 2));
    mfma_step(1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    copy(1, kat(s + 3));
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (K16)
    gemm_epilogue16<EPI, AI>(acc, m0 + wm * 32 * MI, n0 + wn * 128, lane, M, N, out, ldo, bz);
  else
    gemm_epilogue<EPI, MI>(acc, m0 + wm * 32 * MI, n0 + wn * 128, lane, M, N, out, ldo, bz);
}

int gemm_splits(const QWeight& w, int m) {
  // Narrow projections (N = hidden) give too few column tiles to fill 256
  // CUs: split K into chunks of at least 1024 columns, at most 4 ways, or 2
  // from kLargeM tokens on, where the f16 tiles fill the CUs with half the
  // fp32 partials (Q6_K 2048 x 8192 at 2400 tokens: 107 us with its
  // expansion on 2 splits against 122 on 4, and the RMSNorm that sums the
  // partials 11.6 us against 17.0; at 1536 tokens 2 splits lose: 78.5 us
  // against 71.0).
  const int ntiles = (w.n + 127) / 128;
  const int kblocks = w.k / 256;
  if (ntiles >= 24) return 1;
  const int cap = m >= kLargeM ? 2 : 4;
  int s = 1;
  while (s < cap && kblocks % (2 * s) == 0 && w.k / (2 * s) >= 1024) s *= 2;
  return s;
}

int mid_splits(const QWeight& w) {
  // K chunks of at least 512 columns, enough of them that a single 64-row
  // tile of the matrix gives 512 workgroups, and a divisor of the block count.
  const int kblocks = w.k / 256, ntiles = (w.n + 127) / 128;
  const int cap = std::max(1, std::min(w.k / 512, (512 + ntiles - 1) / ntiles));
  int s = 1;
  for (int c = 1; c <= cap; ++c)
    if (kblocks % c == 0) s = c;
  return s;
}

enum GemmVariant { kVarBig = 0, kVarLds128 = 1, kVarLds256 = 2, kVarMid = 3 };

template <int TYPE, int EPI>
// Returns whether the launch carried `side` (only the 64-row tiles do).
static bool launch_typed(int var, int m, int splits, const uint16_t* x, int ldx, const QWeight& w, int kchunk,
                         void* out, int ldo, hipStream_t s, const SideExpand* side) {
  if (var == kVarBig) {
    static bool configured = false;  // one attribute call per instantiation
    if (!configured) {
      (void)hipFuncSetAttribute((const void*)gemm_big_kernel<TYPE, EPI>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                kBigLds);
      configured = true;
    }
    dim3 grid((w.n + kBigBN - 1) / kBigBN, (m + kBigBM - 1) / kBigBM, splits);
    gemm_big_kernel<TYPE, EPI><<<grid, 512, kBigLds, s>>>(x, ldx, w, m, kchunk, out, ldo);
  } else if (var == kVarMid && (kchunk / kBK) % kMidDepth == 0) {
    const int ntx = (w.n + 127) / 128, nty = (m + kMidBM - 1) / kMidBM, ntiles = ntx * nty * splits;
    SideExpand e;
    int nside = 0;
    if (side && side->count && side->nblocks > 0) {
      e = *side;
      nside = (int)std::min<int64_t>(1024, (e.nblocks + 31) / 32);  // 32 blocks per workgroup and round
    }
    gemm_mid_kernel<TYPE, EPI><<<ntiles + nside, 256, 0, s>>>(x, ldx, w, m, kchunk, out, ldo, ntx, nty, ntiles, e);
    return nside > 0;
  } else if (var == kVarLds256) {
    dim3 grid((w.n + 127) / 128, (m + 255) / 256, splits);
    gemm_kernel<TYPE, 256, EPI><<<grid, 256, 0, s>>>(x, ldx, w, m, kchunk, out, ldo);
  } else {
    dim3 grid((w.n + 127) / 128, (m + 127) / 128, splits);
    gemm_kernel<TYPE, 128, EPI><<<grid, 256, 0, s>>>(x, ldx, w, m, kchunk, out, ldo);
  }
  return false;
}

// Fused-kernel choice, from measurements of the encoder's shapes: the 256 x
// 256 Q4_K kernel once it alone gives every CU a workgroup; Q6_K decodes more
// VALU work per weight and does best on the 4-wave LDS-staged tiles.
static int gemm_variant(const QWeight& w, int m, int splits) {
  const int ntiles = (w.n + 127) / 128;
  if ((w.type == kQ4_K || w.type == kQ4_0) && w.n % kBigBN == 0 &&
      ((m + kBigBM - 1) / kBigBM) * (w.n / kBigBN) * splits >= 256)
    return kVarBig;
  if (w.type == kQ6_K && m >= 512) return kVarLds256;
  return (m >= 512 && ((m + 255) / 256) * ntiles * splits >= 512) ? kVarLds256 : kVarLds128;
}

// The 64-row deep-prefetch tiles while they give at most two workgroups per
// CU: there a step's latency, not the machine's throughput, bounds the other
// kernels (measured on the encoder's shapes, 17 <= m <= 1024).
static bool use_mid(const QWeight& w, int m, int splits) {
  // Up to 512 workgroups, 256 for Q6_K, whose fused decode costs more (its
  // 2048 x 8192 matrix in 4 splits at 320 tokens: 41.0 us on 320 workgroups
  // of 64-row tiles against 33.7 expanded onto 128 x 128 tiles; at 192
  // tokens 26.6 against 33.1).
  const int steps = w.k / splits / kBK;
  const int wg = ((m + kMidBM - 1) / kMidBM) * ((w.n + 127) / 128) * splits;
  return steps % kMidDepth == 0 && wg <= (w.type == kQ6_K ? 256 : 512);
}

// f16 GEMM tile configurations of the two-pass path.
// kF16T256Tail: 256 x 256 tiles over the rows that fill whole rounds of 256
// workgroups, then 128 x 256 tiles over the rest in a second launch.
// kF16T384x256: 8 waves of 96 x 128, the whole 160 KB of LDS (two stages of
// 384 + 256 rows of 128 bytes). kF16T192x128: 2 waves of 96 x 128 in 80 KB,
// two workgroups per CU.
enum F16Tile {
  kF16None = 0,
  kF16T256x256,
  kF16T256x128,
  kF16T192x256,
  kF16T128x256,
  kF16T256Tail,
  kF16T128x128,
  kF16T384x256,
  kF16T192x128
};
static int f16_bm(int t) {
  return t == kF16T384x256                           ? 384
         : (t == kF16T192x256 || t == kF16T192x128) ? 192
         : (t == kF16T128x256 || t == kF16T128x128) ? 128
                                                    : 256;
}
static int f16_bn(int t) { return (t == kF16T256x128 || t == kF16T128x128 || t == kF16T192x128) ? 128 : 256; }

// Rounds of 192 x 128 tiles: two workgroups fit on a CU, so a round is 512.
static int rounds_192x128(const QWeight& w, int m, int splits) {
  return (((m + 191) / 192) * (w.n / 128) * splits + 511) / 512;
}

// Rows of a kF16T256Tail launch's 256 x 256 part (n % 256 == 0).
static int tail_main_rows(int m, int n) {
  const int ntn = n / 256, rounds = ((m + 255) / 256) * ntn / 256;
  return std::min(m, 256 * (rounds * 256 / ntn));
}

// Tile of the two-pass GEMM for this problem, or kF16None when the fused
// kernels are the better choice (measured on the encoder's shapes): 256 x 256
// tiles once they alone give every CU a workgroup (Q6_K, whose fused decode
// costs more VALU work per weight: from 192 workgroups, the down projection
// after the merge); 256 x 128 tiles for unsplit problems with at least 64 of
// them (the QKV projection). Split-K problems with fewer 256-column tiles do
// better on the fused 128-row tiles, of which two or more fit on a CU.
static int two_pass_tile(const QWeight& w, int m, int splits, bool with_side = false) {
  const int mt = (m + kBigBM - 1) / kBigBM;
  // A launch that carries side work (another matrix's expansion) and whose
  // 256 x 256 tiles fill 3/4 to all of a round: those tiles, so the idle CUs
  // run the side work beside them from the start. Measured on the encoder's
  // down projection after the merge (Q6_K 2048 x 8192, K split 4 ways, 1536
  // tokens, the next layer's QKV and O expansion as side work): 192 tiles of
  // 256 x 256 took the 16 x 150 pass 4.71 -> 4.60 ms against 512 tiles of
  // 192 x 128 (two per CU, which start the side work only as they finish),
  // although alone the 192 x 128 tiles are faster (61.2 against 67.7 us).
  // The same launch on 160 tiles at 2400 tokens (K split 2) was not faster.
  if (with_side && w.n % 256 == 0 && splits > 1) {
    const int t256 = mt * (w.n / 256) * splits;
    if (4 * t256 >= 3 * 256 && t256 <= 256) return kF16T256x256;
  }
  if (w.n % 256 == 0 && mt * (w.n / 256) * splits >= (w.type == kQ6_K ? 192 : 256)) {
    // 192-row tiles (4 waves; measured at ~0.83 of the 256-row tiles' rate
    // per flop) when their rounds of 256 workgroups cost less: 1536 tokens
    // give 384 tiles of 256 rows (two rounds, the second half empty) but 512
    // of 192 rows (two full rounds of tiles 3/4 the size). Time per round is
    // taken as tile area / rate: 0.75 / 0.83 = 0.904 of a 256-row round.
    // The same count holds per K split (the down projection's 4 splits at
    // 1536 tokens: 192 workgroups of 256 rows, 256 of 192).
    const int t256 = mt * (w.n / 256) * splits, t192 = ((m + 191) / 192) * (w.n / 256) * splits;
    int best = kF16T256x256, cost = 1000 * ((t256 + 255) / 256);
    if (904 * ((t192 + 255) / 256) < cost) best = kF16T192x256, cost = 904 * ((t192 + 255) / 256);
    // 384-row tiles (a round measured at 1.525 times a 256-row round: 1.5 times
    // the work, less LDS traffic per MFMA) when they need fewer rounds: 1536
    // tokens of the gate/up projection fill exactly one round of them
    // (104.6 us for the f16 GEMM against 127.5 on the tiling below).
    const int t384 = ((m + 383) / 384) * (w.n / 256) * splits;
    if (1525 * ((t384 + 255) / 256) < cost) best = kF16T384x256, cost = 1525 * ((t384 + 255) / 256);
    // 192 x 128 tiles on 2 waves, two workgroups per CU: a round of 512
    // charged 850 (f16 GEMM alone, random operands: the down projection's K
    // split 4 ways at 1536 tokens 61.2 us against 61.7 on 192 x 256 tiles and
    // 67.7 on 256 x 256).
    if (850 * rounds_192x128(w, m, splits) < cost) best = kF16T192x128, cost = 850 * rounds_192x128(w, m, splits);
    // Whole rounds of 256-row tiles, then the rows left on 128-row tiles in
    // a second launch, a round of those charged 0.65 of a 256-row round.
    // With that charge the encoder's shapes pick the faster tiling (gate/up,
    // expansion included: 1536 tokens 131.0 us against 134.5 on 192-row
    // tiles; 2400 tokens 190.7 us against 203.4 on 256-row tiles).
    const int main = splits == 1 ? tail_main_rows(m, w.n) : 0;
    if (main > 0 && main < m) {
      const int wg_main = (main / 256) * (w.n / 256), wg_rest = ((m - main + 127) / 128) * (w.n / 256);
      if (1000 * ((wg_main + 255) / 256) + 650 * ((wg_rest + 255) / 256) < cost) best = kF16T256Tail;
    }
    return best;
  }
  if (w.n % 256 == 0 && (splits > 1 || mt * (w.n / 128) >= 64)) {
    // Too few column tiles (or K split) for a round of 256-row tiles: the
    // tiling with the fewest rounds of 256 workgroups, a round charged its
    // tiles' relative time (256 rows 1000, 192 rows 904, 128 rows 650,
    // 128 x 128 380). Measured (expansion included): Q6_K 2048 x 8192 in 2
    // splits at 2400 tokens 101.8 us on 192 x 256 (256 x 256 105.8) against
    // 140.8 fused; Q4_K 2048 x 2048 in 2 splits at 1536 tokens 27.7 on
    // 128 x 256 against 30.2 fused, at 2400 tokens 38.4 on 192 x 256
    // against 39.7; Q6_K 2048 x 8192 in 4 splits at 500 tokens 35.7 on
    // 128 x 128, 41.5 on 128 x 256; Q4_0 12288 x 2048 at 800 tokens 68.4 on
    // 192 x 256 (128 x 256 81.0), at 1024 tokens 72.3 on 256 x 256; the QKV
    // projection's f16 GEMM at 1536 tokens 34.9 on 128 x 256 against 36.4 on
    // 128 x 128.
    // 192 x 128 tiles on 2 waves (two workgroups per CU, so a round is 512)
    // charged 850 (f16 GEMM alone, random operands): the down projection's 2
    // splits at 2400 tokens 91.8 us against 101.1 on 192 x 256, the attention
    // output's 34.9 against 36.5.
    const int tiles[5] = {kF16T256x256, kF16T192x256, kF16T128x256, kF16T128x128, kF16T192x128};
    const int charge[5] = {1000, 904, 650, 380, 850};
    const int slots[5] = {256, 256, 256, 256, 512};
    int best = kF16None, cost = 0;
    for (int i = 0; i < 5; ++i) {
      const int wg = ((m + f16_bm(tiles[i]) - 1) / f16_bm(tiles[i])) * (w.n / f16_bn(tiles[i])) * splits;
      const int c = charge[i] * ((wg + slots[i] - 1) / slots[i]);
      if (best == kF16None || c < cost) best = tiles[i], cost = c;
    }
    return best;
  }
  if (splits == 1 && w.n % 128 == 0 && mt * (w.n / 128) >= 64) {
    // Columns in 128s only: 128 x 128 tiles on 4 waves when 256-row tiles
    // leave CUs without a workgroup and 128-row tiles do not, else 256 x 128.
    if (mt * (w.n / 128) < 256 && ((m + 127) / 128) * (w.n / 128) >= 256) return kF16T128x128;
    return kF16T256x128;
  }
  return kF16None;
}

// Whether the problem takes the two-pass path. Side work never decides
// that: its rule in two_pass_tile only picks among two-pass tilings of
// split problems, which take the two-pass path without it too.
bool gemm_two_pass(const QWeight& w, int m, int splits) {
  return !use_mid(w, m, splits) && two_pass_tile(w, m, splits) != kF16None;
}

bool gemm_two_pass_tail(const QWeight& w, int m, int splits) {
  return !use_mid(w, m, splits) && two_pass_tile(w, m, splits) == kF16T256Tail;
}

// Operand rows the XCDs' L2s fetch for one tile order: per XCD and round of
// concurrent workgroups (slots over the chip), the distinct X row tiles times
// bm plus the distinct W column tiles times bn, each per K split.
static int64_t f16_order_rows(int ntx, int nty, int ntz, int bm, int bn, int slots, int gw) {
  const int ntiles = ntx * nty * ntz, per_xcd = std::max(1, slots / 8);
  std::vector<int> xs((size_t)nty * ntz, -1), ws((size_t)ntx * ntz, -1);
  int64_t rows = 0;
  for (int x = 0; x < 8; ++x)
    for (int j = 0; x + 8 * j < ntiles; ++j) {
      const int grp = x * (ntiles + 1) + j / per_xcd;
      int bx, by, bz;
      f16_tile_coords(x + 8 * j, ntx, nty, ntiles, gw, bx, by, bz);
      int& sx = xs[(size_t)bz * nty + by];
      int& sw = ws[(size_t)bz * ntx + bx];
      if (sx != grp) sx = grp, rows += bm;
      if (sw != grp) sw = grp, rows += bn;
    }
  return rows;
}

// Tile order of a launch (the gw of f16_tile_coords): the one whose XCDs
// fetch the fewest operand rows, the dispatch order unless another saves at
// least 5 %. The encoder's K-split projections gain most (the down
// projection's 4 splits at 1536 tokens: every XCD reads all of X in the
// dispatch order, 235 MB per launch, against 84 MB).
static int f16_order(int ntx, int nty, int ntz, int bm, int bn, int slots) {
  static std::mutex mu;
  static std::unordered_map<uint64_t, int> memo;
  const uint64_t key = (uint64_t)ntx | (uint64_t)nty << 16 | (uint64_t)ntz << 32 | (uint64_t)bm << 40 |
                       (uint64_t)(bn / 128) << 50 | (uint64_t)(slots / 256) << 54;
  std::lock_guard<std::mutex> lock(mu);
  const auto it = memo.find(key);
  if (it != memo.end()) return it->second;
  // Group widths tried: 1..16, the larger powers of two and ntx (the cost
  // of one is linear in the tiles; very large grids keep the dispatch order).
  const int64_t ntiles = (int64_t)ntx * nty * ntz;
  int best = 0;
  if (ntiles >= 16 && ntiles <= 65536) {
    const int64_t base = f16_order_rows(ntx, nty, ntz, bm, bn, slots, 0);
    int64_t cost = base;
    for (int g = 1; g <= ntx; g = g < 16 ? g + 1 : (g * 2 > ntx && g != ntx ? ntx : g * 2)) {
      const int64_t c = f16_order_rows(ntx, nty, ntz, bm, bn, slots, g);
      if (c < cost) best = g, cost = c;
    }
    if (best && cost * 20 > base * 19) best = 0;
  }
  memo.emplace(key, best);
  return best;
}

template <int BN, int WM, int MI>
static void launch_f16(int epilogue, dim3 grid, const uint16_t* x, int ldx, const uint16_t* wexp, const QWeight& w,
                       int m, int kchunk, void* out, int ldo, hipStream_t stream, const SideExpand* side = nullptr) {
  constexpr int lds = f16_lds_bytes(32 * MI * WM, BN), threads = WM * BN / 128 * 64;
  const int ntiles = (int)(grid.x * grid.y * grid.z);
  // two workgroups per CU for the 2-wave tiles
  const int gw = f16_order((int)grid.x, (int)grid.y, (int)grid.z, 32 * MI * WM, BN, threads == 128 ? 512 : 256);
  SideExpand e;
  int nside = 0;
  if (side && side->count && side->nblocks > 0) {
    // Enough workgroups to cover the expansion in a few rounds (more than the
    // CUs the tiles leave idle: the rest start as tiles finish).
    e = *side;
    nside = (int)std::min<int64_t>(1024, (e.nblocks + threads / 8 - 1) / (threads / 8));
  }
  auto launch = [&](auto kernel) {
    static bool configured = false;  // one attribute call per instantiation
    if (!configured) {
      (void)hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      configured = true;
    }
    kernel<<<ntiles + nside, threads, lds, stream>>>(x, ldx, wexp, w.n, w.k, m, kchunk, out, ldo, (int)grid.x,
                                                      (int)grid.y, ntiles, gw, e);
  };
  constexpr bool k16 = WM == 4 && MI >= 2;  // 16 x 16 x 32 MFMAs on the 4- and 8-wave tiles of 64+ rows a wave
  if (epilogue == kEpiStore) launch(gemm_f16_kernel<kEpiStore, BN, WM, MI, k16>);
  else if (epilogue == kEpiPartial) launch(gemm_f16_kernel<kEpiPartial, BN, WM, MI, k16>);
  else if (epilogue == kEpiPartial16) launch(gemm_f16_kernel<kEpiPartial16, BN, WM, MI, k16>);
  else launch(gemm_f16_kernel<kEpiSwiGLU, BN, WM, MI, k16>);
}

static hipError_t launch_two_pass(const uint16_t* x, int ldx, const QWeight& w, int m, int epilogue, int splits,
                                  void* out, int ldo, uint16_t* wexp, hipStream_t stream, int tile,
                                  bool expanded = false, const SideExpand* side = nullptr) {
  const int bm = f16_bm(tile), bn = f16_bn(tile);
  if (epilogue == kEpiSwiGLU && w.n % bn) return hipErrorInvalidValue;
  // gemm_f16_kernel addresses a tile's rows by 32-bit element offsets
  if ((int64_t)bm * ldx > INT32_MAX || (int64_t)bn * w.k > INT32_MAX) return hipErrorInvalidValue;
  const int64_t threads = (int64_t)w.n * (w.k / 32);
  const unsigned blocks = (unsigned)((threads + 255) / 256);
  if (expanded) {
    // wexp already holds the expansion
  } else if (w.type == kQ4_K) {
    // GGUF Q4_K rows are whole blocks: the row-major f16 matrix is the
    // blocks' decode in order (full-line stores, same values).
    const hipError_t e = launch_expand_q4k(w.blocks, (int64_t)w.n * (w.k / 256), wexp, stream);
    if (e != hipSuccess) return e;
  } else if (w.type == kQ6_K) {
    const hipError_t e = launch_expand_q6k(w, wexp, stream);
    if (e != hipSuccess) return e;
  } else {
    expand_kernel<kQ4_0><<<blocks, 256, 0, stream>>>(w, wexp);
  }
  const int kchunk = w.k / splits;
  dim3 grid((w.n + bn - 1) / bn, (m + bm - 1) / bm, splits);
  switch (tile) {
    case kF16T256Tail: {
      if (splits != 1) return hipErrorInvalidValue;
      const int main = tail_main_rows(m, w.n), rest = m - main;
      // side work on the second launch, whose tiles leave CUs idle
      launch_f16<256, 4, 2>(epilogue, dim3(w.n / 256, main / 256, 1), x, ldx, wexp, w, main, kchunk, out, ldo, stream);
      const size_t skip = (size_t)main * ldo * (epilogue == kEpiPartial ? 4 : 2);  // bytes of the rows done
      launch_f16<256, 4, 1>(epilogue, dim3(w.n / 256, (rest + 127) / 128, 1), x + (size_t)main * ldx, ldx, wexp, w,
                            rest, kchunk, (uint8_t*)out + skip, ldo, stream, side);
      break;
    }
    case kF16T256x256: launch_f16<256, 4, 2>(epilogue, grid, x, ldx, wexp, w, m, kchunk, out, ldo, stream, side); break;
    case kF16T256x128: launch_f16<128, 4, 2>(epilogue, grid, x, ldx, wexp, w, m, kchunk, out, ldo, stream, side); break;
    case kF16T192x256: launch_f16<256, 2, 3>(epilogue, grid, x, ldx, wexp, w, m, kchunk, out, ldo, stream, side); break;
    case kF16T128x256: launch_f16<256, 4, 1>(epilogue, grid, x, ldx, wexp, w, m, kchunk, out, ldo, stream, side); break;
    case kF16T128x128: launch_f16<128, 4, 1>(epilogue, grid, x, ldx, wexp, w, m, kchunk, out, ldo, stream, side); break;
    case kF16T384x256: launch_f16<256, 4, 3>(epilogue, grid, x, ldx, wexp, w, m, kchunk, out, ldo, stream, side); break;
    case kF16T192x128: launch_f16<128, 2, 3>(epilogue, grid, x, ldx, wexp, w, m, kchunk, out, ldo, stream, side); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

static hipError_t launch_fused(const uint16_t* x, int ldx, const QWeight& w, int m, int epilogue, int splits,
                               void* out, int ldo, hipStream_t stream, uint16_t* wexp, int forced,
                               bool expanded = false, const SideExpand* side = nullptr) {
  if (m <= 0) return side ? launch_side_expand(*side, stream) : hipSuccess;
  if (splits < 1 || (w.k / 256) % splits) return hipErrorInvalidValue;
  if (epilogue != kEpiPartial && epilogue != kEpiPartial16 && splits != 1) return hipErrorInvalidValue;
  if (epilogue == kEpiSwiGLU && w.n % 128) return hipErrorInvalidValue;
  if (w.type != kQ4_K && w.type != kQ6_K && w.type != kQ4_0) return hipErrorInvalidValue;
  const int kchunk = w.k / splits;
  if (forced < 0 && use_mid(w, m, splits)) forced = kVarMid;
  const int tile = (wexp && forced < 0) ? two_pass_tile(w, m, splits, side && side->count && side->nblocks > 0)
                                         : kF16None;
  if (tile != kF16None)
    return launch_two_pass(x, ldx, w, m, epilogue, splits, out, ldo, wexp, stream, tile, expanded, side);
  const int var = forced >= 0 ? forced : gemm_variant(w, m, splits);
  bool carried = false;
#define NEMO_LAUNCH(T)                                                                                               \
  if (epilogue == kEpiStore)                                                                                         \
    carried = launch_typed<T, kEpiStore>(var, m, splits, x, ldx, w, kchunk, out, ldo, stream, side);                \
  else if (epilogue == kEpiPartial)                                                                                  \
    carried = launch_typed<T, kEpiPartial>(var, m, splits, x, ldx, w, kchunk, out, ldo, stream, side);              \
  else if (epilogue == kEpiPartial16)                                                                                \
    carried = launch_typed<T, kEpiPartial16>(var, m, splits, x, ldx, w, kchunk, out, ldo, stream, side);            \
  else                                                                                                               \
    carried = launch_typed<T, kEpiSwiGLU>(var, m, splits, x, ldx, w, kchunk, out, ldo, stream, side);
  if (w.type == kQ4_K) {
    NEMO_LAUNCH(kQ4_K)
  } else if (w.type == kQ6_K) {
    NEMO_LAUNCH(kQ6_K)
  } else {
    NEMO_LAUNCH(kQ4_0)
  }
#undef NEMO_LAUNCH
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || !side || carried) return e;
  return launch_side_expand(*side, stream);  // the other fused kernels carry no side work
}

hipError_t launch_gemm_ex(const uint16_t* x, int ldx, const QWeight& w, int m, int epilogue, int splits, void* out,
                          int ldo, hipStream_t stream, uint16_t* wexp, bool expanded, const SideExpand* side) {
  return launch_fused(x, ldx, w, m, epilogue, splits, out, ldo, stream, wexp, -1, expanded, side);
}

hipError_t launch_gemm_mid(const uint16_t* x, int ldx, const QWeight& w, int m, int epilogue, int splits, void* out,
                           int ldo, hipStream_t stream) {
  return launch_fused(x, ldx, w, m, epilogue, splits, out, ldo, stream, nullptr, kVarMid);
}

hipError_t launch_gemm(const uint16_t* x, int ldx, const QWeight& w, uint16_t* y, int ldy, int m, hipStream_t stream) {
  return launch_gemm_ex(x, ldx, w, m, kEpiStore, 1, y, ldy, stream);
}

hipError_t launch_gemm_two_pass(const uint16_t* x, int ldx, const QWeight& w, int m, uint16_t* y, int ldy,
                                uint16_t* wexp, hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  if (w.type != kQ4_K && w.type != kQ6_K && w.type != kQ4_0) return hipErrorInvalidValue;
  int tile = two_pass_tile(w, m, 1);  // the plan's tile for this size, else the widest that fits
  if (tile == kF16None) tile = w.n % 256 == 0 ? kF16T256x256 : kF16T256x128;
  return launch_two_pass(x, ldx, w, m, kEpiStore, 1, y, ldy, wexp, stream, tile);
}

}  // namespace nemo
