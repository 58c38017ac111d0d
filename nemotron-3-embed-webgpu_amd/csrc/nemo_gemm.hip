// Fused dequant + MFMA GEMM for gfx950: Y[M, N] = X[M, K] * W[N, K]^T with
// W in Q4_K (GGUF blocks) or Q6_K (split layout), X f16, fp32 accumulate.
//
// Workgroup tile BM x 128 x 64 (BM = 256 or 128), 256 threads = 4 waves.
// Wave w owns rows [w*BM/4, (w+1)*BM/4) and all 128 columns, as a grid of
// v_mfma_f32_32x32x16_f16 blocks (BM/128 x 4). The W tile (128 rows x 64
// columns) is decoded once per workgroup into LDS and shared by the BM rows
// of X; the X tile is copied to LDS. Global loads of step k+1 are issued
// before the MFMAs of step k. LDS rows are padded to 72 halves (144 bytes) so
// the 16-byte fragment reads of 32 consecutive rows hit distinct banks.
//
// Owning all 128 columns lets the gate/up projection finish SwiGLU in
// registers: the plan stores gate_up with rows interleaved per 128-row tile
// (64 gate rows, then the matching 64 up rows), so a lane holds g and u of
// the same (token, feature) in blocks j and j+2.
//
// Split-K: blockIdx.z selects a contiguous K range; partial sums are written
// as fp32 and summed in a fixed order by the consumer (deterministic). The
// split count depends only on the weight's shape, never on M, so a token's
// result does not depend on how many other tokens share the batch.
#include "nemo_blocks.h"
#include "nemo_common.h"
#include "nemo_quant.h"

namespace nemo {

constexpr int kBN = 128, kBK = 64, kLdsK = kBK + 8;

template <int TYPE, int BM, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const uint16_t* __restrict__ x, int ldx, QWeight w, int M,
                                                   int kchunk, void* __restrict__ out, int ldo) {
  constexpr int WM = BM / 4, MI = WM / 32, XP = BM / 32;
  __shared__ __attribute__((aligned(16))) half_t sA[BM * kLdsK];
  __shared__ __attribute__((aligned(16))) half_t sB[kBN * kLdsK];
  const int N = w.n;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * kBN;
  const int kbeg = blockIdx.z * kchunk, kend = kbeg + kchunk;
  const size_t row_bytes = qweight_row_bytes(TYPE, w.k);

  // X loader: 8 threads per row (16 bytes each), 32 rows per pass.
  const int xr = tid >> 3, xc = (tid & 7) * 8;
  const uint16_t* xrow[XP];
#pragma unroll
  for (int i = 0; i < XP; ++i) xrow[i] = x + (size_t)min(m0 + i * 32 + xr, M - 1) * ldx + xc;
  // W loader: 2 threads per weight row.
  const int wr = tid >> 1, wp = tid & 1;
  const int wrow = min(n0 + wr, N - 1);

  u32x4 xa[XP];
  Q4KFetch f4;
  Q6KFetch f6;
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < XP; ++i) xa[i] = *(const u32x4*)(xrow[i] + k0);
    if constexpr (TYPE == kQ4_K) f4 = q4k_fetch(w, row_bytes, wrow, k0, wp);
    else f6 = q6k_fetch(w, row_bytes, wrow, k0, wp);
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
    if constexpr (TYPE == kQ4_K) q4k_expand(f4, lo, hi);
    else q6k_expand(f6, lo, hi);
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

  // D layout of a 32x32 block: lane l, register r -> row 8*(r/4) + 4*(l/32)
  // + r%4, column l%32.
  const int rbase = m0 + wave * WM + 4 * (lane >> 5);
  if constexpr (EPI == kEpiSwiGLU) {
    // Columns j*32 + l%32 (j = 0, 1) are gate features n0/2 + j*32 + l%32;
    // columns 64 + j*32 + l%32 are their up rows. SwiGLU as
    // src/webgpu/ops.ts:85-87 on the f16-rounded gate/up values.
    uint16_t* y = (uint16_t*)out;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int col = (n0 >> 1) + j * 32 + (lane & 31);
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
        const int col = n0 + j * 32 + (lane & 31);
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = rbase + i * 32 + 8 * (r >> 2) + (r & 3);
          if (row >= M) continue;
          if constexpr (EPI == kEpiStore)
            ((uint16_t*)out)[(size_t)row * ldo + col] = f2h(acc[i][j][r]);
          else
            ((float*)out)[((size_t)blockIdx.z * M + row) * ldo + col] = acc[i][j][r];
        }
      }
  }
}

int gemm_splits(const QWeight& w) {
  // Narrow projections (N = hidden) give too few column tiles to fill 256
  // CUs: split K into chunks of at least 1024 columns, at most 4 ways.
  const int ntiles = (w.n + kBN - 1) / kBN;
  const int kblocks = w.k / 256;
  if (ntiles >= 24) return 1;
  int s = 1;
  while (s < 4 && kblocks % (2 * s) == 0 && w.k / (2 * s) >= 1024) s *= 2;
  return s;
}

template <int TYPE, int EPI>
static void launch_typed(int bm, dim3 grid, const uint16_t* x, int ldx, const QWeight& w, int m, int kchunk, void* out,
                         int ldo, hipStream_t s) {
  if (bm == 256) gemm_kernel<TYPE, 256, EPI><<<grid, 256, 0, s>>>(x, ldx, w, m, kchunk, out, ldo);
  else gemm_kernel<TYPE, 128, EPI><<<grid, 256, 0, s>>>(x, ldx, w, m, kchunk, out, ldo);
}

hipError_t launch_gemm_ex(const uint16_t* x, int ldx, const QWeight& w, int m, int epilogue, int splits, void* out,
                          int ldo, hipStream_t stream) {
  if (m <= 0) return hipSuccess;
  if (splits < 1 || (w.k / 256) % splits) return hipErrorInvalidValue;
  if (epilogue != kEpiPartial && splits != 1) return hipErrorInvalidValue;
  if (epilogue == kEpiSwiGLU && w.n % kBN) return hipErrorInvalidValue;
  const int ntiles = (w.n + kBN - 1) / kBN;
  const int bm = (m >= 512 && ((m + 255) / 256) * ntiles * splits >= 512) ? 256 : 128;
  dim3 grid(ntiles, (m + bm - 1) / bm, splits);
  const int kchunk = w.k / splits;
#define NEMO_LAUNCH(T)                                                                           \
  if (epilogue == kEpiStore) launch_typed<T, kEpiStore>(bm, grid, x, ldx, w, m, kchunk, out, ldo, stream);   \
  else if (epilogue == kEpiPartial) launch_typed<T, kEpiPartial>(bm, grid, x, ldx, w, m, kchunk, out, ldo, stream); \
  else launch_typed<T, kEpiSwiGLU>(bm, grid, x, ldx, w, m, kchunk, out, ldo, stream);
  if (w.type == kQ4_K) {
    NEMO_LAUNCH(kQ4_K)
  } else if (w.type == kQ6_K) {
    NEMO_LAUNCH(kQ6_K)
  } else {
    return hipErrorInvalidValue;
  }
#undef NEMO_LAUNCH
  return hipGetLastError();
}

hipError_t launch_gemm(const uint16_t* x, int ldx, const QWeight& w, uint16_t* y, int ldy, int m, hipStream_t stream) {
  return launch_gemm_ex(x, ldx, w, m, kEpiStore, 1, y, ldy, stream);
}

}  // namespace nemo
