// Quantized-weight kernels of libnemo: GGML block decoding, the MFMA GEMM and
// the small-M GEMV. Host-side launch helpers; kernels live in nemo_quant.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nemo {

// GGML tensor type codes (src/gguf/types.ts:17-23).
enum GgmlType : int { kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ4_K = 12, kQ6_K = 14 };

// A quantized weight matrix of n rows by k columns (GGUF dims [k, n]) as it
// sits in device memory.
//  Q4_K: `blocks` holds the GGUF bytes unchanged, 144-byte super-blocks, row
//        major ((k / 256) blocks per row). Every block is 16-byte aligned.
//  Q6_K: GGUF's 210-byte blocks are split at upload so that loads stay
//        16-byte aligned: `blocks` holds 208-byte records (ql[128] qh[64]
//        scales[16]) and `d` the per-block f16 scale, both row major.
//  Q4_0: likewise split (from GGUF's 18-byte blocks or the wgpack
//        tile32-compact records): `blocks` holds the 16 nibble bytes of each
//        32-value block, `d` its f16 scale, both row major.
struct QWeight {
  int type;
  int n;
  int k;
  const uint8_t* blocks;
  const uint16_t* d;
  // Optional: the same blocks regrouped for the GEMV (launch_tile_gemv);
  // null when absent.
  const uint8_t* gv = nullptr;
};

// Bytes per row of `blocks`.
__host__ __device__ inline size_t qweight_row_bytes(int type, int k) {
  return type == kQ4_K ? (size_t)(k / 256) * 144 : type == kQ6_K ? (size_t)(k / 256) * 208 : (size_t)(k / 32) * 16;
}

// GEMM epilogues.
enum GemmEpilogue : int {
  kEpiStore = 0,    // out f16 [m, ldo]: f16(sum)
  kEpiPartial = 1,  // out float [splits][m][ldo]: the fp32 sum of each K split
  kEpiSwiGLU = 2,   // out f16 [m, ldo]: silu(g) * u over rows interleaved per 128-row tile
  kEpiPartial16 = 3,  // out f16 [splits][m][ldo]: each K split's fp32 sum rounded to f16
                      // (half kEpiPartial's bytes; the encoder's residual projections)
};

// Y[m, n] = f16( sum_k X[m, k] * W[n, k] ), fp32 accumulate. X is f16 with
// row stride ldx, Y f16 with row stride ldy (MFMA GEMM, no K split).
hipError_t launch_gemm(const uint16_t* x, int ldx, const QWeight& w, uint16_t* y, int ldy, int m,
                       hipStream_t stream);

// launch_gemm through the two-pass path: W expanded into `wexp` (n * k
// halves), then the f16 MFMA GEMM. Bit-identical to launch_gemm.
hipError_t launch_gemm_two_pass(const uint16_t* x, int ldx, const QWeight& w, int m, uint16_t* y, int ldy,
                                uint16_t* wexp, hipStream_t stream);

// The K-split count the encoder uses for `w` in a pass of m > kGemvMaxM
// tokens: a function of the weight's shape and of whether m reaches
// kLargeM (narrow projections split at most 2 ways from there on).
constexpr int kLargeM = 2048;
int gemm_splits(const QWeight& w, int m);

// Whether launch_gemm_ex, given scratch, expands `w` to f16 before an f16 x
// f16 MFMA GEMM (large batches) rather than decoding inside the GEMM.
bool gemm_two_pass(const QWeight& w, int m, int splits);
// Whether that two-pass GEMM ends with a launch of 128-row tiles for the rows
// left after whole rounds of 256-row tiles, which leaves CUs idle (side work
// given to such a GEMM goes to that launch).
bool gemm_two_pass_tail(const QWeight& w, int m, int splits);

// Blocks [first, first + nblocks) of a matrix's Q4_K or Q6_K -> f16
// expansion (row-major, the values launch_expand_q4k / launch_expand_q6k
// write). type 0: none.
struct SidePart {
  int type = 0;
  const uint8_t* blocks = nullptr;  // the range's Q4_K blocks or Q6_K 208-byte records
  const uint16_t* d = nullptr;      // Q6_K per-block scales of the range
  int64_t nblocks = 0;              // 256-value blocks
  uint16_t* out = nullptr;          // nblocks * 256 halves
};
// Up to kMaxParts such ranges carried by a GEMM launch: the f16 GEMM's
// workgroups past its tiles do them on the CUs the tiles leave idle, the
// parts' blocks numbered one after another.
struct SideExpand {
  static constexpr int kMaxParts = 2;
  int count = 0;
  int64_t nblocks = 0;  // over all parts
  SidePart part[kMaxParts];
  // Appends p (nothing for an empty part); false when the parts are full.
  bool add(const SidePart& p) {
    if (!p.type || p.nblocks <= 0) return true;
    if (count == kMaxParts) return false;
    part[count++] = p;
    nblocks += p.nblocks;
    return true;
  }
};
// The expansion of `w` into `out`, or none (type 0) for a type it does not
// cover (Q4_0, or a Q6_K matrix kept raw); with `out` null, only whether it
// covers `w`.
SidePart side_part_of(const QWeight& w, uint16_t* out);
// Blocks [first, first + count) of p.
SidePart side_part_range(const SidePart& p, int64_t first, int64_t count);
// The expansions alone, for a GEMM that cannot carry them.
hipError_t launch_side_expand(const SideExpand& e, hipStream_t stream);

// The MFMA GEMM with an epilogue; `splits` > 1 only with kEpiPartial. With
// `wexp` (room for n * k halves) large problems take the two-pass path, whose
// results are bit-identical to the fused kernels'. `expanded`: wexp already
// holds w's f16 expansion (launch_expand_q4k_pair), which the two-pass path
// then uses as it is. `side`: an expansion to do in the same launch (or, if
// this GEMM does not take the two-pass path, right after it); it must not
// write memory the GEMM reads.
hipError_t launch_gemm_ex(const uint16_t* x, int ldx, const QWeight& w, int m, int epilogue, int splits, void* out,
                          int ldo, hipStream_t stream, uint16_t* wexp = nullptr, bool expanded = false,
                          const SideExpand* side = nullptr);
// Two Q4_K matrices' blocks -> f16, row-major, in one launch (each alone
// would be latency-bound): n0 blocks of blocks0 to out0, n1 of blocks1 to out1.
hipError_t launch_expand_q4k_pair(const uint8_t* blocks0, int64_t n0, uint16_t* out0, const uint8_t* blocks1,
                                  int64_t n1, uint16_t* out1, hipStream_t stream);
// A matrix's blocks regrouped for the GEMV (n % 16 == 0): per 16-row tile
// and 256 values, the bytes each lane group of a GEMV wave loads sit
// side by side for the 16 rows, so every load of the wave reads whole
// contiguous lines (loading from the row-major blocks touches 16 lines per
// load). gemv_tile_bytes: the copy's size (0: the matrix has no tiled form).
size_t gemv_tile_bytes(const QWeight& w);
hipError_t launch_tile_gemv(const QWeight& w, uint8_t* out, hipStream_t stream);
// Q4_K blocks -> f16, row-major (the two-pass GEMM's first pass for Q4_K).
hipError_t launch_expand_q4k(const uint8_t* blocks, int64_t n_blocks, uint16_t* out16, hipStream_t stream);
// A Q6_K matrix (split layout) -> f16, row-major.
hipError_t launch_expand_q6k(const QWeight& w, uint16_t* out16, hipStream_t stream);

// K-split count of the 64-row split tiles (NEMO_MATMUL_GEMM_SPLIT): chunks
// of at least 512 columns, enough for ~512 workgroups; a function of the
// weight's shape only.
int mid_splits(const QWeight& w);

// launch_gemm_ex on the 64-row deep-prefetch tiles whatever the size
// (bit-identical to the other fused kernels).
hipError_t launch_gemm_mid(const uint16_t* x, int ldx, const QWeight& w, int m, int epilogue, int splits, void* out,
                           int ldo, hipStream_t stream);

// y[m, n] = f16(sum over s of partials[s][m][n]) in split order.
hipError_t launch_reduce_partials(const float* partials, int splits, int m, int n, uint16_t* y, int ldy,
                                  hipStream_t stream);
// SwiGLU of the gate/up projection from its split-K partials
// ([splits][m][n], rows interleaved per 128-row group): y[m, n / 2] f16.
hipError_t launch_reduce_swiglu(const float* partials, int splits, int m, int n, uint16_t* y, int ldy,
                                hipStream_t stream);

// Small-M path (m <= kGemvMaxM): MFMA GEMV, 64 rows x 2048 K per workgroup
// with an in-workgroup reduction, every decoded weight fragment applied to up
// to 10 groups of 16 tokens; K beyond 2048 splits into fp32 partials summed in
// split order through `partials` (float, at least gemv_partials_floats()).
constexpr int kGemvMaxM = 160;
size_t gemv_partials_floats(const QWeight& w, int m);
// The GEMV's K-split count: a function of the weight's shape only.
int gemv_splits(const QWeight& w);
hipError_t launch_gemv(const uint16_t* x, int ldx, const QWeight& w, uint16_t* y, int ldy, int m,
                       float* partials, hipStream_t stream);

// The GEMV with the GEMM's epilogues (m <= kGemvMaxM): kEpiStore as launch_gemv;
// kEpiPartial writes [gemv_splits(w)][m][n] fp32 sums to `out` (ldo == n);
// kEpiSwiGLU sums into `partials` (room for gemv_splits(w) * m * n floats),
// then applies SwiGLU over the 128-row interleaved gate/up columns.
hipError_t launch_gemv_ex(const uint16_t* x, int ldx, const QWeight& w, int m, int epilogue, void* out, int ldo,
                          float* partials, hipStream_t stream);

// Decode raw GGUF blocks (Q4_K 144 B, Q6_K 210 B, Q4_0 18 B) to float32 and/or
// f16 (either output may be null). n_blocks consecutive blocks.
hipError_t launch_dequant_raw(int type, const uint8_t* raw, int64_t n_blocks, float* out_f32,
                              uint16_t* out_f16, hipStream_t stream);

// Roofline probes (nemo_probe.hip): one empty launch; one read of `bytes`
// (a multiple of 16, 16-byte aligned) with `loads` (1, 2, 4 or 8) 16-byte
// loads per thread. `sink` holds 256 words and is never written in practice.
hipError_t launch_probe_empty(hipStream_t stream);
hipError_t launch_probe_stream(const void* src, int64_t bytes, int loads, uint32_t* sink, hipStream_t stream);

// requantizeMatrixToQ40 on the device: raw GGUF Q4_K / Q6_K / Q4_0 rows of a
// k x n matrix (k % 256 == 0) -> n * k / 32 GGUF Q4_0 blocks (18 bytes),
// bit-exact with the reference's JavaScript (nemo_requant.hip).
hipError_t launch_requant_q40(int src_type, const uint8_t* src, int64_t k, int64_t n, uint8_t* out,
                              hipStream_t stream);

// Decode an uploaded weight (any layout above) to float32 [n, k].
hipError_t launch_dequant_weight(const QWeight& w, float* out_f32, hipStream_t stream);

}  // namespace nemo
