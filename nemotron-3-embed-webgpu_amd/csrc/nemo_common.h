// Shared device/host helpers of libnemo (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nemo {

typedef _Float16 half_t;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Largest number of requests one execution plan carries (ragged tables are
// passed by value as kernel arguments).
constexpr int kMaxBatch = 64;

// Prefix offsets of a ragged token layout: request b owns packed rows
// [start[b], start[b + 1]).
struct Ragged {
  int count;
  int start[kMaxBatch + 1];
};

// Per-request work-tile prefix for kernels that tile each request separately
// (attention query tiles): request b owns tiles [tile[b], tile[b + 1]).
struct RaggedTiles {
  int count;
  int tile[kMaxBatch + 1];
};

__device__ __forceinline__ float h2f(uint16_t bits) { return (float)__builtin_bit_cast(half_t, bits); }
__device__ __forceinline__ uint16_t f2h(float v) { return __builtin_bit_cast(uint16_t, (half_t)v); }

// Request index owning packed row t (t < r.start[r.count]).
__device__ __forceinline__ int ragged_find(const Ragged& r, int t) {
  int b = 0;
  while (b + 1 < r.count && t >= r.start[b + 1]) ++b;
  return b;
}

// s_waitcnt immediate waiting for at most `n` outstanding vector memory
// operations (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt
// left at their maxima).
constexpr int vmcnt_imm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

}  // namespace nemo
