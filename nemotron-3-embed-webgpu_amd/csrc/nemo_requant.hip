// Offline requantization of GGML matrices to Q4_0 on the GPU:
// requantizeMatrixToQ40 / quantizeQ40Block (src/gguf/quantization.ts:77-131),
// bit-exact with the reference's JavaScript.
//
// One thread per output Q4_0 block (32 values). The source values are decoded
// to the float32 values the reference's decoders store (exact single
// roundings, see nemo_blocks.h), then quantized as quantizeQ40Block does in
// double precision: the first value of largest magnitude sets
// scale = signed max / -8, the stored scale is that value rounded to float32
// and encoded to binary16 with the reference's round-half-away-from-zero
// (src/math/f16.ts:4-25), and each quant is clamp(floor(v * (1 / scale) +
// 8.5), 0, 15) with the product and the sum rounded separately (no fused
// multiply-add), as JavaScript evaluates them. Q6_K sub-blocks put many
// v / scale exactly on half-integers, where one fused rounding would move
// the floor. A NaN quant becomes 0 (NaN | x is x in JavaScript).
#include "nemo_blocks.h"
#include "nemo_common.h"
#include "nemo_quant.h"

// JavaScript rounds every product and sum: no fused multiply-add here.
#pragma clang fp contract(off)

namespace nemo {

// binary32 -> binary16 bits, nearest with ties away from zero; overflow and
// NaN give infinity; values below half the smallest subnormal give zero.
__device__ __forceinline__ uint16_t f16_bits_ties_away(float value) {
  const uint32_t bits = __float_as_uint(value);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  int exponent = (int)((bits >> 23) & 0xffu) - 127 + 15;
  uint32_t mantissa = bits & 0x7fffffu;
  if (exponent <= 0) {
    if (exponent < -10) return (uint16_t)sign;
    mantissa = (mantissa | 0x800000u) >> (1 - exponent);
    return (uint16_t)(sign | ((mantissa + 0x1000u) >> 13));
  }
  if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
  if (mantissa & 0x1000u) {
    mantissa += 0x2000u;
    if (mantissa & 0x800000u) {
      mantissa = 0;
      exponent += 1;
      if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    }
  }
  return (uint16_t)(sign | ((uint32_t)exponent << 10) | (mantissa >> 13));
}

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// The 32 float32 values of sub-block `sub` (0..7) of a 256-value K-quant
// block, or of a Q4_0 block (sub ignored).
template <int TYPE>
__device__ __forceinline__ void decode32(const uint8_t* blk, int sub, float* v) {
  if constexpr (TYPE == kQ4_K) {
    // src/gguf/quantization.ts:11-38
    const float d = h2f((uint16_t)ld_u16(blk)), dmin = h2f((uint16_t)ld_u16(blk + 2));
    const uint8_t* s = blk + 4;
    int sc, m;
    if (sub < 4) {
      sc = s[sub] & 63;
      m = s[sub + 4] & 63;
    } else {
      sc = (s[sub + 4] & 15) | ((s[sub - 4] >> 6) << 4);
      m = (s[sub + 4] >> 4) | ((s[sub] >> 6) << 4);
    }
    const float dsc = d * (float)sc, ndm = -(dmin * (float)m);
    const uint8_t* q = blk + 16 + 32 * (sub >> 1);
    const int sh = 4 * (sub & 1);
    for (int l = 0; l < 32; ++l) v[l] = fmaf(dsc, (float)((q[l] >> sh) & 15), ndm);
  } else if constexpr (TYPE == kQ6_K) {
    // src/gguf/quantization.ts:46-74: value 128h + 32Q + l
    const float d = h2f((uint16_t)ld_u16(blk + 208));
    const int h = sub >> 2, Q = sub & 3;
    const uint8_t* ql = blk + 64 * h + 32 * (Q & 1);
    const uint8_t* qh = blk + 128 + 32 * h;
    const int8_t* sc = (const int8_t*)(blk + 192 + 8 * h + 2 * Q);
    for (int l = 0; l < 32; ++l) {
      const int low = Q >= 2 ? (ql[l] >> 4) : (ql[l] & 15);
      const int high = (qh[l] >> (2 * Q)) & 3;
      v[l] = (d * (float)sc[l >> 4]) * (float)((low | (high << 4)) - 32);
    }
  } else {
    // src/gguf/quantization.ts:40-44
    const float d = h2f((uint16_t)ld_u16(blk));
    for (int l = 0; l < 16; ++l) {
      v[l] = d * (float)((blk[2 + l] & 15) - 8);
      v[l + 16] = d * (float)((blk[2 + l] >> 4) - 8);
    }
  }
}

__device__ __forceinline__ uint32_t quant_nibble(float value, double inverse) {
  double product = (double)value * inverse;
  asm volatile("" : "+v"(product));  // keep the product rounded on its own
  const double q = floor(product + 8.5);
  if (isnan(q)) return 0;
  return (uint32_t)(q < 0.0 ? 0.0 : (q > 15.0 ? 15.0 : q));
}

template <int TYPE>
__global__ __launch_bounds__(256) void requant_q40_kernel(const uint8_t* __restrict__ src, int64_t k, int64_t n,
                                                          uint8_t* __restrict__ out) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = k / 32;
  if (o >= n * per_row) return;
  const int64_t row = o / per_row, j = o % per_row;
  float v[32];
  if constexpr (TYPE == kQ4_0) {
    decode32<TYPE>(src + o * 18, 0, v);
  } else {
    const int bytes = TYPE == kQ4_K ? 144 : 210;
    decode32<TYPE>(src + (row * (k / 256) + j / 8) * bytes, (int)(j % 8), v);
  }
  // quantizeQ40Block (src/gguf/quantization.ts:77-98)
  double signed_max = 0.0, max_abs = 0.0;
  for (int l = 0; l < 32; ++l) {
    const double a = fabs((double)v[l]);
    if (a > max_abs) {
      max_abs = a;
      signed_max = (double)v[l];
    }
  }
  const double scale = signed_max == 0.0 ? 0.0 : signed_max / -8.0;
  const double inverse = scale == 0.0 ? 0.0 : 1.0 / scale;
  uint16_t words[9];
  words[0] = f16_bits_ties_away((float)scale);
  for (int l = 0; l < 16; l += 2) {
    const uint32_t b0 = quant_nibble(v[l], inverse) | (quant_nibble(v[l + 16], inverse) << 4);
    const uint32_t b1 = quant_nibble(v[l + 1], inverse) | (quant_nibble(v[l + 17], inverse) << 4);
    words[1 + l / 2] = (uint16_t)(b0 | (b1 << 8));
  }
  uint16_t* dst = (uint16_t*)(out + o * 18);  // 18-byte records: 2-byte aligned
  for (int i = 0; i < 9; ++i) dst[i] = words[i];
}

hipError_t launch_requant_q40(int src_type, const uint8_t* src, int64_t k, int64_t n, uint8_t* out,
                              hipStream_t stream) {
  const int64_t blocks = n * (k / 32);
  if (blocks <= 0) return hipSuccess;
  const unsigned grid = (unsigned)((blocks + 255) / 256);
  if (src_type == kQ4_K) requant_q40_kernel<kQ4_K><<<grid, 256, 0, stream>>>(src, k, n, out);
  else if (src_type == kQ6_K) requant_q40_kernel<kQ6_K><<<grid, 256, 0, stream>>>(src, k, n, out);
  else if (src_type == kQ4_0) requant_q40_kernel<kQ4_0><<<grid, 256, 0, stream>>>(src, k, n, out);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace nemo
