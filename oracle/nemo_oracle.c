/*
 * CPU oracle for the Nemotron-3-Embed encoder hot path: codec half.
 *
 * TEST INFRASTRUCTURE ONLY. This file restates, in plain C, the reference's
 * CPU arithmetic for the quantized-weight codecs and the few integer helpers
 * of the execution plan. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker (or the timed CPU
 * baseline); the product path never links or calls it.
 *
 * Every function cites the reference file:line it follows. Pins (what checks
 * each function against something other than itself) are listed in the
 * header of oracle/oracle.py.
 *
 * Arithmetic model: the reference is JavaScript, so every expression is
 * evaluated in IEEE double and stored into a Float32Array (round to nearest
 * even). We do exactly that: compute in double, cast once to float.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <string.h>

/* src/gguf/quantization.ts:2-9 halfToFloat: binary16 bits -> JS number. */
double oracle_half_to_float(uint32_t bits) {
  const double sign = (bits & 0x8000u) ? -1.0 : 1.0;
  const uint32_t exponent = (bits >> 10) & 0x1fu;
  const uint32_t fraction = bits & 0x3ffu;
  if (exponent == 0) return sign * ldexp(1.0, -14) * ((double)fraction / 1024.0);
  if (exponent == 0x1f) return fraction ? NAN : sign * INFINITY;
  return sign * ldexp(1.0, (int)exponent - 15) * (1.0 + (double)fraction / 1024.0);
}

/* src/math/f16.ts:4-25 floatToHalf. The value is first stored into a
 * Float32Array (f16.ts:5), then rounded half-away-from-zero on the mantissa
 * (f16.ts:16-22), not round-to-nearest-even. NaN maps to infinity, as there. */
uint16_t oracle_float_to_half(float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  int32_t exponent = (int32_t)((bits >> 23) & 0xffu) - 127 + 15;
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

void oracle_float_to_half_array(const float* values, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_float_to_half(values[i]);
}

static uint16_t load_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* src/gguf/quantization.ts:11-17 scaleAndMin: 6-bit scale and min of
 * sub-block `index` (0..7) from the 12 packed scale bytes. */
void oracle_q4k_scale_min(const uint8_t* scales, int index, int* scale, int* minimum) {
  if (index < 4) {
    *scale = scales[index] & 63;
    *minimum = scales[index + 4] & 63;
    return;
  }
  *scale = (scales[index + 4] & 0x0f) | ((scales[index - 4] >> 6) << 4);
  *minimum = (scales[index + 4] >> 4) | ((scales[index] >> 6) << 4);
}

/* src/gguf/quantization.ts:19-38 dequantizeQ4KBlock, over `nblocks`
 * consecutive 144-byte super-blocks. */
void oracle_dequant_q4k(const uint8_t* bytes, int64_t nblocks, float* out) {
  for (int64_t b = 0; b < nblocks; ++b) {
    const uint8_t* block = bytes + b * 144;
    float* output = out + b * 256;
    const double d = oracle_half_to_float(load_u16(block));
    const double dmin = oracle_half_to_float(load_u16(block + 2));
    const uint8_t* scales = block + 4;
    const uint8_t* quants = block + 16;
    int scale_index = 0;
    for (int group = 0; group < 4; ++group) {
      int scale_low, min_low, scale_high, min_high;
      oracle_q4k_scale_min(scales, scale_index++, &scale_low, &min_low);
      oracle_q4k_scale_min(scales, scale_index++, &scale_high, &min_high);
      for (int lane = 0; lane < 32; ++lane) {
        const uint32_t packed = quants[group * 32 + lane];
        output[group * 64 + lane] = (float)(d * scale_low * (double)(packed & 0x0f) - dmin * min_low);
        output[group * 64 + lane + 32] = (float)(d * scale_high * (double)(packed >> 4) - dmin * min_high);
      }
    }
  }
}

/* src/gguf/quantization.ts:40-44 dequantizeQ40Block, over 18-byte blocks. */
void oracle_dequant_q40(const uint8_t* bytes, int64_t nblocks, float* out) {
  for (int64_t b = 0; b < nblocks; ++b) {
    const uint8_t* block = bytes + b * 18;
    const double d = oracle_half_to_float(load_u16(block));
    for (int lane = 0; lane < 16; ++lane) {
      const int packed = block[2 + lane];
      out[b * 32 + lane] = (float)(d * (double)((packed & 15) - 8));
      out[b * 32 + lane + 16] = (float)(d * (double)((packed >> 4) - 8));
    }
  }
}

/* src/gguf/quantization.ts:46-74 dequantizeQ6KBlock, over 210-byte blocks. */
void oracle_dequant_q6k(const uint8_t* bytes, int64_t nblocks, float* out) {
  for (int64_t b = 0; b < nblocks; ++b) {
    const uint8_t* block = bytes + b * 210;
    float* output = out + b * 256;
    const uint8_t* ql = block;
    const uint8_t* qh = block + 128;
    const int8_t* scales = (const int8_t*)(block + 192);
    const double d = oracle_half_to_float(load_u16(block + 208));
    for (int half = 0; half < 2; ++half) {
      const int low_offset = half * 64, high_offset = half * 32, scale_offset = half * 8, output_offset = half * 128;
      for (int lane = 0; lane < 32; ++lane) {
        const int scale_pair = lane >> 4;
        const int high = qh[high_offset + lane];
        const int low_a = ql[low_offset + lane];
        const int low_b = ql[low_offset + lane + 32];
        const int q1 = (low_a & 15) | ((high & 3) << 4);
        const int q2 = (low_b & 15) | (((high >> 2) & 3) << 4);
        const int q3 = (low_a >> 4) | (((high >> 4) & 3) << 4);
        const int q4 = (low_b >> 4) | (((high >> 6) & 3) << 4);
        output[output_offset + lane] = (float)(d * scales[scale_offset + scale_pair] * (double)(q1 - 32));
        output[output_offset + lane + 32] = (float)(d * scales[scale_offset + scale_pair + 2] * (double)(q2 - 32));
        output[output_offset + lane + 64] = (float)(d * scales[scale_offset + scale_pair + 4] * (double)(q3 - 32));
        output[output_offset + lane + 96] = (float)(d * scales[scale_offset + scale_pair + 6] * (double)(q4 - 32));
      }
    }
  }
}

/* src/gguf/quantization.ts:77-98 quantizeQ40Block: 32 values -> 18 bytes. */
void oracle_quantize_q40_block(const float* values, uint8_t* output) {
  double signed_maximum = 0, maximum_absolute = 0;
  for (int i = 0; i < 32; ++i) {
    const double value = values[i];
    const double absolute = fabs(value);
    if (absolute > maximum_absolute) {
      maximum_absolute = absolute;
      signed_maximum = value;
    }
  }
  const double scale = signed_maximum == 0 ? 0 : signed_maximum / -8;
  const double inverse_scale = scale == 0 ? 0 : 1 / scale;
  const uint16_t scale_bits = oracle_float_to_half((float)scale);
  output[0] = (uint8_t)(scale_bits & 0xff);
  output[1] = (uint8_t)(scale_bits >> 8);
  for (int i = 0; i < 16; ++i) {
    /* Math.min(15, Math.max(0, NaN)) is NaN, and NaN | x == x in JS. */
    double low = floor((double)values[i] * inverse_scale + 8.5);
    double high = floor((double)values[i + 16] * inverse_scale + 8.5);
    low = isnan(low) ? 0 : (low < 0 ? 0 : (low > 15 ? 15 : low));
    high = isnan(high) ? 0 : (high < 0 ? 0 : (high > 15 ? 15 : high));
    output[i + 2] = (uint8_t)((int)low | ((int)high << 4));
  }
}

/* src/gguf/quantization.ts:101-131 requantizeMatrixToQ40 (type 2, 12 or 14).
 * Returns 0 on success, -1 for an unsupported K, -2 for an unknown type. */
int oracle_requantize_to_q40(const uint8_t* bytes, int type, int64_t k, int64_t n, uint8_t* output) {
  if (k % 256 != 0) return -1;
  const int source_block_bytes = type == 12 ? 144 : type == 14 ? 210 : 18;
  const int source_block_values = type == 2 ? 32 : 256;
  if (type != 2 && type != 12 && type != 14) return -2;
  float decoded[256];
  int64_t source_offset = 0, output_offset = 0;
  for (int64_t row = 0; row < n; ++row) {
    for (int64_t column = 0; column < k; column += source_block_values) {
      if (type == 12) oracle_dequant_q4k(bytes + source_offset, 1, decoded);
      else if (type == 14) oracle_dequant_q6k(bytes + source_offset, 1, decoded);
      else oracle_dequant_q40(bytes + source_offset, 1, decoded);
      for (int sub = 0; sub < source_block_values; sub += 32) {
        oracle_quantize_q40_block(decoded + sub, output + output_offset);
        output_offset += 18;
      }
      source_offset += source_block_bytes;
    }
  }
  return 0;
}

/* src/prepacked/format.ts:65-99 packQ40Tile32 for one concatenated Q4_0
 * matrix of n rows x k columns (18-byte blocks, row-major): output is
 * tile -> kBlock -> row32 records of [f16 d][2 zero bytes][16 nibble bytes]. */
void oracle_pack_q40_tile32(const uint8_t* q40, int64_t k, int64_t n, uint8_t* output) {
  const int64_t k_blocks = k / 32;
  const int64_t n_tiles = (n + 31) / 32;
  memset(output, 0, (size_t)(n_tiles * k_blocks * 32 * 20));
  for (int64_t tile = 0; tile < n_tiles; ++tile)
    for (int64_t kb = 0; kb < k_blocks; ++kb)
      for (int64_t local_row = 0; local_row < 32; ++local_row) {
        const int64_t row = tile * 32 + local_row;
        if (row >= n) continue;
        const uint8_t* source = q40 + (row * k_blocks + kb) * 18;
        uint8_t* destination = output + ((tile * k_blocks + kb) * 32 + local_row) * 20;
        destination[0] = source[0];
        destination[1] = source[1];
        memcpy(destination + 4, source + 2, 16);
      }
}

/* src/webgpu/model.ts:30-32 contextualMergedLength, in double like JS. */
int oracle_contextual_merged_length(int sequence) {
  const double merged = ceil((double)sequence * 0.64);
  return merged < 1 ? 1 : (int)merged;
}

/* Scalar reference dot products of the dead kernel microbenchmark
 * (src/main.ts:97-104): expected = sum_k x[m][k] * dequant(W)[n][k] in
 * double, for every (m, n). x is float (the JS inputValues), W is the f32
 * dequantized matrix. This is also the timed CPU baseline of the Q4_K
 * dequant-matmul. */
void oracle_matmul_f64(const float* x, const float* w, int64_t m, int64_t n, int64_t k, double* out) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double expected = 0;
      const float* xr = x + i * k;
      const float* wr = w + j * k;
      for (int64_t t = 0; t < k; ++t) expected += (double)xr[t] * (double)wr[t];
      out[i * n + j] = expected;
    }
}

/* The CPU baseline of the Q4_K dequant-matmul as the reference CPU path does
 * it: dequantize each weight row block by block (src/main.ts:98-100 with
 * src/gguf/quantization.ts:19-38), then a scalar double dot per output
 * (src/main.ts:101-104). Returns a checksum so the work cannot be elided. */
double oracle_q4k_matmul_cpu(const uint8_t* w, const float* x, int64_t m, int64_t n, int64_t k, float* row_scratch, double* out) {
  const int64_t blocks = k / 256;
  double checksum = 0;
  for (int64_t j = 0; j < n; ++j) {
    oracle_dequant_q4k(w + j * blocks * 144, blocks, row_scratch);
    for (int64_t i = 0; i < m; ++i) {
      double expected = 0;
      const float* xr = x + i * k;
      for (int64_t t = 0; t < k; ++t) expected += (double)xr[t] * (double)row_scratch[t];
      out[i * n + j] = expected;
      checksum += expected;
    }
  }
  return checksum;
}

/* The same computation spread over `threads` OpenMP threads by weight row
 * (each row's outputs computed exactly as above, so the results are the same
 * bits); the all-cores variant of the CPU baseline. row_scratch holds
 * threads * k floats. */
double oracle_q4k_matmul_cpu_mt(const uint8_t* w, const float* x, int64_t m, int64_t n, int64_t k, int threads,
                                float* row_scratch, double* out) {
  const int64_t blocks = k / 256;
  double checksum = 0;
#pragma omp parallel for num_threads(threads) schedule(static) reduction(+ : checksum)
  for (int64_t j = 0; j < n; ++j) {
    float* row = row_scratch + (int64_t)omp_get_thread_num() * k;
    oracle_dequant_q4k(w + j * blocks * 144, blocks, row);
    for (int64_t i = 0; i < m; ++i) {
      double expected = 0;
      const float* xr = x + i * k;
      for (int64_t t = 0; t < k; ++t) expected += (double)xr[t] * (double)row[t];
      out[i * n + j] = expected;
      checksum += expected;
    }
  }
  return checksum;
}
