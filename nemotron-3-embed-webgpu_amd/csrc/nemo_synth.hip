// Seeded synthetic weights, generated on the device: N(0, sigma) values from
// a counter-based splitmix64 stream with Box-Muller, quantized to Q4_K
// (144-byte GGUF blocks) or Q6_K (the split layout of QWeight), or stored as
// f16. Used by nemo_model_synthesize for shape-true benchmark models.
//
// The Q4_K quantizer: per 32-value sub-block, offset = -min(0, min x) and
// step = (max x + offset) / 15; d = max step / 63, dmin = max offset / 63
// (both f16); sc = round(step / d), m = round(offset / dmin) clamped to
// 0..63; q = round((x + dmin m) / (d sc)) clamped to 0..15. The 6-bit
// scale/min packing is the inverse of scaleAndMin
// (src/gguf/quantization.ts:11-17).
// The Q6_K quantizer: per 16-value group, step = amax / 31; d = max step /
// 127 (f16); scale = round(step / d) clamped to 1..127; q = round(x / (d
// scale)) + 32 clamped to 0..63, placed per src/gguf/quantization.ts:53-71.
#include "nemo_common.h"
#include "nemo_synth.h"

namespace nemo {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Value `index` of stream `key`: the index-th splitmix64 output, mapped to a
// normal deviate by Box-Muller on its two 24-bit halves.
__device__ __forceinline__ float synth_normal(uint64_t key, uint64_t index) {
  const uint64_t r = mix64(key + (index + 1) * 0x9E3779B97F4A7C15ull);
  const float u1 = ((float)((r >> 40) & 0xffffffu) + 1.0f) * (1.0f / 16777216.0f);
  const float u2 = (float)((r >> 8) & 0xffffffu) * (1.0f / 16777216.0f);
  return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}

__device__ __forceinline__ float round_f16(float v) { return h2f(f2h(v)); }

__global__ void synth_q4k_kernel(uint64_t key, float sigma, int64_t n_blocks, uint8_t* __restrict__ out) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const uint64_t base = (uint64_t)b * 256;
  float step[8], offset[8];
  float max_step = 0.f, max_offset = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float lo = 0.f, hi = -INFINITY;
    for (int i = 0; i < 32; ++i) {
      const float x = sigma * synth_normal(key, base + 32 * j + i);
      lo = fminf(lo, x);
      hi = fmaxf(hi, x);
    }
    offset[j] = -lo;
    step[j] = (hi + offset[j]) / 15.0f;
    max_step = fmaxf(max_step, step[j]);
    max_offset = fmaxf(max_offset, offset[j]);
  }
  const uint16_t d_bits = f2h(max_step / 63.0f), dmin_bits = f2h(max_offset / 63.0f);
  const float d = h2f(d_bits), dmin = h2f(dmin_bits);
  uint32_t sc[8], m[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    sc[j] = d > 0.f ? (uint32_t)fminf(63.f, fmaxf(0.f, rintf(step[j] / d))) : 0u;
    m[j] = dmin > 0.f ? (uint32_t)fminf(63.f, fmaxf(0.f, rintf(offset[j] / dmin))) : 0u;
  }
  uint8_t* blk = out + b * 144;
  blk[0] = d_bits & 0xff;
  blk[1] = d_bits >> 8;
  blk[2] = dmin_bits & 0xff;
  blk[3] = dmin_bits >> 8;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    blk[4 + j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
    blk[8 + j] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
    blk[12 + j] = (uint8_t)((sc[j + 4] & 15u) | ((m[j + 4] & 15u) << 4));
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float s0 = d * (float)sc[2 * g], s1 = d * (float)sc[2 * g + 1];
    const float o0 = dmin * (float)m[2 * g], o1 = dmin * (float)m[2 * g + 1];
    for (int l = 0; l < 32; ++l) {
      const float x0 = sigma * synth_normal(key, base + 64 * g + l);
      const float x1 = sigma * synth_normal(key, base + 64 * g + 32 + l);
      const uint32_t q0 = s0 > 0.f ? (uint32_t)fminf(15.f, fmaxf(0.f, rintf((x0 + o0) / s0))) : 0u;
      const uint32_t q1 = s1 > 0.f ? (uint32_t)fminf(15.f, fmaxf(0.f, rintf((x1 + o1) / s1))) : 0u;
      blk[16 + 32 * g + l] = (uint8_t)(q0 | (q1 << 4));
    }
  }
}

__global__ void synth_q6k_kernel(uint64_t key, float sigma, int64_t n_blocks, uint8_t* __restrict__ rec_out,
                                 uint16_t* __restrict__ d_out) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const uint64_t base = (uint64_t)b * 256;
  float step[16];
  float max_step = 0.f;
#pragma unroll
  for (int g = 0; g < 16; ++g) {
    float amax = 0.f;
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(sigma * synth_normal(key, base + 16 * g + i)));
    step[g] = amax / 31.0f;
    max_step = fmaxf(max_step, step[g]);
  }
  const uint16_t d_bits = f2h(max_step / 127.0f);
  const float d = h2f(d_bits);
  int sc[16];
  uint8_t* rec = rec_out + b * 208;
#pragma unroll
  for (int g = 0; g < 16; ++g) {
    sc[g] = d > 0.f ? (int)fminf(127.f, fmaxf(1.f, rintf(step[g] / d))) : 1;
    rec[192 + g] = (uint8_t)(int8_t)sc[g];
  }
  d_out[b] = d_bits;
  // Value e = 128 h + 32 Q + l sits in ql[64h + l + 32 (Q & 1)] (high nibble
  // for Q >= 2) and qh[32h + l] bits 2Q..2Q+1; its scale is group e / 16.
  for (int h = 0; h < 2; ++h) {
    for (int l = 0; l < 32; ++l) {
      uint32_t q[4];
#pragma unroll
      for (int Q = 0; Q < 4; ++Q) {
        const int e = 128 * h + 32 * Q + l;
        const float s = d * (float)sc[8 * h + 2 * Q + (l >> 4)];
        const float x = sigma * synth_normal(key, base + e);
        q[Q] = (uint32_t)fminf(63.f, fmaxf(0.f, rintf(x / s) + 32.f));
      }
      rec[64 * h + l] = (uint8_t)((q[0] & 15u) | ((q[2] & 15u) << 4));
      rec[64 * h + 32 + l] = (uint8_t)((q[1] & 15u) | ((q[3] & 15u) << 4));
      rec[128 + 32 * h + l] = (uint8_t)((q[0] >> 4) | ((q[1] >> 4) << 2) | ((q[2] >> 4) << 4) | ((q[3] >> 4) << 6));
    }
  }
}

__global__ void synth_f16_kernel(uint64_t key, float sigma, int64_t n, uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = f2h(sigma * synth_normal(key, (uint64_t)i));
}

__global__ void fill_f32_kernel(float value, int64_t n, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = value;
}

static uint64_t host_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t synth_key(uint64_t seed, uint64_t stream_id) { return host_mix64(seed ^ host_mix64(stream_id + 1)); }

hipError_t launch_synth_q4k(uint64_t key, float sigma, int64_t n_blocks, uint8_t* out, hipStream_t stream) {
  synth_q4k_kernel<<<(unsigned)((n_blocks + 127) / 128), 128, 0, stream>>>(key, sigma, n_blocks, out);
  return hipGetLastError();
}

hipError_t launch_synth_q6k(uint64_t key, float sigma, int64_t n_blocks, uint8_t* rec, uint16_t* d, hipStream_t stream) {
  synth_q6k_kernel<<<(unsigned)((n_blocks + 127) / 128), 128, 0, stream>>>(key, sigma, n_blocks, rec, d);
  return hipGetLastError();
}

hipError_t launch_synth_f16(uint64_t key, float sigma, int64_t n, uint16_t* out, hipStream_t stream) {
  synth_f16_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(key, sigma, n, out);
  return hipGetLastError();
}

hipError_t launch_fill_f32(float value, int64_t n, float* out, hipStream_t stream) {
  fill_f32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(value, n, out);
  return hipGetLastError();
}

}  // namespace nemo
