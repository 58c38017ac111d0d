// Device-side GGML block decoding shared by the GEMM, GEMV and dequant
// kernels (gfx950).
//
// Decoding follows src/gguf/quantization.ts:11-74 (and the WGSL decoders of
// src/webgpu/quant-matmul.ts:37-154). Every decoded weight is formed in fp32
// exactly as the reference's JavaScript forms it: d*sc and dmin*m are exact
// products of an 11-bit and a 6-bit significand, d*sc*q is exact (<= 21
// bits), so one fmaf(d*sc, q, -dmin*m) rounds the exact value once - the
// same single rounding as the JS double expression stored to Float32Array.
// Q6_K: d*scale*(q-32) has <= 23 significant bits and is exact in fp32.
// MFMA operands are f16(RNE(that fp32 value)), as the WGSL tiles are.
#pragma once

#include "nemo_common.h"
#include "nemo_quant.h"

namespace nemo {

typedef float float8v __attribute__((ext_vector_type(8)));

// fp32 factors of group g (sub-blocks 2g, 2g+1): w = fmaf(dsc, q, ndm).
// scaleAndMin (src/gguf/quantization.ts:11-17) on whole words, branch-free:
// with the 12 scale bytes s[0..11] in hdr.y, hdr.z, hdr.w, sub-block j < 4
// has scale s[j] & 63 and min s[j+4] & 63; sub-block j >= 4 has scale
// (s[j+4] & 15) | (s[j-4] >> 6) << 4 and min (s[j+4] >> 4) | (s[j] >> 6) << 4.
// Per byte, (x >> 6) << 4 is ((word >> 2) & 0x30).
__device__ __forceinline__ void q4k_group_factors(const u32x4& hdr, int g, float& dsc0, float& ndm0, float& dsc1,
                                                  float& ndm1) {
  const float d = h2f((uint16_t)(hdr.x & 0xffffu));
  const float dmin = h2f((uint16_t)(hdr.x >> 16));
  // Bitwise blend rather than a conditional: g is uniform, and a branch would
  // split the GEMM's step into several basic blocks.
  const uint32_t hi = 0u - (uint32_t)(g >> 1);
  const uint32_t scw = ((hdr.y & 0x3f3f3f3fu) & ~hi) | (((hdr.w & 0x0f0f0f0fu) | ((hdr.y >> 2) & 0x30303030u)) & hi);
  const uint32_t mw =
      ((hdr.z & 0x3f3f3f3fu) & ~hi) | ((((hdr.w >> 4) & 0x0f0f0f0fu) | ((hdr.z >> 2) & 0x30303030u)) & hi);
  const int sh = 16 * (g & 1);
  dsc0 = d * (float)((scw >> sh) & 0xffu);
  ndm0 = -(dmin * (float)((mw >> sh) & 0xffu));
  dsc1 = d * (float)((scw >> (sh + 8)) & 0xffu);
  ndm1 = -(dmin * (float)((mw >> (sh + 8)) & 0xffu));
}

// Hides a value's known bits from the optimizer so that byte extraction of a
// masked word compiles to v_cvt_f32_ubyte{0..3} (one instruction per value)
// rather than a bit-field extract followed by a conversion.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Four packed bytes (one value per byte) -> four fp32 values scale*b + bias.
__device__ __forceinline__ void bytes4_fma(uint32_t w, float scale, float bias, float* out) {
  out[0] = fmaf(scale, (float)(w & 0xffu), bias);
  out[1] = fmaf(scale, (float)((w >> 8) & 0xffu), bias);
  out[2] = fmaf(scale, (float)((w >> 16) & 0xffu), bias);
  out[3] = fmaf(scale, (float)(w >> 24), bias);
}

// Four packed 4-bit values (one per byte, each 0..15) -> four fp32 values
// fmaf(scale, b, bias), the same results as bytes4_fma. Read as OCP e4m3,
// a byte b <= 15 is exactly b * 2^-9 (the subnormals and the first binade
// share one spacing), so one conversion yields two values, and the fma takes
// scale * 2^9, which is exact: the product, and so the rounded sum, is the
// same. Half the conversions of bytes4_fma (the decoders are VALU-bound).
__device__ __forceinline__ void nibbles4_fma(uint32_t w, float scale, float bias, float* out) {
  const float s9 = scale * 512.0f;
  const float2v a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const float2v b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  out[0] = fmaf(s9, a.x, bias);
  out[1] = fmaf(s9, a.y, bias);
  out[2] = fmaf(s9, b.x, bias);
  out[3] = fmaf(s9, b.y, bias);
}

// Round-to-nearest-even f32 -> f16 of eight values (v_cvt_pk_f16_f32 pairs).
__device__ __forceinline__ half8v to_half8(const float* v) {
  const float8v f = {v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
  return __builtin_convertvector(f, half8v);
}

// ---------------------------------------------------------------------------
// Tile loaders. A loader fetches, for one weight row and one 64-column chunk
// starting at k0, the bytes of "part" p (0/1) and later expands them to 32
// f16 values: lo[16] for columns k0+16p..k0+16p+15 and hi[16] for columns
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
    nibbles4_fma(words[i] & 0x0f0f0f0fu, dsc0, ndm0, vl + 4 * i);
    nibbles4_fma((words[i] >> 4) & 0x0f0f0f0fu, dsc1, ndm1, vh + 4 * i);
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
    bytes4_fma(opaque(q0), dsc0, -32.0f * dsc0, vl + 4 * i);
    bytes4_fma(opaque(q1), dsc1, -32.0f * dsc1, vh + 4 * i);
  }
  lo[0] = to_half8(vl);
  lo[1] = to_half8(vl + 8);
  hi[0] = to_half8(vh);
  hi[1] = to_half8(vh + 8);
}

// Q4_0 split layout: 16 nibble bytes per 32-value block, f16 d separate.
// Value j < 16 of a block is d (low nibble of byte j - 8), value 16 + j is
// d (high nibble of byte j - 8) (src/gguf/quantization.ts:40-44); d (q - 8)
// has at most 15 significant bits and is exact in fp32. For chunk k0 (a
// multiple of 64) and part p: lo = block k0/32, hi = block k0/32 + 1, each
// the low (p = 0) or high (p = 1) nibbles.
struct Q40Fetch {
  u32x4 q0, q1;
  uint16_t d0, d1;
  int p;
};

__device__ __forceinline__ Q40Fetch q40_fetch(const QWeight& w, size_t row_bytes, int row, int k0, int p) {
  const int b = k0 >> 5;
  const uint8_t* base = w.blocks + (size_t)row * row_bytes + (size_t)b * 16;
  Q40Fetch f;
  f.q0 = *(const u32x4*)base;
  f.q1 = *(const u32x4*)(base + 16);
  const uint16_t* d = w.d + (size_t)row * (w.k >> 5) + b;
  f.d0 = d[0];
  f.d1 = d[1];
  f.p = p;
  return f;
}

__device__ __forceinline__ void q40_expand(const Q40Fetch& f, half8v* lo, half8v* hi) {
  const float d0 = h2f(f.d0), d1 = h2f(f.d1);
  const int sh = 4 * f.p;
  const uint32_t a[4] = {f.q0.x, f.q0.y, f.q0.z, f.q0.w};
  const uint32_t b[4] = {f.q1.x, f.q1.y, f.q1.z, f.q1.w};
  float vl[16], vh[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    nibbles4_fma((a[i] >> sh) & 0x0f0f0f0fu, d0, -8.0f * d0, vl + 4 * i);
    nibbles4_fma((b[i] >> sh) & 0x0f0f0f0fu, d1, -8.0f * d1, vh + 4 * i);
  }
  lo[0] = to_half8(vl);
  lo[1] = to_half8(vl + 8);
  hi[0] = to_half8(vh);
  hi[1] = to_half8(vh + 8);
}

// Q4_K raw: 8 threads per 144-byte block. Thread c writes output chunks c,
// c + 8, c + 16, c + 24 of 8 values (values 64 i + 8 c .. +8 for group i),
// so each store instruction of 8 neighbouring lanes fills 128 contiguous
// bytes (f16) or 256 (f32): the low nibbles of bytes 8c .. 8c + 8 of every
// group's 32 (c < 4) or the high nibbles of bytes 8(c - 4) .. (c >= 4).
// NT: non-temporal stores, for output that is not read back soon.
// Thread c (0..7) of the 144-byte block at `blk`, whose values start at
// element o of the outputs.
template <bool NT>
__device__ __forceinline__ void q4k_block_part(const uint8_t* __restrict__ blk, int c, int64_t o0,
                                               float* __restrict__ out32, uint16_t* __restrict__ out16) {
  const int part = c & 3, high = c >> 2;
  const u32x4 hdr = *(const u32x4*)blk;
  uint32_t q[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint2 w = *(const uint2*)(blk + 16 + 32 * i + 8 * part);
    q[i][0] = w.x;
    q[i][1] = w.y;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float dsc0, ndm0, dsc1, ndm1;
    q4k_group_factors(hdr, i, dsc0, ndm0, dsc1, ndm1);
    const float dsc = high ? dsc1 : dsc0, ndm = high ? ndm1 : ndm0;
    const int sh = 4 * high;
    float v[8];
    nibbles4_fma((q[i][0] >> sh) & 0x0f0f0f0fu, dsc, ndm, v);
    nibbles4_fma((q[i][1] >> sh) & 0x0f0f0f0fu, dsc, ndm, v + 4);
    const int64_t o = o0 + 64 * i + 8 * c;
    if constexpr (NT) {
      if (out32) {
        __builtin_nontemporal_store(float4v{v[0], v[1], v[2], v[3]}, (float4v*)(out32 + o));
        __builtin_nontemporal_store(float4v{v[4], v[5], v[6], v[7]}, (float4v*)(out32 + o + 4));
      }
      if (out16) __builtin_nontemporal_store(to_half8(v), (half8v*)(out16 + o));
    } else {
      if (out32) {
        *(float4v*)(out32 + o) = float4v{v[0], v[1], v[2], v[3]};
        *(float4v*)(out32 + o + 4) = float4v{v[4], v[5], v[6], v[7]};
      }
      if (out16) *(half8v*)(out16 + o) = to_half8(v);
    }
  }
}

// Q6_K split layout -> f16 (the two-pass GEMM's first pass), 8 threads per
// 256-value block, thread c writing chunks c + 8 i of 8 values, so 8
// neighbouring lanes fill 128 contiguous bytes per store. Value 64 i + 8 c + j
// is (half h = i / 2, quadrant Q = 2 (i % 2) + c / 4, lane l = 8 (c % 4) + j)
// (src/gguf/quantization.ts:53-71): its low bits are the low (Q < 2) or high
// nibble of ql[64 h + 8 c + j], its high bits bits 2Q of
// qh[32 h + 8 (c % 4) + j], its scale sc[8 h + (c % 4) / 2 + 2 Q]. `rec` is the
// block's 208-byte record, `d_bits` its f16 scale, `out` its 256 values.
__device__ __forceinline__ void q6k_block_part(const uint8_t* __restrict__ rec, uint16_t d_bits, int c,
                                               uint16_t* __restrict__ out) {
  uint2 ql[2], qh[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    ql[h] = *(const uint2*)(rec + 64 * h + 8 * c);
    qh[h] = *(const uint2*)(rec + 128 + 32 * h + 8 * (c & 3));
  }
  const u32x4 sc = *(const u32x4*)(rec + 192);
  const uint32_t scw[4] = {sc.x, sc.y, sc.z, sc.w};
  const float d = h2f(d_bits);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = i >> 1, Q = 2 * (i & 1) + (c >> 2);
    const int si = 8 * h + ((c & 3) >> 1) + 2 * Q;
    const float dsc = d * (float)(int8_t)((scw[si >> 2] >> (8 * (si & 3))) & 0xffu);
    const int ls = 4 * (i & 1), hs = 2 * Q;
    const uint32_t w0 = ((ql[h].x >> ls) & 0x0f0f0f0fu) | (((qh[h].x >> hs) & 0x03030303u) << 4);
    const uint32_t w1 = ((ql[h].y >> ls) & 0x0f0f0f0fu) | (((qh[h].y >> hs) & 0x03030303u) << 4);
    float v[8];
    bytes4_fma(opaque(w0), dsc, -32.0f * dsc, v);
    bytes4_fma(opaque(w1), dsc, -32.0f * dsc, v + 4);
    *(half8v*)(out + 64 * i + 8 * c) = to_half8(v);
  }
}

// A matrix's Q4_K / Q6_K -> f16 expansion given to an f16 GEMM launch as side
// work, done by the workgroups past the GEMM's tiles (see gemm_f16_kernel).
// Thread c (0..7) of 256-value block b.
// Block b counts over the parts in order; each field is picked by value
// (no copy of a part that the compiler would index in private memory).
__device__ __forceinline__ void side_expand_part(const SideExpand& e, int64_t b, int c) {
  const bool second = e.count > 1 && b >= e.part[0].nblocks;
  if (second) b -= e.part[0].nblocks;
  const int type = second ? e.part[1].type : e.part[0].type;
  const uint8_t* blocks = second ? e.part[1].blocks : e.part[0].blocks;
  uint16_t* out = second ? e.part[1].out : e.part[0].out;
  if (type == kQ4_K) {
    q4k_block_part<false>(blocks + b * 144, c, b * 256, nullptr, out);
  } else {
    const uint16_t* d = second ? e.part[1].d : e.part[0].d;
    q6k_block_part(blocks + b * 208, d[b], c, out + b * 256);
  }
}

}  // namespace nemo
