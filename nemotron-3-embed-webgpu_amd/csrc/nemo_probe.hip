// Roofline probes: the launch and streaming floors that the HBM-bound kernels
// (the GEMV, the dequantization) are measured against. An empty kernel gives
// the cost of one launch replayed back to back; the streaming kernel reads a
// buffer once with fully coalesced 16-byte loads and does nothing else, so
// its time is the least any kernel reading those bytes in one launch can take.
#include "nemo_common.h"
#include "nemo_quant.h"

namespace nemo {

__global__ __launch_bounds__(64) void probe_empty_kernel() {}

// Workgroup g reads vectors [g 256 U, (g + 1) 256 U) of the buffer, thread t
// the vectors g 256 U + 256 u + t (u < U), so each load instruction of a wave
// covers 1 KiB of consecutive bytes. The xor of what a thread read is stored
// only if it equals a value the caller passes and the data never yields in
// practice, so the loads cannot be dropped and nothing is written.
template <int U>
__global__ __launch_bounds__(256) void probe_stream_kernel(const u32x4* __restrict__ src, int64_t nvec, uint32_t magic,
                                                           uint32_t* __restrict__ sink) {
  const int64_t base = (int64_t)blockIdx.x * (256 * U) + threadIdx.x;
  u32x4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + 256 * u;
    v[u] = i < nvec ? __builtin_nontemporal_load(src + i) : u32x4{0, 0, 0, 0};
  }
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  if (acc == magic) sink[blockIdx.x & 255] = acc;
}

hipError_t launch_probe_empty(hipStream_t stream) {
  probe_empty_kernel<<<1, 64, 0, stream>>>();
  return hipGetLastError();
}

hipError_t launch_probe_stream(const void* src, int64_t bytes, int loads, uint32_t* sink, hipStream_t stream) {
  if (bytes <= 0 || bytes % 16 || ((uintptr_t)src & 15)) return hipErrorInvalidValue;
  const int64_t nvec = bytes / 16;
  const unsigned grid = (unsigned)((nvec + 256 * loads - 1) / (256 * loads));
  const uint32_t magic = 0x9e3779b9u;
  const u32x4* s = (const u32x4*)src;
  switch (loads) {
    case 1: probe_stream_kernel<1><<<grid, 256, 0, stream>>>(s, nvec, magic, sink); break;
    case 2: probe_stream_kernel<2><<<grid, 256, 0, stream>>>(s, nvec, magic, sink); break;
    case 4: probe_stream_kernel<4><<<grid, 256, 0, stream>>>(s, nvec, magic, sink); break;
    case 8: probe_stream_kernel<8><<<grid, 256, 0, stream>>>(s, nvec, magic, sink); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace nemo
