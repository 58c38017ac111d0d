// Seeded synthetic weights on the device (see nemo_synth.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nemo {

uint64_t synth_key(uint64_t seed, uint64_t stream_id);
hipError_t launch_synth_q4k(uint64_t key, float sigma, int64_t n_blocks, uint8_t* out, hipStream_t stream);
hipError_t launch_synth_q6k(uint64_t key, float sigma, int64_t n_blocks, uint8_t* rec, uint16_t* d, hipStream_t stream);
hipError_t launch_synth_f16(uint64_t key, float sigma, int64_t n, uint16_t* out, hipStream_t stream);
hipError_t launch_fill_f32(float value, int64_t n, float* out, hipStream_t stream);

}  // namespace nemo
