// Seeded synthetic parameters on the device (synth.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace presk {

// n values mean + std * z at dst, z ~ N(0, 1) from a counter-based hash of
// (seed, element index), stored as `type` (convert_type's codes: 1 f32,
// 2 bf16, 4 f16), each rounded once to nearest even.
hipError_t synth_normal_launch(void* dst, int type, long long n, unsigned long long seed, float mean, float std,
                               hipStream_t s);

}  // namespace presk
