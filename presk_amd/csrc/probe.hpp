// The measured MFMA peak (probe.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace presk {

// One timed launch (after an untimed one) of independent MFMA loops on every
// CU: kind 0 bf16 32x32x16, 1 f32 16x16x4, `iters` rounds of eight MFMAs a
// wave; *ms its duration, *flops the flops it performed.
hipError_t mfma_probe(int kind, long long iters, hipStream_t stream, double* ms, double* flops);

}  // namespace presk
