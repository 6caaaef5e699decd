// The edge conversion between storage types (convert.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

namespace presk {

// 0 f64, 1 f32, 2 bf16, 4 f16, 5 e8m15 (3, i64, is never converted); -1 else
int convert_type(const char* name);
hipError_t convert_launch(const void* src, int from, void* dst, int to, long long n, unsigned* flag, hipStream_t s);
// a training dropout mask of n elements of type `type` (convert_type's
// codes) from the 32-byte key at `key` (device memory, 4-byte aligned)
hipError_t dropout_launch(const void* key, double rate, int type, long long n, void* dst, hipStream_t s);

}  // namespace presk
