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

// A float format given by its parameters (crates/presk-format/src/lib.rs:101-118),
// as a .psk.d version 3 header describes it: p bits of significand, the
// exponent range, subnormals, the special values (0 IEEE, 1 NaN only, 2 none);
// ebits, bits and width derived (exponent field bits, bits of a code, bytes).
struct PskFormat {
    int p, emin, emax;
    bool subnormals;
    int specials;
    int ebits, bits, width;
};
// n elements of a .psk.d real leaf (enc 0 f64, 1 f32, 2 bf16, 3 the format f),
// as the file holds them at src (device memory), stored as type `to`
hipError_t pskd_decode_launch(const void* src, int enc, const PskFormat& f, long long n, void* dst, int to, unsigned* flag,
                              hipStream_t s);
// n elements of an idx leaf of `width` bytes widened to i64
hipError_t pskd_idx_launch(const void* src, int width, long long n, long long* dst, hipStream_t s);

}  // namespace presk
