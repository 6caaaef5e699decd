// Seeded synthetic parameters generated where they are used: a model whose
// weights fill a good part of HBM (config 5's 13.5 GB of bf16) is
// initialized in place rather than drawn on the host and copied.
//
// Element i of a fill with seed s: h = mix(s, i) (two rounds of the
// splitmix64 finalizer over s + (i + 1) * 0x9E3779B97F4A7C15); u1 = the top
// 24 bits of h plus one, times 2^-24, in (0, 1]; u2 = the next 24 bits times
// 2^-24, in [0, 1); z = sqrt(-2 ln u1) * cos(2 pi u2) (Box-Muller, one of the
// pair), evaluated in f32 with the device's restated logf and cosf; the
// stored value mean + std * z rounded once to the storage type.  The draw is
// a function of (seed, i) alone, so any launch shape gives the same bits.
#include "synth.hpp"

#include "devfmt.hpp"

namespace presk {
namespace {

__device__ __forceinline__ unsigned long long mix64(unsigned long long z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float draw(unsigned long long seed, unsigned long long i, float mean, float std) {
    const unsigned long long h = mix64(mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ull));
    const float u1 = (float)((h >> 40) + 1) * 5.9604644775390625e-8f;            // (0, 1]
    const float u2 = (float)((h >> 16) & 0xffffffull) * 5.9604644775390625e-8f;   // [0, 1)
    const float r = __builtin_sqrtf(-2.0f * pk_logf(u1));
    const float z = r * pk_cosf(6.28318530717958647692f * u2);
    return mean + std * z;
}

template <int T>
__global__ void __launch_bounds__(256) synth_kernel(void* dst, long long n, unsigned long long seed, float mean,
                                                    float std) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float v = draw(seed, (unsigned long long)i, mean, std);
        if (T == 1) ((float*)dst)[i] = v;
        else if (T == 2) ((unsigned short*)dst)[i] = pk_f32_to_bf16(v);
        else ((unsigned short*)dst)[i] = pk_f32_to_f16(v);
    }
}

}  // namespace

hipError_t synth_normal_launch(void* dst, int type, long long n, unsigned long long seed, float mean, float std,
                               hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const long long blocks = (n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192;
    const dim3 grid((unsigned)blocks), block(256);
    switch (type) {
        case 1: synth_kernel<1><<<grid, block, 0, s>>>(dst, n, seed, mean, std); break;
        case 2: synth_kernel<2><<<grid, block, 0, s>>>(dst, n, seed, mean, std); break;
        case 4: synth_kernel<4><<<grid, block, 0, s>>>(dst, n, seed, mean, std); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace presk
