// The measured MFMA peak: loops of independent MFMAs, eight waves a CU (two
// a SIMD), each wave keeping eight accumulators in flight, nothing else
// issued -- the rate the matrix cores reach on this device at the clock they
// run under that load, reported beside the vendor's nominal figure.
// bf16: v_mfma_f32_32x32x16_bf16 (32 768 flops a wave instruction); f32:
// v_mfma_f32_16x16x4_f32 (2 048).
#include <hip/hip_runtime.h>

#include "probe.hpp"

namespace presk {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWaves = 8, kAcc = 8, kSink = 4096;

// `sink`: one word a workgroup in device memory, written only when the sums
// take a value they cannot take (they are sums of nonnegative products), so
// that the compiler keeps the loops
template <int KIND>
__global__ void __launch_bounds__(64 * kWaves) mfma_probe_kernel(long long iters, float* sink) {
    float r = 0.f;
    if constexpr (KIND == 0) {
        bf16x8 a, b;
        for (int j = 0; j < 8; ++j) {
            a[j] = (__bf16)(float)((threadIdx.x + j) & 7);
            b[j] = (__bf16)(float)((threadIdx.x * 3 + j) & 7);
        }
        f32x16 acc[kAcc];
        for (int i = 0; i < kAcc; ++i) acc[i] = f32x16{};
        for (long long it = 0; it < iters; ++it) {
#pragma unroll
            for (int i = 0; i < kAcc; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[i], 0, 0, 0);
        }
        for (int i = 0; i < kAcc; ++i) r += acc[i][0];
    } else {
        const float a = (float)(threadIdx.x & 7), b = (float)((threadIdx.x * 3) & 7);
        f32x4 acc[kAcc];
        for (int i = 0; i < kAcc; ++i) acc[i] = f32x4{};
        for (long long it = 0; it < iters; ++it) {
#pragma unroll
            for (int i = 0; i < kAcc; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[i], 0, 0, 0);
        }
        for (int i = 0; i < kAcc; ++i) r += acc[i][0];
    }
    if (r == -1.0f && blockIdx.x < kSink) sink[blockIdx.x] = r;
}

}  // namespace

hipError_t mfma_probe(int kind, long long iters, hipStream_t stream, double* ms, double* flops) {
    if ((kind != 0 && kind != 1) || iters <= 0) return hipErrorInvalidValue;
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    if (cus <= 0 || cus > kSink) return hipErrorInvalidValue;
    float* sink = nullptr;
    e = hipMalloc(&sink, kSink * sizeof(float));
    if (e != hipSuccess) return e;
    auto launch = [&]() {
        if (kind == 0) mfma_probe_kernel<0><<<cus, 64 * kWaves, 0, stream>>>(iters, sink);
        else mfma_probe_kernel<1><<<cus, 64 * kWaves, 0, stream>>>(iters, sink);
        return hipGetLastError();
    };
    hipEvent_t a = nullptr, b = nullptr;
    e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    if (e == hipSuccess) e = launch();                       // untimed: the clock rises under the load
    if (e == hipSuccess) e = hipEventRecord(a, stream);
    if (e == hipSuccess) e = launch();
    if (e == hipSuccess) e = hipEventRecord(b, stream);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    float t = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&t, a, b);
    if (a) hipEventDestroy(a);
    if (b) hipEventDestroy(b);
    hipFree(sink);   // after the synchronized launches
    if (e != hipSuccess) return e;
    *ms = t;
    *flops = (double)cus * kWaves * kAcc * (double)iters * (kind == 0 ? 2.0 * 32 * 32 * 16 : 2.0 * 16 * 16 * 4);
    return hipSuccess;
}

}  // namespace presk
