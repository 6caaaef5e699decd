// Column reductions in a declared chunked order (FAST mode): `sum_to` of a
// tensor onto its trailing axes (a bias's gradient, lower.rs:1670-1680),
// out[c] = sum_r x[r][c].
//
// The interpreter's order adds the R rows one after another into the output
// (a running sum of R dependent additions per column: latency-bound with one
// thread per column).  This kernel uses the reference's declared order
// `ReductionOrder::Chunked { size }` (crates/presk-rt/src/lib.rs:262-268;
// semantics lower.rs:427-464): the rows in chunks of CH consecutive ones, each
// chunk summed from zero in row order, the chunk sums then added in chunk
// order from zero -- in f32, and stored once in the storage type (an f32
// accumulation format).  Two launches, deterministic.
#include <hip/hip_runtime.h>

#include "devfmt.hpp"
#include "reduce.hpp"

namespace presk {

namespace {

template <typename S>
__device__ __forceinline__ float widen(const S* p, long long i);
template <>
__device__ __forceinline__ float widen<float>(const float* p, long long i) { return p[i]; }
template <>
__device__ __forceinline__ float widen<unsigned short>(const unsigned short* p, long long i) { return pk_bf16_to_f32(p[i]); }

// one thread per (chunk, column): the chunk's rows summed in order
template <int ST>
__global__ void __launch_bounds__(256) colsum_chunks(ColSumArgs a) {
    const long long col = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long ch = blockIdx.y;
    if (col >= a.cols) return;
    const long long r0 = ch * a.chunk;
    long long r1 = r0 + a.chunk;
    if (r1 > a.rows) r1 = a.rows;
    float part = 0.f;
    if (ST == 0) {
        const float* x = (const float*)a.x;
#pragma unroll 8
        for (long long r = r0; r < r1; ++r) part = part + x[r * a.cols + col];
    } else if (ST == 1) {
        const unsigned short* x = (const unsigned short*)a.x;
#pragma unroll 8
        for (long long r = r0; r < r1; ++r) part = part + pk_bf16_to_f32(x[r * a.cols + col]);
    } else {
        const unsigned short* x = (const unsigned short*)a.x;
#pragma unroll 8
        for (long long r = r0; r < r1; ++r) part = part + pk_f16_to_f32(x[r * a.cols + col]);
    }
    a.work[ch * a.cols + col] = part;
}

// the chunk sums added in chunk order from zero, then one store
template <int ST>
__global__ void __launch_bounds__(256) colsum_total(ColSumArgs a) {
    const long long col = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (col >= a.cols) return;
    float acc = 0.f;
    for (long long ch = 0; ch < a.nchunks; ++ch) acc = acc + a.work[ch * a.cols + col];
    if (ST == 0) {
        ((float*)a.out)[col] = acc;
    } else if (ST == 1) {
        ((unsigned short*)a.out)[col] = pk_f32_to_bf16(acc);
    } else {
        if (pk_overflows_f16(acc) && a.flag) atomicOr(a.flag, 1u);
        ((unsigned short*)a.out)[col] = pk_f32_to_f16(acc);
    }
}

}  // namespace

hipError_t colsum_launch(const ColSumArgs& a, hipStream_t stream) {
    const unsigned bx = (unsigned)((a.cols + 255) / 256);
    dim3 g1(bx, (unsigned)a.nchunks);
    switch (a.storage) {
        case 0: colsum_chunks<0><<<g1, 256, 0, stream>>>(a); break;
        case 1: colsum_chunks<1><<<g1, 256, 0, stream>>>(a); break;
        case 2: colsum_chunks<2><<<g1, 256, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    switch (a.storage) {
        case 0: colsum_total<0><<<bx, 256, 0, stream>>>(a); break;
        case 1: colsum_total<1><<<bx, 256, 0, stream>>>(a); break;
        case 2: colsum_total<2><<<bx, 256, 0, stream>>>(a); break;
    }
    return hipGetLastError();
}

}  // namespace presk
