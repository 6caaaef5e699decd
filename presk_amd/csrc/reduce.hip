// Column reductions in the executor's own chunked order (FAST mode): `sum_to` of a
// tensor onto its trailing axes (a bias's gradient, lower.rs:1670-1680),
// out[c] = sum_r x[r][c]; and `sum_all`/`mean_all` (lower.rs:1221-1233) and
// `sum_squares` (lower.rs:1693-1703, the terms x * x) as the one column of
// all elements, the mean dividing the total once.
//
// The interpreter's order adds the R rows one after another into the output
// (a running sum of R dependent additions per column: latency-bound with one
// thread per column).  This kernel declares an order of its own, in the
// kernel's info as `rows-in-chunks(64)-f32` -- the shape of the reference's
// `ReductionOrder::Chunked { size }` (crates/presk-rt/src/lib.rs:262-268;
// semantics lower.rs:427-464), which a realization applies to contractions
// only, never to these sums: the rows in chunks of CH consecutive ones, each
// chunk summed from zero in row order, the chunk sums then added in chunk
// order from zero -- in f32, and stored once in the storage type (an f32
// accumulation format).  Two launches, deterministic.
#include <hip/hip_runtime.h>

#include "devfmt.hpp"
#include "reduce.hpp"

namespace presk {

namespace {

template <int ST>
__device__ __forceinline__ float ld(const void* p, long long i) {
    if (ST == 0) return ((const float*)p)[i];
    if (ST == 1) return pk_bf16_to_f32(((const unsigned short*)p)[i]);
    return pk_f16_to_f32(((const unsigned short*)p)[i]);
}

// one lane per (chunk, column): the chunk's rows summed in order, all of a
// full chunk's loads in flight before the first add; a term is x, or x * x
// rounded once (`sum_squares`: Product then Accum, lower.rs:1693-1703)
template <int ST>
__device__ __forceinline__ float term(float x, bool square) {
    return square ? x * x : x;
}

template <int ST>
__global__ void __launch_bounds__(64) colsum_chunks(ColSumArgs a) {
    const long long col = (long long)blockIdx.x * 64 + threadIdx.x;
    const long long ch = blockIdx.y;
    if (col >= a.cols) return;
    const long long r0 = ch * a.chunk;
    float part = 0.f;
    if (a.chunk == 64 && r0 + 64 <= a.rows) {
        float v[64];
#pragma unroll
        for (int i = 0; i < 64; ++i) v[i] = ld<ST>(a.x, (r0 + i) * a.ld + col);
#pragma unroll
        for (int i = 0; i < 64; ++i) part = part + term<ST>(v[i], a.square);
    } else {
        long long r1 = r0 + a.chunk;
        if (r1 > a.rows) r1 = a.rows;
        for (long long r = r0; r < r1; ++r) part = part + term<ST>(ld<ST>(a.x, r * a.ld + col), a.square);
    }
    a.work[ch * a.cols + col] = part;
}

// the total of column `col`, divided once for a mean, stored in the storage type
template <int ST>
__device__ __forceinline__ void store_total(const ColSumArgs& a, long long col, float acc) {
    if (a.div != 0.f) acc = acc / a.div;
    if (ST == 0) {
        ((float*)a.out)[col] = acc;
    } else if (ST == 1) {
        ((unsigned short*)a.out)[col] = pk_f32_to_bf16(acc);
    } else {
        if (pk_overflows_f16(acc) && a.flag) atomicOr(a.flag, 1u);
        ((unsigned short*)a.out)[col] = pk_f32_to_f16(acc);
    }
}

// the chunk sums added in chunk order from zero, then one store: sixteen
// waves stage SEG chunk sums of 64 columns in LDS (SEG/16 loads a lane, all
// in flight), lane c of wave 0 adds them in order, reading LDS 32 at a time
// so the chain of adds waits on one LDS round trip per 32
constexpr int SEG = 256, TW = 16, BATCH = 32;

template <int ST>
__global__ void __launch_bounds__(TW * 64) colsum_total(ColSumArgs a) {
    __shared__ float part[SEG][64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long long col = (long long)blockIdx.x * 64 + lane;
    const bool live = col < a.cols;
    float acc = 0.f;
    for (long long c0 = 0; c0 < a.nchunks; c0 += SEG) {
        const int n = (int)(a.nchunks - c0 < SEG ? a.nchunks - c0 : SEG);
        float v[SEG / TW];
#pragma unroll
        for (int i = 0; i < SEG / TW; ++i) {
            const int c = i * TW + w;
            v[i] = live && c < n ? a.work[(c0 + c) * a.cols + col] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < SEG / TW; ++i) part[i * TW + w][lane] = v[i];
        __syncthreads();
        if (w == 0) {
            int c = 0;
            for (; c + BATCH <= n; c += BATCH) {
                float t[BATCH];
#pragma unroll
                for (int i = 0; i < BATCH; ++i) t[i] = part[c + i][lane];
#pragma unroll
                for (int i = 0; i < BATCH; ++i) acc = acc + t[i];
            }
            for (; c < n; ++c) acc = acc + part[c][lane];
        }
        __syncthreads();
    }
    if (w != 0 || !live) return;
    store_total<ST>(a, col, acc);
}

// One column (`sum_all`, `mean_all`, `sum_squares`: every element, chunk c
// the elements 64c .. 64c+63).  A lane sums one chunk in order, its 64
// elements read as 16-byte vectors (256 B of f32 or 128 B of a 16-bit
// type), all in flight before the first add; the wave's lanes read 16 KB
// (f32) contiguous between them, each line fetched once into the cache.
template <int ST>
__global__ void __launch_bounds__(256) total_chunks(ColSumArgs a) {
    const long long ch = (long long)blockIdx.x * 256 + threadIdx.x;
    if (ch >= a.nchunks) return;
    const long long r0 = ch * 64;
    float part = 0.f;
    if (r0 + 64 <= a.rows) {
        constexpr int PER = ST == 0 ? 4 : 8;       // elements a 16-byte vector
        const uint4* p = (const uint4*)((const char*)a.x + r0 * (ST == 0 ? 4 : 2));
        uint4 v[64 / PER];
#pragma unroll
        for (int i = 0; i < 64 / PER; ++i) v[i] = p[i];
#pragma unroll
        for (int i = 0; i < 64 / PER; ++i) {
            const unsigned u[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (ST == 0) {
                    part = part + term<ST>(__uint_as_float(u[j]), a.square);
                } else {
                    const unsigned short lo = (unsigned short)(u[j] & 0xffffu), hi = (unsigned short)(u[j] >> 16);
                    part = part + term<ST>(ST == 1 ? pk_bf16_to_f32(lo) : pk_f16_to_f32(lo), a.square);
                    part = part + term<ST>(ST == 1 ? pk_bf16_to_f32(hi) : pk_f16_to_f32(hi), a.square);
                }
            }
        }
    } else {
        for (long long r = r0; r < a.rows; ++r) part = part + term<ST>(ld<ST>(a.x, r), a.square);
    }
    a.work[ch] = part;
}

// The chunk sums of one column added in chunk order from zero by one wave:
// a segment of SEG1 sums staged in LDS, every lane running the same chain
// of adds over LDS broadcasts read 64 at a time, while the next segment's
// loads are in flight.  The chain (one dependent add a chunk) bounds it.
constexpr int SEG1 = 2048, SEG1_LANE = SEG1 / 256;   // float4s a lane

template <int ST>
__global__ void __launch_bounds__(64) total_sum(ColSumArgs a) {
    __shared__ float4 seg[SEG1 / 4];
    const int lane = threadIdx.x;
    const float4* w4 = (const float4*)a.work;
    const long long n4 = a.nchunks / 4;             // whole float4s of chunk sums
    float4 nxt[SEG1_LANE];
    auto fetch = [&](long long q0) {
#pragma unroll
        for (int i = 0; i < SEG1_LANE; ++i) {
            const long long q = q0 + i * 64 + lane;
            nxt[i] = q < n4 ? w4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    float acc = 0.f;
    fetch(0);
    for (long long c0 = 0; c0 < a.nchunks; c0 += SEG1) {
#pragma unroll
        for (int i = 0; i < SEG1_LANE; ++i) seg[i * 64 + lane] = nxt[i];
        __syncthreads();
        fetch((c0 + SEG1) / 4);
        const int cnt = (int)(a.nchunks - c0 < SEG1 ? a.nchunks - c0 : SEG1);
        const int g4 = cnt / 4;
        int g = 0;
        for (; g + 16 <= g4; g += 16) {
            float4 t[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) t[i] = seg[g + i];
#pragma unroll
            for (int i = 0; i < 16; ++i) acc = ((acc + t[i].x) + t[i].y + t[i].z) + t[i].w;
        }
        for (; g < g4; ++g) {
            const float4 t = seg[g];
            acc = ((acc + t.x) + t.y + t.z) + t.w;
        }
        for (int c = g4 * 4; c < cnt; ++c) acc = acc + a.work[c0 + c];
        __syncthreads();
    }
    if (lane == 0) store_total<ST>(a, 0, acc);
}

}  // namespace

hipError_t colsum_launch(const ColSumArgs& a, hipStream_t stream) {
    if (a.cols == 0) return hipSuccess;
    if (a.cols == 1 && a.chunk == 64 && ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.work & 15) == 0) {
        const unsigned nb = (unsigned)((a.nchunks + 255) / 256);
        switch (a.storage) {
            case 0: total_chunks<0><<<nb, 256, 0, stream>>>(a); break;
            case 1: total_chunks<1><<<nb, 256, 0, stream>>>(a); break;
            case 2: total_chunks<2><<<nb, 256, 0, stream>>>(a); break;
            default: return hipErrorInvalidValue;
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        switch (a.storage) {
            case 0: total_sum<0><<<1, 64, 0, stream>>>(a); break;
            case 1: total_sum<1><<<1, 64, 0, stream>>>(a); break;
            case 2: total_sum<2><<<1, 64, 0, stream>>>(a); break;
        }
        return hipGetLastError();
    }
    if (a.nchunks > 65535) return hipErrorInvalidValue;
    const unsigned bx = (unsigned)((a.cols + 63) / 64);
    dim3 g1(bx, (unsigned)a.nchunks);
    switch (a.storage) {
        case 0: colsum_chunks<0><<<g1, 64, 0, stream>>>(a); break;
        case 1: colsum_chunks<1><<<g1, 64, 0, stream>>>(a); break;
        case 2: colsum_chunks<2><<<g1, 64, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    switch (a.storage) {
        case 0: colsum_total<0><<<bx, TW * 64, 0, stream>>>(a); break;
        case 1: colsum_total<1><<<bx, TW * 64, 0, stream>>>(a); break;
        case 2: colsum_total<2><<<bx, TW * 64, 0, stream>>>(a); break;
    }
    return hipGetLastError();
}

}  // namespace presk
