// Row nests in the interpreter's own order (EXACT in both modes): the
// softmax over the last axis in three passes, in two, and masked
// (crates/presk-kernel/src/lower.rs:1274-1419), `mean`/`sum` over the last
// axis (lower.rs:1239-1255), `sum_to` onto leading axes (lower.rs:1670-1680),
// `cross_entropy` and `cross_entropy_vjp` (lower.rs:1459-1488).
//
// Only the running reductions of these nests (a sum, a max) have an order;
// everything elementwise (the exponentials, the divisions, the mask tests,
// the stores) does not.  So one wave owns R rows and works in chunks of 64
// columns: lane j loads column c0 + j of every row (R coalesced loads in
// flight), computes the elementwise part in that layout, and for a reduction
// parks the chunk in LDS, where lane i walks row i in index order -- the
// interpreter's sequential sum, bit for bit.  Passes that only write (the
// last pass of a softmax, the vjp) stay in the coalesced layout throughout,
// with the row's max and sum read from the walking lane.  Each pass of the
// nest over its row reads the row again, as the nest does.
#include <hip/hip_runtime.h>

#include "devfmt.hpp"
#include "rows.hpp"

namespace presk {

namespace {

constexpr int R = 16;   // rows per wave (one wave per workgroup)
constexpr int CW = 64;  // columns per chunk, one per lane

template <int ST>
__device__ __forceinline__ float ld(const void* p, long long i) {
    if (ST == 0) return ((const float*)p)[i];
    if (ST == 1) return pk_bf16_to_f32(((const unsigned short*)p)[i]);
    return pk_f16_to_f32(((const unsigned short*)p)[i]);
}

// A store of v to element i, rounded to the storage type, under the guard.
template <int ST>
__device__ __forceinline__ void st(void* p, long long i, float v, bool& ovf) {
    if (ST == 0) {
        ((float*)p)[i] = v;
    } else if (ST == 1) {
        ((unsigned short*)p)[i] = pk_f32_to_bf16(v);
    } else {
        ovf |= pk_overflows_f16(v);
        ((unsigned short*)p)[i] = pk_f32_to_f16(v);
    }
}

// The value a store of v leaves in memory, as a load reads it back.
template <int ST>
__device__ __forceinline__ float stored(float v) {
    if (ST == 0) return v;
    if (ST == 1) return pk_bf16_to_f32(pk_f32_to_bf16(v));
    return pk_f16_to_f32(pk_f32_to_f16(v));
}

// lane i's value, in every lane
__device__ __forceinline__ float from_lane(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

template <int OP, int ST>
__global__ void __launch_bounds__(64) rows_kernel(RowArgs a) {
    constexpr bool MASKED = OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2;
    __shared__ float tile[R][CW + 1];
    __shared__ unsigned char mtile[MASKED ? R : 1][MASKED ? CW + 4 : 1];
    const int lane = threadIdx.x;
    const long long row0 = (long long)blockIdx.x * R;
    const long long n = a.n;
    const int nr = (int)(a.rows - row0 < R ? a.rows - row0 : R);  // live rows here
    const bool walker = lane < nr;
    const long long r = row0 + lane;  // the walking lane's row
    bool ovf = false;

    // the mask row of each of the R rows (the mask repeats over leading axes)
    long long moff[MASKED ? R : 1];
    if (MASKED) {
        long long mr = row0 % a.mask_rows;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            moff[i] = mr * n;
            mr = mr + 1 == a.mask_rows ? 0 : mr + 1;
        }
    }

    // x[row0 + i][c0 + lane] for every row, and whether the mask allows it
    auto load = [&](long long c0, int cw, float (&v)[R], bool (&al)[R]) {
        const bool col = lane < cw;
#pragma unroll
        for (int i = 0; i < R; ++i) v[i] = col && i < nr ? ld<ST>(a.x, (row0 + i) * n + c0 + lane) : 0.f;
        if (MASKED) {
            const long long* mask = (const long long*)a.mask;
#pragma unroll
            for (int i = 0; i < R; ++i)
                // allowed: real(mask) > 0.5 in the nest's f32
                al[i] = col && i < nr ? (float)(double)mask[moff[i] + c0 + lane] > 0.5f : false;
        }
    };
    // lane i walks tile row i over columns [0, cw) in order
    auto walk = [&](int cw, auto&& f) {
        __syncthreads();
        if (walker)
            for (int j = 0; j < cw; ++j) f(tile[lane][j], MASKED ? mtile[lane][j] != 0 : true);
        __syncthreads();
    };
    // a reduction pass: the chunk transformed elementwise, then walked
    auto reduce_pass = [&](auto&& elem, auto&& f) {
        for (long long c0 = 0; c0 < n; c0 += CW) {
            const int cw = (int)(n - c0 < CW ? n - c0 : CW);
            float v[R];
            bool al[R];
            load(c0, cw, v, al);
#pragma unroll
            for (int i = 0; i < R; ++i) {
                tile[i][lane] = elem(i, v[i], al[i]);
                if (MASKED) mtile[i][lane] = al[i] ? 1 : 0;
            }
            walk(cw, f);
        }
    };
    // a write pass: out[row0 + i][k] = g(i, k, value, allowed), coalesced
    auto write_pass = [&](auto&& g) {
        for (long long c0 = 0; c0 < n; c0 += CW) {
            const int cw = (int)(n - c0 < CW ? n - c0 : CW);
            float v[R];
            bool al[R];
            load(c0, cw, v, al);
            if (lane < cw) {
#pragma unroll
                for (int i = 0; i < R; ++i)
                    if (i < nr) st<ST>(a.out, (row0 + i) * n + c0 + lane, g(i, c0 + lane, v[i], al[i]), ovf);
            }
        }
    };
    auto same = [](int, float v, bool) { return v; };

    if (OP == kRowMean || OP == kRowSum) {
        float acc = 0.f;
        reduce_pass(same, [&](float v, bool) { acc = acc + v; });
        if (walker) st<ST>(a.out, r, OP == kRowMean ? acc / a.n_real : acc, ovf);
    } else if (OP == kSumToRows) {
        // the running sum lives in the output: every step stored (rounded)
        float acc = 0.f;
        reduce_pass(same, [&](float v, bool) {
            const float s = acc + v;
            if (ST == 2) ovf |= pk_overflows_f16(s);
            acc = stored<ST>(s);
        });
        if (walker) st<ST>(a.out, r, acc, ovf);
    } else if (OP == kSoftmax3 || OP == kSoftmax2 || OP == kCrossEntropy || OP == kCrossEntropyVjp) {
        if (n == 0) return;
        float m = walker ? ld<ST>(a.x, r * n) : 0.f;
        reduce_pass(same, [&](float v, bool) { if (v > m) m = v; });
        float mi[R];
#pragma unroll
        for (int i = 0; i < R; ++i) mi[i] = from_lane(m, i);
        float z = 0.f;
        reduce_pass([&](int i, float v, bool) { return pk_expf(v - mi[i]); }, [&](float e, bool) { z = z + e; });
        float zi[R];
#pragma unroll
        for (int i = 0; i < R; ++i) zi[i] = from_lane(z, i);
        if (OP == kSoftmax3) {
            write_pass([&](int i, long long, float v, bool) { return pk_expf(v - mi[i]) / zi[i]; });
        } else if (OP == kSoftmax2) {
            // the stored exponential over z (the first pass's stores are overwritten)
            write_pass([&](int i, long long, float v, bool) {
                const float e = pk_expf(v - mi[i]);
                if (ST == 2) ovf |= pk_overflows_f16(e);
                return stored<ST>(e) / zi[i];
            });
        } else if (OP == kCrossEntropy) {
            if (walker) {
                const long long y = ((const long long*)a.y)[r];
                st<ST>(a.out, r, (pk_logf(z) + m) - ld<ST>(a.x, r * n + y), ovf);
            }
        } else {
            const float ct = walker ? ld<ST>(a.ct, r) : 0.f;
            const float fy = walker ? (float)(double)((const long long*)a.y)[r] : 0.f;
            float cti[R], fyi[R];
#pragma unroll
            for (int i = 0; i < R; ++i) {
                cti[i] = from_lane(ct, i);
                fyi[i] = from_lane(fy, i);
            }
            write_pass([&](int i, long long k, float v, bool) {
                const float sm = pk_expf(v - mi[i]) / zi[i];
                const float onehot = (float)(double)k == fyi[i] ? 1.f : 0.f;
                return (sm - onehot) * cti[i];
            });
        }
    } else if (MASKED) {
        if (n == 0) return;
        float first = 1.f, mx = 0.f;
        reduce_pass(same, [&](float v, bool al) {
            mx = al ? (first > 0.5f ? v : (v > mx ? v : mx)) : mx;
            first = al ? 0.f : first;
        });
        float mi[R];
#pragma unroll
        for (int i = 0; i < R; ++i) mi[i] = from_lane(mx, i);
        float z = 0.f;
        reduce_pass([&](int i, float v, bool al) { return al ? pk_expf(v - mi[i]) : 0.f; },
                    [&](float e, bool) { z = z + e; });
        float zi[R];
#pragma unroll
        for (int i = 0; i < R; ++i) zi[i] = from_lane(z, i);
        if (OP == kMaskedSoftmax3) {
            write_pass([&](int i, long long, float v, bool al) { return al ? pk_expf(v - mi[i]) / zi[i] : 0.f; });
        } else {
            write_pass([&](int i, long long, float v, bool al) {
                const float e = al ? pk_expf(v - mi[i]) : 0.f;
                if (ST == 2) ovf |= pk_overflows_f16(e);
                return al ? stored<ST>(e) / zi[i] : 0.f;
            });
        }
    }
    if (ovf && a.flag) atomicOr(a.flag, 1u);
}

template <int OP>
hipError_t launch_op(const RowArgs& a, hipStream_t stream) {
    if (a.rows == 0) return hipSuccess;
    if ((OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2) && a.mask_rows <= 0) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)((a.rows + R - 1) / R);
    switch (a.storage) {
        case 0: rows_kernel<OP, 0><<<grid, 64, 0, stream>>>(a); break;
        case 1: rows_kernel<OP, 1><<<grid, 64, 0, stream>>>(a); break;
        case 2: rows_kernel<OP, 2><<<grid, 64, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t rows_launch(const RowArgs& a, hipStream_t stream) {
    switch (a.op) {
        case kRowMean: return launch_op<kRowMean>(a, stream);
        case kRowSum: return launch_op<kRowSum>(a, stream);
        case kSumToRows: return launch_op<kSumToRows>(a, stream);
        case kSoftmax3: return launch_op<kSoftmax3>(a, stream);
        case kSoftmax2: return launch_op<kSoftmax2>(a, stream);
        case kMaskedSoftmax3: return launch_op<kMaskedSoftmax3>(a, stream);
        case kMaskedSoftmax2: return launch_op<kMaskedSoftmax2>(a, stream);
        case kCrossEntropy: return launch_op<kCrossEntropy>(a, stream);
        case kCrossEntropyVjp: return launch_op<kCrossEntropyVjp>(a, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace presk
