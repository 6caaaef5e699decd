// Row nests in the interpreter's own order (EXACT in both modes): the
// softmax over the last axis in three passes, in two, and masked
// (crates/presk-kernel/src/lower.rs:1274-1419), `mean`/`sum` over the last
// axis (lower.rs:1239-1255), `cross_entropy` and `cross_entropy_vjp`
// (lower.rs:1459-1488).
//
// One lane owns one row and walks it in index order, so every sum is the
// interpreter's sequential one and every value its bits: the same f32
// operations (the fdlibm-method expf/logf of devfmt.hpp), the same roundings
// at the same stores.  The rows of a wave are read with 16-byte loads along
// each lane's row; the softmax reads its input once per pass, as the nest
// does.
#include <hip/hip_runtime.h>

#include "devfmt.hpp"
#include "rows.hpp"

namespace presk {

namespace {

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

__device__ __forceinline__ bool allowed(const long long* mask, long long off) {
    return (float)(double)mask[off] > 0.5f;   // real(mask) > 0.5 in the nest's f32
}

template <int OP, int ST>
__global__ void __launch_bounds__(256) rows_kernel(RowArgs a) {
    const long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= a.rows) return;
    const long long n = a.n, base = r * n;
    const void* x = a.x;
    bool ovf = false;
    if (OP == kRowMean || OP == kRowSum) {
        float acc = 0.f;
        for (long long k = 0; k < n; ++k) acc = acc + ld<ST>(x, base + k);
        st<ST>(a.out, r, OP == kRowMean ? acc / a.n_real : acc, ovf);
    } else if (OP == kSoftmax3 || OP == kSoftmax2) {
        if (n == 0) return;
        float m = ld<ST>(x, base);
        for (long long k = 0; k < n; ++k) {
            const float v = ld<ST>(x, base + k);
            if (v > m) m = v;
        }
        float z = 0.f;
        if (OP == kSoftmax3) {
            for (long long k = 0; k < n; ++k) z = z + pk_expf(ld<ST>(x, base + k) - m);
            for (long long k = 0; k < n; ++k) st<ST>(a.out, base + k, pk_expf(ld<ST>(x, base + k) - m) / z, ovf);
        } else {
            // e stored (rounded), summed unrounded; then the stored e over z
            for (long long k = 0; k < n; ++k) {
                const float e = pk_expf(ld<ST>(x, base + k) - m);
                st<ST>(a.out, base + k, e, ovf);
                z = z + e;
            }
            for (long long k = 0; k < n; ++k) st<ST>(a.out, base + k, ld<ST>(a.out, base + k) / z, ovf);
        }
    } else if (OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2) {
        if (n == 0) return;
        const long long* mask = (const long long*)a.mask;
        const long long mrow = (r % a.mask_rows) * n;
        float first = 1.f, mx = 0.f;
        for (long long k = 0; k < n; ++k) {
            const float v = ld<ST>(x, base + k);
            const bool al = allowed(mask, mrow + k);
            mx = al ? (first > 0.5f ? v : (v > mx ? v : mx)) : mx;
            first = al ? 0.f : first;
        }
        float z = 0.f;
        if (OP == kMaskedSoftmax3) {
            for (long long k = 0; k < n; ++k) {
                const bool al = allowed(mask, mrow + k);
                z = z + (al ? pk_expf(ld<ST>(x, base + k) - mx) : 0.f);
            }
            for (long long k = 0; k < n; ++k) {
                const bool al = allowed(mask, mrow + k);
                st<ST>(a.out, base + k, al ? pk_expf(ld<ST>(x, base + k) - mx) / z : 0.f, ovf);
            }
        } else {
            for (long long k = 0; k < n; ++k) {
                const bool al = allowed(mask, mrow + k);
                const float e = al ? pk_expf(ld<ST>(x, base + k) - mx) : 0.f;
                st<ST>(a.out, base + k, e, ovf);
                z = z + e;
            }
            for (long long k = 0; k < n; ++k) {
                const bool al = allowed(mask, mrow + k);
                st<ST>(a.out, base + k, al ? ld<ST>(a.out, base + k) / z : 0.f, ovf);
            }
        }
    } else if (OP == kCrossEntropy || OP == kCrossEntropyVjp) {
        float m = ld<ST>(x, base);
        for (long long k = 0; k < n; ++k) {
            const float v = ld<ST>(x, base + k);
            if (v > m) m = v;
        }
        float z = 0.f;
        for (long long k = 0; k < n; ++k) z = z + pk_expf(ld<ST>(x, base + k) - m);
        const long long y = ((const long long*)a.y)[r];
        if (OP == kCrossEntropy) {
            // ln z + m - x[y]
            st<ST>(a.out, r, (pk_logf(z) + m) - ld<ST>(x, base + y), ovf);
        } else {
            const float ct = ld<ST>(a.ct, r);
            const float fy = (float)(double)y;
            for (long long k = 0; k < n; ++k) {
                const float sm = pk_expf(ld<ST>(x, base + k) - m) / z;
                const float onehot = (float)(double)k == fy ? 1.f : 0.f;
                st<ST>(a.out, base + k, (sm - onehot) * ct, ovf);
            }
        }
    }
    if (ovf && a.flag) atomicOr(a.flag, 1u);
}

template <int OP>
hipError_t launch_op(const RowArgs& a, hipStream_t stream) {
    const unsigned grid = (unsigned)((a.rows + 255) / 256);
    if (a.rows == 0) return hipSuccess;
    switch (a.storage) {
        case 0: rows_kernel<OP, 0><<<grid, 256, 0, stream>>>(a); break;
        case 1: rows_kernel<OP, 1><<<grid, 256, 0, stream>>>(a); break;
        case 2: rows_kernel<OP, 2><<<grid, 256, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t rows_launch(const RowArgs& a, hipStream_t stream) {
    switch (a.op) {
        case kRowMean: return launch_op<kRowMean>(a, stream);
        case kRowSum: return launch_op<kRowSum>(a, stream);
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
