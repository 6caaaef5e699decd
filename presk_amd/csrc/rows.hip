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
// with the row's max and sum read from the walking lane.  A row of at most
// four chunks is loaded once and kept in registers for all the nest's passes
// (the nest reads the same values each pass); a longer row is read again at
// each pass, as the nest does.
#include <hip/hip_runtime.h>

#include "devfmt.hpp"
#include "rows.hpp"

namespace presk {

namespace {

constexpr int CW = 64;     // columns per chunk, one per lane
constexpr int NRES = 4;    // rows of at most NRES chunks stay in registers for every pass

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

// R rows per wave (one wave per workgroup); RES: the row fits in NRES chunks,
// loaded once and kept in registers across the nest's passes
template <int OP, int ST, int R, bool RES>
__global__ void __launch_bounds__(64) rows_kernel(RowArgs a) {
    constexpr bool MASKED = OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2;
    __shared__ float tile[R][CW + 1];
    const int lane = threadIdx.x;
    const long long row0 = (long long)blockIdx.x * R;
    const long long n = a.n;
    const int nr = (int)(a.rows - row0 < R ? a.rows - row0 : R);  // live rows here
    const bool walker = lane < nr;
    const long long r = row0 + lane;  // the walking lane's row
    const float qnan = __int_as_float(0x7fc00000);
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

    // x[row0 + i][c0 + lane] for every row, and the mask's verdicts as bits
    // (bit i: row i).  Addresses are clamped into the rows and the chunk, so
    // every load is issued unconditionally and all are in flight together;
    // a clamped lane's values are never used.
    auto load = [&](long long c0, int cw, float (&v)[R], unsigned& mb) {
        const long long col = c0 + (lane < cw ? lane : cw - 1);
#pragma unroll
        for (int i = 0; i < R; ++i) v[i] = ld<ST>(a.x, (row0 + (i < nr ? i : nr - 1)) * n + col);
        if (MASKED) {
            const long long* mask = (const long long*)a.mask;
            long long mv[R];
#pragma unroll
            for (int i = 0; i < R; ++i) mv[i] = mask[moff[i] + col];
            unsigned b = 0;
#pragma unroll
            for (int i = 0; i < R; ++i)
                // allowed: real(mask) > 0.5 in the nest's f32
                b |= ((float)(double)mv[i] > 0.5f ? 1u : 0u) << i;
            mb = lane < cw ? b & ((1u << nr) - 1u) : 0u;
        }
    };
    // lane i walks tile row i over columns [0, cw) in order
    auto walk = [&](int cw, auto&& f) {
        __syncthreads();
        if (walker) {
#pragma unroll 8
            for (int j = 0; j < cw; ++j) f(tile[lane][j]);
        }
        __syncthreads();
    };
    // the row's chunks: resident ones loaded once here, others at each pass
    constexpr int NV = RES ? NRES : 1;
    float v[NV][R];
    unsigned mb[NV];
    auto for_chunks = [&](auto&& body) {
        if constexpr (RES) {
#pragma unroll
            for (int ch = 0; ch < NRES; ++ch)
                if (ch * CW < n) body(ch, (long long)ch * CW, (int)(n - ch * CW < CW ? n - ch * CW : CW));
        } else {
            for (long long c0 = 0; c0 < n; c0 += CW) {
                const int cw = (int)(n - c0 < CW ? n - c0 : CW);
                load(c0, cw, v[0], mb[0]);
                body(0, c0, cw);
            }
        }
    };
    if constexpr (RES) {
#pragma unroll
        for (int ch = 0; ch < NRES; ++ch)
            if (ch * CW < n) load(ch * CW, (int)(n - ch * CW < CW ? n - ch * CW : CW), v[ch], mb[ch]);
    }
    auto allowed = [&](int ch, int i) { return MASKED ? ((mb[ch] >> i) & 1u) != 0 : true; };
    // a reduction pass: each element transformed in the coalesced layout
    // (elem may rewrite a resident value), then the chunk walked in order
    auto reduce_pass = [&](auto&& elem, auto&& f) {
        for_chunks([&](int ch, long long, int cw) {
#pragma unroll
            for (int i = 0; i < R; ++i) tile[i][lane] = elem(i, v[ch][i], allowed(ch, i));
            walk(cw, f);
        });
    };
    // a write pass: out[row0 + i][k] = g(i, k, value, allowed), coalesced
    auto write_pass = [&](auto&& g) {
        for_chunks([&](int ch, long long c0, int cw) {
            if (lane < cw) {
#pragma unroll
                for (int i = 0; i < R; ++i)
                    if (i < nr) st<ST>(a.out, (row0 + i) * n + c0 + lane, g(i, c0 + lane, v[ch][i], allowed(ch, i)), ovf);
            }
        });
    };
    auto same = [](int, float& v, bool) { return v; };

    if (OP == kRowMean || OP == kRowSum) {
        float acc = 0.f;
        reduce_pass(same, [&](float x) { acc = acc + x; });
        if (walker) st<ST>(a.out, r, OP == kRowMean ? acc / a.n_real : acc, ovf);
    } else if (OP == kSumToRows) {
        // the running sum lives in the output: every step stored (rounded)
        float acc = 0.f;
        reduce_pass(same, [&](float x) {
            const float s = acc + x;
            if (ST == 2) ovf |= pk_overflows_f16(s);
            acc = stored<ST>(s);
        });
        if (walker) st<ST>(a.out, r, acc, ovf);
    } else {
        if (n == 0) return;
        float m;
        if (!MASKED) {
            // m = x[0]; then m = x[k] wherever x[k] > m
            m = walker ? ld<ST>(a.x, r * n) : 0.f;
            reduce_pass(same, [&](float x) { m = x > m ? x : m; });
        } else {
            // The nest's masked max: the first allowed element, then any
            // later allowed one greater than the running max.  Walked as the
            // plain max from -inf over the allowed elements (a disallowed one
            // walks as NaN, which is never greater), which agrees except when
            // the first allowed element is NaN (the nest's max is then NaN)
            // or none is allowed (the nest's max stays 0): both found here by
            // ballots over the chunks in order.
            unsigned found = 0, nanfirst = 0;  // bit i: row i
            m = -__builtin_inff();
            reduce_pass([&](int i, float& x, bool al) {
                const unsigned long long A = __ballot(al), N = __ballot(al && x != x);
                if (!((found >> i) & 1u) && A) {
                    found |= 1u << i;
                    if (N & (A & (~A + 1ull))) nanfirst |= 1u << i;
                }
                return al ? x : qnan;
            }, [&](float x) { m = x > m ? x : m; });
            m = ((nanfirst >> lane) & 1u) ? qnan : ((found >> lane) & 1u) ? m : 0.f;
        }
        float mi[R];
#pragma unroll
        for (int i = 0; i < R; ++i) mi[i] = from_lane(m, i);
        // the exponentials: a resident row keeps them for the write pass (the
        // nest computes the same exp(x - m) there)
        float z = 0.f;
        reduce_pass([&](int i, float& x, bool al) {
            const float e = al ? pk_expf(x - mi[i]) : 0.f;
            if (RES) x = e;
            return e;
        }, [&](float e) { z = z + e; });
        auto expo = [&](int i, float x, bool al) -> float {
            if (RES) return x;
            return al ? pk_expf(x - mi[i]) : 0.f;
        };
        float zi[R];
#pragma unroll
        for (int i = 0; i < R; ++i) zi[i] = from_lane(z, i);
        if (OP == kSoftmax3 || OP == kMaskedSoftmax3) {
            write_pass([&](int i, long long, float x, bool al) { return al ? expo(i, x, al) / zi[i] : 0.f; });
        } else if (OP == kSoftmax2 || OP == kMaskedSoftmax2) {
            // the stored exponential over z (the first pass's stores of e,
            // guarded, are overwritten)
            write_pass([&](int i, long long, float x, bool al) {
                const float e = expo(i, x, al);
                if (ST == 2) ovf |= pk_overflows_f16(e);
                return al ? stored<ST>(e) / zi[i] : 0.f;
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
            write_pass([&](int i, long long k, float x, bool al) {
                const float sm = expo(i, x, al) / zi[i];
                const float onehot = (float)(double)k == fyi[i] ? 1.f : 0.f;
                return (sm - onehot) * cti[i];
            });
        }
    }
    if (ovf && a.flag) atomicOr(a.flag, 1u);
}

// A few long rows (a total, `mean_all`, or rows too few to give each lane
// its own): one workgroup per row stages the row through LDS 4096 elements at
// a time, the next stage's loads issued before the current one is walked,
// and one lane adds the stage in index order.
constexpr int LSTAGE = 4096;

template <int OP, int ST>
__global__ void __launch_bounds__(256) rows_long_kernel(RowArgs a) {
    __shared__ __attribute__((aligned(16))) float buf[2][LSTAGE];
    constexpr int PER = LSTAGE / 256;
    const int t = threadIdx.x;
    const long long n = a.n, base = (long long)blockIdx.x * n;
    float acc = 0.f;
    bool ovf = false;
    float nx[PER];
    auto fetch = [&](long long c0) {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const long long c = c0 + j * 256 + t;
            nx[j] = c < n ? ld<ST>(a.x, base + c) : 0.f;
        }
    };
    auto put = [&](int s) {
#pragma unroll
        for (int j = 0; j < PER; ++j) buf[s][j * 256 + t] = nx[j];
    };
    fetch(0);
    put(0);
    __syncthreads();
    int s = 0;
    for (long long c0 = 0; c0 < n; c0 += LSTAGE, s ^= 1) {
        const bool more = c0 + LSTAGE < n;
        if (more) fetch(c0 + LSTAGE);
        if (t == 0) {
            const int cw = (int)(n - c0 < LSTAGE ? n - c0 : LSTAGE);
            int j = 0;
            for (; j + 4 <= cw; j += 4) {
                const float4 q = *(const float4*)&buf[s][j];
                const float e[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (OP == kSumToRows) {
                        const float y = acc + e[u];
                        if (ST == 2) ovf |= pk_overflows_f16(y);
                        acc = stored<ST>(y);
                    } else {
                        acc = acc + e[u];
                    }
                }
            }
            for (; j < cw; ++j) {
                if (OP == kSumToRows) {
                    const float y = acc + buf[s][j];
                    if (ST == 2) ovf |= pk_overflows_f16(y);
                    acc = stored<ST>(y);
                } else {
                    acc = acc + buf[s][j];
                }
            }
        }
        if (more) put(s ^ 1);  // the other buffer was walked last round
        __syncthreads();
    }
    if (t == 0) st<ST>(a.out, blockIdx.x, OP == kRowMean ? acc / a.n_real : acc, ovf);
    if (ovf && a.flag) atomicOr(a.flag, 1u);
}

template <int OP>
hipError_t launch_long(const RowArgs& a, hipStream_t stream) {
    switch (a.storage) {
        case 0: rows_long_kernel<OP, 0><<<(unsigned)a.rows, 256, 0, stream>>>(a); break;
        case 1: rows_long_kernel<OP, 1><<<(unsigned)a.rows, 256, 0, stream>>>(a); break;
        case 2: rows_long_kernel<OP, 2><<<(unsigned)a.rows, 256, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int OP, int R, bool RES>
hipError_t launch_r(const RowArgs& a, hipStream_t stream) {
    const unsigned grid = (unsigned)((a.rows + R - 1) / R);
    switch (a.storage) {
        case 0: rows_kernel<OP, 0, R, RES><<<grid, 64, 0, stream>>>(a); break;
        case 1: rows_kernel<OP, 1, R, RES><<<grid, 64, 0, stream>>>(a); break;
        case 2: rows_kernel<OP, 2, R, RES><<<grid, 64, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Rows per wave: a walk costs the same issue slots however many of its
// lanes are live, so 16 rows a wave -- unless that leaves fewer waves than
// SIMDs (under 8192 rows), when 4 rows a wave spreads the walks wider.
template <int OP>
hipError_t launch_op(const RowArgs& a, hipStream_t stream) {
    if (a.rows == 0) return hipSuccess;
    if constexpr (OP == kRowMean || OP == kRowSum || OP == kSumToRows) {
        // rows too few for a lane each and long enough to stage
        if (a.rows < 1024 && a.n >= 1024) return launch_long<OP>(a, stream);
    }
    if ((OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2) && a.mask_rows <= 0) return hipErrorInvalidValue;
    if ((a.rows + 3) / 4 > 0x7fffffffll) return hipErrorInvalidValue;
    const bool res = a.n <= NRES * CW;
    if (a.rows >= 8192)
        return res ? launch_r<OP, 16, true>(a, stream) : launch_r<OP, 16, false>(a, stream);
    return res ? launch_r<OP, 4, true>(a, stream) : launch_r<OP, 4, false>(a, stream);
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
