// FAST mode's row nests: `mean`/`sum` over the last axis, `sum_to` onto
// leading axes, the softmax (three passes, two, masked), `cross_entropy` and
// its vjp -- the nests of rows.hip, with every running sum in a declared
// order of the executor's own and the exponentials by pk_expf_fast.
//
// One wave owns a row.  The row is cut into blocks of VEC elements (one
// 16-byte load: 4 f32 or 8 bf16/f16; 8 bytes, 4 bf16/f16, for 16-bit rows
// of at most 256; VEC 1 where rows are not whole vectors), block b held by
// lane b mod 64; the cross-lane steps are register moves (DPP and gfx950's
// lane swaps), not LDS round trips.  The order of a sum,
// `lanes64-tree`: each lane adds its own elements in index order (block by
// block, element by element, from zero), then the 64 lane sums are added by
// a balanced pairwise tree over the lane index ((s0 + s1) + (s2 + s3)) + ...,
// whose result every lane holds.  Maxima have no order.  Every element the
// nest computes is otherwise computed as the nest does (f32 arithmetic, the
// stores rounded once, under the guard), except that exp is pk_expf_fast
// and a division by the row's sum z is q0 = e y with y the reciprocal of z
// refined once, corrected by Markstein's step (q0 + y (e - z q0)).
//
// The row stays in registers (at most 64 x 16 VEC elements); longer rows are
// left to rows.hip.  A masked softmax reads the mask packed to bits (the
// workspace rows.hip packs) and skips the loads of blocks its row does not
// allow (their outputs are zeros): a causal mask's upper triangle is never
// read.
#include <hip/hip_runtime.h>

#include "devfmt.hpp"
#include "rows.hpp"

namespace presk {

namespace {

constexpr int WAVES = 4;   // rows (waves) a workgroup

template <int ST>
__device__ __forceinline__ float ld1(const void* p, long long i) {
    if (ST == 0) return ((const float*)p)[i];
    if (ST == 1) return pk_bf16_to_f32(((const unsigned short*)p)[i]);
    return pk_f16_to_f32(((const unsigned short*)p)[i]);
}

template <int ST>
__device__ __forceinline__ unsigned short narrow16(float v, bool& ovf) {
    if (ST == 1) return pk_f32_to_bf16(v);
    ovf |= pk_overflows_f16(v);
    return pk_f32_to_f16(v);
}

template <int ST>
__device__ __forceinline__ float stored(float v) {
    if (ST == 0) return v;
    if (ST == 1) return pk_bf16_to_f32(pk_f32_to_bf16(v));
    return pk_f16_to_f32(pk_f32_to_f16(v));
}

// VEC elements from element e (e a multiple of VEC; VEC elements aligned
// to their size when VEC > 1: 16 bytes, or 8 for 16-bit rows in blocks of 4)
template <int ST, int VEC>
__device__ __forceinline__ void ldv(const void* p, long long e, float (&v)[VEC]) {
    if constexpr (VEC == 1) {
        v[0] = ld1<ST>(p, e);
    } else if constexpr (ST == 0) {
        const float4 q = *(const float4*)((const float*)p + e);
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
    } else if constexpr (VEC == 4) {
        const uint2 q = *(const uint2*)((const unsigned short*)p + e);
        const unsigned w[2] = {q.x, q.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (ST == 1) {
                v[2 * i] = pk_bf16_to_f32((unsigned short)(w[i] & 0xffffu));
                v[2 * i + 1] = pk_bf16_to_f32((unsigned short)(w[i] >> 16));
            } else {
                v[2 * i] = pk_f16_to_f32((unsigned short)(w[i] & 0xffffu));
                v[2 * i + 1] = pk_f16_to_f32((unsigned short)(w[i] >> 16));
            }
        }
    } else {
        const uint4 q = *(const uint4*)((const unsigned short*)p + e);
        const unsigned w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (ST == 1) {
                v[2 * i] = pk_bf16_to_f32((unsigned short)(w[i] & 0xffffu));
                v[2 * i + 1] = pk_bf16_to_f32((unsigned short)(w[i] >> 16));
            } else {
                v[2 * i] = pk_f16_to_f32((unsigned short)(w[i] & 0xffffu));
                v[2 * i + 1] = pk_f16_to_f32((unsigned short)(w[i] >> 16));
            }
        }
    }
}

// VEC values stored from element e, each rounded to the storage type
template <int ST, int VEC>
__device__ __forceinline__ void stv(void* p, long long e, const float (&v)[VEC], bool& ovf) {
    if constexpr (VEC == 1) {
        if (ST == 0) ((float*)p)[e] = v[0];
        else ((unsigned short*)p)[e] = narrow16<ST>(v[0], ovf);
    } else if constexpr (ST == 0) {
        *(float4*)((float*)p + e) = make_float4(v[0], v[1], v[2], v[3]);
    } else if constexpr (VEC == 4) {
        unsigned w[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            w[i] = (unsigned)narrow16<ST>(v[2 * i], ovf) | ((unsigned)narrow16<ST>(v[2 * i + 1], ovf) << 16);
        *(uint2*)((unsigned short*)p + e) = make_uint2(w[0], w[1]);
    } else {
        unsigned w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = (unsigned)narrow16<ST>(v[2 * i], ovf) | ((unsigned)narrow16<ST>(v[2 * i + 1], ovf) << 16);
        *(uint4*)((unsigned short*)p + e) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// lane l ^ D's value (the whole wave active), by register moves instead of
// the LDS crossbar: DPP quad permutations for 1 and 2, a half-row mirror of
// a quad reversal for 4 ((l & ~7) + 7 - (l & 7) of (l & ~3) + 3 - (l & 3)
// is l ^ 4), a row rotation by 8 for 8, and gfx950's row and half-wave
// swaps for 16 and 32: swapping a value with itself leaves each lane's
// partner in one of the two results (the odd rows' partners in the first),
// chosen by the lane's row or half
template <int D>
__device__ __forceinline__ float xor_lane(float v) {
    const int b = __builtin_bit_cast(int, v);
    int r;
    if constexpr (D == 1) {
        r = __builtin_amdgcn_update_dpp(0, b, 0xB1, 0xF, 0xF, false);       // quad_perm [1,0,3,2]
    } else if constexpr (D == 2) {
        r = __builtin_amdgcn_update_dpp(0, b, 0x4E, 0xF, 0xF, false);       // quad_perm [2,3,0,1]
    } else if constexpr (D == 4) {
        const int q = __builtin_amdgcn_update_dpp(0, b, 0x1B, 0xF, 0xF, false);   // quad_perm [3,2,1,0]
        r = __builtin_amdgcn_update_dpp(0, q, 0x141, 0xF, 0xF, false);            // row_half_mirror
    } else if constexpr (D == 8) {
        r = __builtin_amdgcn_update_dpp(0, b, 0x128, 0xF, 0xF, false);      // row_ror:8
    } else if constexpr (D == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap((unsigned)b, (unsigned)b, false, false);
        r = (int)(((threadIdx.x >> 4) & 1) ? p[0] : p[1]);
    } else {
        static_assert(D == 32, "a lane distance of the wave");
        const auto p = __builtin_amdgcn_permlane32_swap((unsigned)b, (unsigned)b, false, false);
        r = (int)(((threadIdx.x >> 5) & 1) ? p[0] : p[1]);
    }
    return __builtin_bit_cast(float, r);
}

// the 64 lanes' sums by the balanced pairwise tree over lane index: at
// distance d lane l adds lane l ^ d's value, and since a + b = b + a both
// lanes of a pair hold the same sum, so every lane ends with the tree's
// total
__device__ __forceinline__ float lanes_sum(float s) {
    s = s + xor_lane<1>(s);
    s = s + xor_lane<2>(s);
    s = s + xor_lane<4>(s);
    s = s + xor_lane<8>(s);
    s = s + xor_lane<16>(s);
    s = s + xor_lane<32>(s);
    return s;
}
__device__ __forceinline__ float lanes_max(float m) {
    m = __builtin_fmaxf(m, xor_lane<1>(m));
    m = __builtin_fmaxf(m, xor_lane<2>(m));
    m = __builtin_fmaxf(m, xor_lane<4>(m));
    m = __builtin_fmaxf(m, xor_lane<8>(m));
    m = __builtin_fmaxf(m, xor_lane<16>(m));
    m = __builtin_fmaxf(m, xor_lane<32>(m));
    return m;
}

// e / z for FAST: the reciprocal of z refined once, the quotient corrected
// once (Markstein)
struct Quot {
    float z, y;
    __device__ __forceinline__ explicit Quot(float z_) : z(z_) {
        const float y0 = __builtin_amdgcn_rcpf(z_);
        y = __builtin_fmaf(__builtin_fmaf(-z_, y0, 1.0f), y0, y0);
    }
    __device__ __forceinline__ float operator()(float e) const {
        const float q0 = e * y;
        return __builtin_fmaf(__builtin_fmaf(-q0, z, e), y, q0);
    }
};

// mask bits of block b (VEC bits from bit b * VEC of the row's bit array)
template <int VEC>
__device__ __forceinline__ unsigned block_bits(const unsigned char* mrow, long long b) {
    if constexpr (VEC == 8) return mrow[b];
    else if constexpr (VEC == 4) return (mrow[b >> 1] >> ((b & 1) * 4)) & 0xfu;
    else return (mrow[b >> 3] >> (b & 7)) & 1u;
}

// KIND 0: sum / mean / sum_to onto rows; 1: softmax (masked or not, three
// passes or two); 2: cross entropy; 3: its vjp.  CH blocks a lane.
template <int KIND, int ST, int VEC, int CH>
__global__ void __launch_bounds__(64 * WAVES) wrows_kernel(RowArgs a) {
    const int lane = threadIdx.x & 63;
    const long long row = (long long)blockIdx.x * WAVES + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const long long n = a.n;
    const long long base = row * n;
    const long long nb = (n + VEC - 1) / VEC;     // blocks of the row (the last whole when VEC > 1)
    const bool masked = a.op == kMaskedSoftmax3 || a.op == kMaskedSoftmax2;
    const unsigned char* mrow = nullptr;
    // the packed mask's rows: (n + 63) / 64 * 2 words each (rows.hip's layout)
    if (KIND == 1 && masked) {
        // the mask's row, in 32-bit arithmetic where the operands fit (a
        // 64-bit remainder is a long scalar sequence ahead of the loads)
        const unsigned long long r = (unsigned long long)(row + a.mask_row0);
        const unsigned long long mr = (r >> 32) == 0 && ((unsigned long long)a.mask_rows >> 32) == 0
                                          ? (unsigned long long)((unsigned)r % (unsigned)a.mask_rows)
                                          : r % (unsigned long long)a.mask_rows;
        mrow = (const unsigned char*)(a.mbits + (long long)mr * ((n + 63) / 64 * 2));
    }
    bool ovf = false;

    // the lane's blocks, loaded once (a block past the row or wholly masked
    // is not read)
    float v[CH][VEC];
    unsigned allow[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const long long b = (long long)j * 64 + lane;
        allow[j] = 0;
        if (b < nb) {
            allow[j] = (1u << VEC) - 1;
            if (KIND == 1 && masked) allow[j] &= block_bits<VEC>(mrow, b);
        }
        if (allow[j]) {
            ldv<ST, VEC>(a.x, base + b * VEC, v[j]);
        } else {
#pragma unroll
            for (int i = 0; i < VEC; ++i) v[j][i] = 0.0f;
        }
    }

    if constexpr (KIND == 0) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < CH; ++j)
#pragma unroll
            for (int i = 0; i < VEC; ++i) s = s + v[j][i];     // absent elements are +0: a sum from +0 is unchanged by them
        s = lanes_sum(s);
        if (lane == 0) {
            const float r = a.op == kRowMean ? s / a.n_real : s;
            float o[1] = {r};
            stv<ST, 1>(a.out, row, o, ovf);
        }
    } else {
        // the row's max over its allowed elements.  Where each lane's block j
        // is wholly allowed or wholly not (every block of an unmasked row,
        // all but the diagonal's of a causal one), the wave takes a path
        // without the per-element test; elsewhere every lane tests (one path,
        // not both)
        constexpr unsigned FULL = (1u << VEC) - 1;
        bool whole[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) whole[j] = __all(allow[j] == FULL || allow[j] == 0);
        float m = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            if (whole[j]) {
                if (allow[j]) {
#pragma unroll
                    for (int i = 0; i < VEC; ++i) m = __builtin_fmaxf(m, v[j][i]);
                }
            } else if (allow[j]) {
#pragma unroll
                for (int i = 0; i < VEC; ++i)
                    if ((allow[j] >> i) & 1u) m = __builtin_fmaxf(m, v[j][i]);
            }
        }
        m = lanes_max(m);
        // every allowed element's exponential, their sum in the declared
        // order; a block with no allowed element holds zeros already, and
        // adding them to a sum of nonnegative terms changes no bit, so its
        // lanes skip it (a wave skips a block no lane's row allows: a causal
        // mask's upper triangle)
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            if (whole[j]) {
                if (allow[j]) {
#pragma unroll
                    for (int i = 0; i < VEC; ++i) {
                        const float e = pk_expf_fast(v[j][i] - m);
                        v[j][i] = e;
                        s = s + e;
                    }
                }
            } else if (allow[j]) {
#pragma unroll
                for (int i = 0; i < VEC; ++i) {
                    const float e = (allow[j] >> i) & 1u ? pk_expf_fast(v[j][i] - m) : 0.0f;
                    v[j][i] = e;
                    s = s + e;
                }
            }
        }
        const float z = lanes_sum(s);
        if constexpr (KIND == 1) {
            const Quot q(z);
            const bool two = a.op == kSoftmax2 || a.op == kMaskedSoftmax2;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const long long b = (long long)j * 64 + lane;
                if (b >= nb) continue;
                float o[VEC];
                if (whole[j] && allow[j]) {
#pragma unroll
                    for (int i = 0; i < VEC; ++i)
                        // the two-pass nest divides the stored exponential
                        o[i] = q(two ? stored<ST>(v[j][i]) : v[j][i]);
                } else if (allow[j]) {
#pragma unroll
                    for (int i = 0; i < VEC; ++i)
                        o[i] = (allow[j] >> i) & 1u ? q(two ? stored<ST>(v[j][i]) : v[j][i]) : 0.0f;
                } else {
#pragma unroll
                    for (int i = 0; i < VEC; ++i) o[i] = 0.0f;
                }
                stv<ST, VEC>(a.out, base + b * VEC, o, ovf);
            }
        } else if constexpr (KIND == 2) {
            // log(z) + m - x[y]
            if (lane == 0) {
                long long y = ((const long long*)a.y)[row];
                y = y < 0 ? 0 : y >= n ? n - 1 : y;
                float o[1] = {(pk_logf(z) + m) - ld1<ST>(a.x, base + y)};
                stv<ST, 1>(a.out, row, o, ovf);
            }
        } else {
            // (exp(x - m) / z - onehot(y)) * ct
            const Quot q(z);
            long long y = ((const long long*)a.y)[row];
            const float ct = ld1<ST>(a.ct, row);
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const long long b = (long long)j * 64 + lane;
                if (b >= nb) continue;
                float o[VEC];
#pragma unroll
                for (int i = 0; i < VEC; ++i) {
                    const float hot = b * VEC + i == y ? 1.0f : 0.0f;
                    o[i] = (q(v[j][i]) - hot) * ct;
                }
                stv<ST, VEC>(a.out, base + b * VEC, o, ovf);
            }
        }
    }
    if (ovf && a.flag) atomicOr(a.flag, 1u);
}

template <int KIND, int ST, int VEC>
hipError_t launch_ch(const RowArgs& a, int ch, hipStream_t stream) {
    const unsigned grid = (unsigned)((a.rows + WAVES - 1) / WAVES);
    switch (ch) {
        case 1: wrows_kernel<KIND, ST, VEC, 1><<<grid, 64 * WAVES, 0, stream>>>(a); break;
        case 2: wrows_kernel<KIND, ST, VEC, 2><<<grid, 64 * WAVES, 0, stream>>>(a); break;
        case 4: wrows_kernel<KIND, ST, VEC, 4><<<grid, 64 * WAVES, 0, stream>>>(a); break;
        case 8: wrows_kernel<KIND, ST, VEC, 8><<<grid, 64 * WAVES, 0, stream>>>(a); break;
        case 16: wrows_kernel<KIND, ST, VEC, 16><<<grid, 64 * WAVES, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int KIND, int ST>
hipError_t launch_st(const RowArgs& a, int vec, int ch, hipStream_t stream) {
    if (vec == 1) return launch_ch<KIND, ST, 1>(a, ch, stream);
    if constexpr (ST != 0)
        if (vec == 4) return launch_ch<KIND, ST, 4>(a, ch, stream);
    return launch_ch<KIND, ST, ST == 0 ? 4 : 8>(a, ch, stream);
}

template <int KIND>
hipError_t launch_kind(const RowArgs& a, int vec, int ch, hipStream_t stream) {
    switch (a.storage) {
        case 0: return launch_st<KIND, 0>(a, vec, ch, stream);
        case 1: return launch_st<KIND, 1>(a, vec, ch, stream);
        case 2: return launch_st<KIND, 2>(a, vec, ch, stream);
    }
    return hipErrorInvalidValue;
}

int kind_of(int op) {
    switch (op) {
        case kRowMean: case kRowSum: case kSumToRows: return 0;
        case kSoftmax3: case kSoftmax2: case kMaskedSoftmax3: case kMaskedSoftmax2: return 1;
        case kCrossEntropy: return 2;
        case kCrossEntropyVjp: return 3;
    }
    return -1;
}

// 16-byte blocks when every row is whole vectors, else single elements;
// 16-bit rows of at most 256 elements in 8-byte blocks (4 elements), so
// that all 64 lanes hold a part of the row (the course's attention rows:
// 64 blocks of 4, not 32 of 8 with half the wave idle); the blocks a lane
// holds, a power of two up to 16.  0 when the rows are too long to hold.
int vec_of(const RowArgs& a) {
    const int esz = a.storage == 0 ? 4 : 2;
    if (esz == 2 && a.n <= 256 && a.n % 4 == 0) return 4;
    return (a.n * esz) % 16 == 0 ? 16 / esz : 1;
}
int ch_of(long long n, int vec) {
    const long long blocks = (n + vec - 1) / vec;
    long long c = 1;
    while (c * 64 < blocks) c *= 2;
    return c > 16 ? 0 : (int)c;
}

bool writes_rows(int op) {
    return op == kSoftmax3 || op == kSoftmax2 || op == kMaskedSoftmax3 || op == kMaskedSoftmax2 || op == kCrossEntropyVjp;
}

}  // namespace

bool wrows_ok(const RowArgs& a) {
    return kind_of(a.op) >= 0 && a.n > 0 && a.storage >= 0 && a.storage <= 2 && ch_of(a.n, vec_of(a)) > 0 &&
           (a.rows + WAVES - 1) / WAVES <= 0x7fffffffll;
}

int wrows_vec(const RowArgs& a) { return vec_of(a); }

bool wrows_fits(const RowArgs& a) {
    if (!wrows_ok(a)) return false;
    const int vec = vec_of(a);
    return vec == 1 || ((uintptr_t)a.x % 16 == 0 && (!writes_rows(a.op) || (uintptr_t)a.out % 16 == 0));
}

hipError_t wrows_launch(const RowArgs& a, hipStream_t stream) {
    if (a.rows == 0) return hipSuccess;
    if (!wrows_fits(a)) return hipErrorInvalidValue;
    const int vec = vec_of(a), ch = ch_of(a.n, vec);
    if (a.op == kMaskedSoftmax3 || a.op == kMaskedSoftmax2) {
        if (!a.mbits || a.mask_rows <= 0) return hipErrorInvalidValue;
        hipError_t e = rows_pack_mask(a, stream);
        if (e != hipSuccess) return e;
    }
    switch (kind_of(a.op)) {
        case 0: return launch_kind<0>(a, vec, ch, stream);
        case 1: return launch_kind<1>(a, vec, ch, stream);
        case 2: return launch_kind<2>(a, vec, ch, stream);
        case 3: return launch_kind<3>(a, vec, ch, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace presk
