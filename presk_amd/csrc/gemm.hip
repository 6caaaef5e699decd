// The contraction class: `dot`, `dot+add`, `dot_vjp_l`, `dot_vjp_r` and
// two-operand `ein` nests (crates/presk-kernel/src/lower.rs:695-784, the
// "contraction nest") as LDS-tiled MFMA kernels for gfx950.
//
// C[b][m][n] = sum_k A(b, m, k) * B(b, k, n), then the epilogue of
// lower.rs:846-864 (+ bias), stored in the storage type.  Operands are read
// through general strides, so NN (`dot`), NT (`dot_vjp_l`, QK^T), TN
// (`dot_vjp_r`) and batched (`ein`) forms are one kernel.
//
// Order (declared, not the interpreter's index order): each 16x16 output tile
// accumulates on MFMA in f32 -- v_mfma_f32_16x16x32_{bf16,f16} for 16-bit
// storage (the products of two 16-bit values are exact in f32), and
// v_mfma_f32_16x16x4_f32 for f32 storage -- over k-blocks of 64 (32 for f32)
// in increasing k, and, when K is split across workgroups, the split partial
// sums are added in increasing split order by a second kernel (deterministic).
//
// Tile: 128x128 per workgroup of 256 threads (4 waves of 64, each 64x64 =
// 4x4 MFMA tiles), operands staged through LDS k-contiguous; an operand whose
// contiguous axis is m or n is transposed on its way into LDS.
#include <hip/hip_runtime.h>

#include "devfmt.hpp"
#include "gemm.hpp"

namespace presk {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, NT = 256;

// Storage traits: S = element in memory and LDS, BK = k-block, VEC = elements
// per 16-byte global load.
template <int ST> struct St;
template <> struct St<kF32> {
    typedef float S;
    static constexpr int BK = 32, VEC = 4, PAD = 4;
    static __device__ __forceinline__ float widen(float x) { return x; }
};
template <> struct St<kBF16> {
    typedef unsigned short S;
    static constexpr int BK = 64, VEC = 8, PAD = 8;
    static __device__ __forceinline__ float widen(unsigned short x) { return pk_bf16_to_f32(x); }
};
template <> struct St<kF16> {
    typedef unsigned short S;
    static constexpr int BK = 64, VEC = 8, PAD = 8;
    static __device__ __forceinline__ float widen(unsigned short x) { return pk_f16_to_f32(x); }
};

__device__ __forceinline__ long long batch_offset(const GemmArgs& g, long long b, const long long* strides) {
    long long off = 0;
    for (int d = g.nbatch - 1; d >= 0; --d) {
        long long i = b % g.bdim[d];
        b /= g.bdim[d];
        off += i * strides[d];
    }
    return off;
}

// One operand's tile (rows x BK) staged into LDS as tile[row][k], k contiguous.
// `rs`/`ks` are the operand's element strides along its row axis (m or n) and k.
template <int ST, bool KCONTIG>
struct Loader {
    typedef typename St<ST>::S S;
    static constexpr int BK = St<ST>::BK, VEC = St<ST>::VEC, LD = BK + St<ST>::PAD;
    // registers: KCONTIG: 4 rounds of one 16-byte vector; else VEC rows x 4 k
    static constexpr int REGS = KCONTIG ? 4 * VEC : 4 * VEC;
    S r[REGS];

    __device__ __forceinline__ void load(const S* __restrict__ p, long long rows, long long K, long long rs, long long ks,
                                         long long row0, long long k0, bool vec_ok) {
        const int t = threadIdx.x;
        if (KCONTIG) {
            // BK/VEC threads per row, NT/(BK/VEC) rows per round, 4 rounds
            constexpr int TPR = BK / VEC, RPR = NT / TPR;
            const int kc = (t % TPR) * VEC;
#pragma unroll
            for (int round = 0; round < 4; ++round) {
                const long long row = row0 + (t / TPR) + round * RPR;
                const long long k = k0 + kc;
                const S* src = p + row * rs + k;
                if (row < rows && vec_ok && k + VEC <= K) {
                    if (VEC == 8) {
                        u16x8 v = *(const u16x8*)src;
#pragma unroll
                        for (int j = 0; j < VEC; ++j) r[round * VEC + j] = (S)v[j];
                    } else {
                        f32x4 v = *(const f32x4*)src;
#pragma unroll
                        for (int j = 0; j < VEC; ++j) r[round * VEC + j] = (S)v[j];
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < VEC; ++j) r[round * VEC + j] = (row < rows && k + j < K) ? src[j * ks] : (S)0;
                }
            }
        } else {
            // the row axis contiguous: each thread a VEC(rows) x 4(k) block
            constexpr int TPK = BM / VEC;   // threads along rows per k-quad
            const long long row = row0 + (t % TPK) * VEC;
            const long long kq = k0 + (t / TPK) * 4;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const long long k = kq + kk;
                const S* src = p + k * ks + row * rs;
                if (k < K && vec_ok && row + VEC <= rows) {
                    if (VEC == 8) {
                        u16x8 v = *(const u16x8*)src;
#pragma unroll
                        for (int j = 0; j < VEC; ++j) r[kk * VEC + j] = (S)v[j];
                    } else {
                        f32x4 v = *(const f32x4*)src;
#pragma unroll
                        for (int j = 0; j < VEC; ++j) r[kk * VEC + j] = (S)v[j];
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < VEC; ++j) r[kk * VEC + j] = (k < K && row + j < rows) ? src[j * rs] : (S)0;
                }
            }
        }
    }

    __device__ __forceinline__ void store(S* tile) const {
        const int t = threadIdx.x;
        if (KCONTIG) {
            constexpr int TPR = BK / VEC, RPR = NT / TPR;
            const int kc = (t % TPR) * VEC;
#pragma unroll
            for (int round = 0; round < 4; ++round) {
                S* dst = tile + ((t / TPR) + round * RPR) * LD + kc;
#pragma unroll
                for (int j = 0; j < VEC; ++j) dst[j] = r[round * VEC + j];
            }
        } else {
            constexpr int TPK = BM / VEC;
            const int row = (t % TPK) * VEC, kq = (t / TPK) * 4;
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                S* dst = tile + (row + j) * LD + kq;
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) dst[kk] = r[kk * VEC + j];
            }
        }
    }
};

template <int ST>
__device__ __forceinline__ f32x4 mfma_step(const typename St<ST>::S* a, const typename St<ST>::S* b, f32x4 acc);

template <>
__device__ __forceinline__ f32x4 mfma_step<kBF16>(const unsigned short* a, const unsigned short* b, f32x4 acc) {
    u16x8 va = *(const u16x8*)a, vb = *(const u16x8*)b;
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, va), __builtin_bit_cast(bf16x8, vb), acc, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma_step<kF16>(const unsigned short* a, const unsigned short* b, f32x4 acc) {
    u16x8 va = *(const u16x8*)a, vb = *(const u16x8*)b;
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, va), __builtin_bit_cast(f16x8, vb), acc, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma_step<kF32>(const float* a, const float* b, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(*a, *b, acc, 0, 0, 0);
}

// The storage-type store of an output element with the epilogue: f32 storage
// adds the bias to the sum; narrow storage stores the sum rounded, reads it
// back and adds (lower.rs:1053-1060), each store under the overflow guard.
template <int ST>
__device__ __forceinline__ void store_out(void* C, long long off, float sum, bool has_bias, float bias, bool& ovf) {
    if (ST == kF32) {
        ((float*)C)[off] = has_bias ? sum + bias : sum;
    } else if (ST == kBF16) {
        unsigned short h = pk_f32_to_bf16(sum);
        if (has_bias) h = pk_f32_to_bf16(pk_bf16_to_f32(h) + bias);
        ((unsigned short*)C)[off] = h;
    } else {
        ovf |= pk_overflows_f16(sum);
        unsigned short h = pk_f32_to_f16(sum);
        if (has_bias) {
            const float v = pk_f16_to_f32(h) + bias;
            ovf |= pk_overflows_f16(v);
            h = pk_f32_to_f16(v);
        }
        ((unsigned short*)C)[off] = h;
    }
}

template <int ST>
__device__ __forceinline__ float load_bias(const void* p, long long off) {
    if (ST == kF32) return ((const float*)p)[off];
    return St<ST>::widen(((const unsigned short*)p)[off]);
}

template <int ST, bool AK, bool BK_>
__global__ void __launch_bounds__(NT) gemm_kernel(GemmArgs g) {
    typedef typename St<ST>::S S;
    constexpr int BK = St<ST>::BK, LD = BK + St<ST>::PAD;
    __shared__ __attribute__((aligned(16))) S As[BM * LD];
    __shared__ __attribute__((aligned(16))) S Bs[BN * LD];

    // tile order: blocks of one XCD (block id mod 8) take consecutive tiles,
    // and tiles go row-group by row-group so that concurrent tiles share A rows
    const long long tiles = (long long)g.tiles_m * g.tiles_n;
    long long bid = blockIdx.x;
    const long long per_xcd = (tiles + 7) / 8;
    if (tiles >= 64 && tiles % 8 == 0) bid = (bid % 8) * per_xcd + bid / 8;
    constexpr long long GROUP = 8;
    const long long group_size = GROUP * g.tiles_n;
    const long long grp = bid / group_size;
    const long long first_m = grp * GROUP;
    const long long gm = (g.tiles_m - first_m) < GROUP ? (g.tiles_m - first_m) : GROUP;
    const long long tm_idx = first_m + (bid % group_size) % gm;
    const long long tn_idx = (bid % group_size) / gm;
    const long long m0 = tm_idx * BM, n0 = tn_idx * BN;
    const long long batch = blockIdx.y;
    const int split = blockIdx.z;

    const S* A = (const S*)g.A + batch_offset(g, batch, g.sa_b);
    const S* B = (const S*)g.B + batch_offset(g, batch, g.sb_b);
    const long long kbeg = (long long)split * g.k_per_split;
    long long kend = kbeg + g.k_per_split;
    if (kend > g.K) kend = g.K;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    Loader<ST, AK> la;
    Loader<ST, BK_> lb;
    const long long nk = (kend - kbeg + BK - 1) / BK;
    if (nk > 0) {
        la.load(A, g.M, kend, g.sa_m, g.sa_k, m0, kbeg, g.a_vec);
        lb.load(B, g.N, kend, g.sb_n, g.sb_k, n0, kbeg, g.b_vec);
        la.store(As);
        lb.store(Bs);
    }
    __syncthreads();
    for (long long kt = 0; kt < nk; ++kt) {
        const long long knext = kbeg + (kt + 1) * BK;
        if (kt + 1 < nk) {
            la.load(A, g.M, kend, g.sa_m, g.sa_k, m0, knext, g.a_vec);
            lb.load(B, g.N, kend, g.sb_n, g.sb_k, n0, knext, g.b_vec);
        }
        if (ST == kF32) {
#pragma unroll
            for (int kk = 0; kk < BK; kk += 4) {
                const int kl = kk + (lane >> 4);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = mfma_step<ST>(&As[(wm + i * 16 + (lane & 15)) * LD + kl], &Bs[(wn + j * 16 + (lane & 15)) * LD + kl], acc[i][j]);
            }
        } else {
#pragma unroll
            for (int kk = 0; kk < BK; kk += 32) {
                const int kl = kk + (lane >> 4) * 8;
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = mfma_step<ST>(&As[(wm + i * 16 + (lane & 15)) * LD + kl], &Bs[(wn + j * 16 + (lane & 15)) * LD + kl], acc[i][j]);
            }
        }
        __syncthreads();
        if (kt + 1 < nk) {
            la.store(As);
            lb.store(Bs);
            __syncthreads();
        }
    }

    // the tile's outputs: lane holds column (lane & 15), rows 4*(lane >> 4) + r
    bool ovf = false;
    const long long cbase = batch_offset(g, batch, g.sc_b);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const long long n = n0 + wn + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const long long m = m0 + wm + i * 16 + (lane >> 4) * 4 + r;
                if (m < g.M && n < g.N) {
                    const float v = acc[i][j][r];
                    if (g.splits > 1) {
                        g.work[((long long)split * g.M + m) * g.N + n] = v;
                    } else {
                        float b = 0.f;
                        if (g.bias) b = load_bias<ST>(g.bias, ((m / g.bias_div) % g.bias_mod) * g.sbias_m + n * g.sbias_n);
                        store_out<ST>(g.C, cbase + m * g.N + n, v, g.bias != nullptr, b, ovf);
                    }
                }
            }
        }
    }
    if (ovf && g.flag) atomicOr(g.flag, 1u);
}

// The split partial sums added in increasing split order, then the epilogue.
template <int ST>
__global__ void __launch_bounds__(256) split_reduce_kernel(GemmArgs g) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= g.M * g.N) return;
    const long long m = idx / g.N, n = idx % g.N;
    float s = g.work[idx];
    for (int p = 1; p < g.splits; ++p) s = s + g.work[(long long)p * g.M * g.N + idx];
    bool ovf = false;
    float b = 0.f;
    if (g.bias) b = load_bias<ST>(g.bias, ((m / g.bias_div) % g.bias_mod) * g.sbias_m + n * g.sbias_n);
    store_out<ST>(g.C, idx, s, g.bias != nullptr, b, ovf);
    if (ovf && g.flag) atomicOr(g.flag, 1u);
}

template <int ST>
hipError_t launch_typed(const GemmArgs& g, hipStream_t stream) {
    dim3 grid((unsigned)(g.tiles_m * g.tiles_n), (unsigned)g.batch, (unsigned)g.splits);
    if (g.a_kcontig && g.b_kcontig) gemm_kernel<ST, true, true><<<grid, NT, 0, stream>>>(g);
    else if (g.a_kcontig) gemm_kernel<ST, true, false><<<grid, NT, 0, stream>>>(g);
    else if (g.b_kcontig) gemm_kernel<ST, false, true><<<grid, NT, 0, stream>>>(g);
    else gemm_kernel<ST, false, false><<<grid, NT, 0, stream>>>(g);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || g.splits <= 1) return e;
    const long long n = g.M * g.N;
    split_reduce_kernel<ST><<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(g);
    return hipGetLastError();
}

}  // namespace

int gemm_block_k(int storage) { return storage == kF32 ? St<kF32>::BK : St<kBF16>::BK; }
int gemm_tile_m() { return BM; }
int gemm_tile_n() { return BN; }

hipError_t gemm_launch(const GemmArgs& g, hipStream_t stream) {
    switch (g.storage) {
        case kF32: return launch_typed<kF32>(g, stream);
        case kBF16: return launch_typed<kBF16>(g, stream);
        case kF16: return launch_typed<kF16>(g, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace presk
