// The contraction class: `dot`, `dot+add`, `dot_vjp_l`, `dot_vjp_r` and
// two-operand `ein` nests (crates/presk-kernel/src/lower.rs:695-784, the
// "contraction nest") as LDS-tiled MFMA kernels for gfx950.
//
// C[b][m][n] = sum_k A(b, m, k) * B(b, k, n), then the epilogue of
// lower.rs:846-864 (+ bias), stored in the storage type.  Operands are read
// through general strides, so NN (`dot`), NT (`dot_vjp_l`, QK^T), TN
// (`dot_vjp_r`) and batched (`ein`) forms are one kernel.
//
// Order (declared, not the interpreter's index order): each output tile
// accumulates on MFMA in f32 -- v_mfma_f32_32x32x16_{bf16,f16} (order
// "mfma-k16") or, on the 128 x 96 tiles, v_mfma_f32_16x16x32_{bf16,f16}
// ("mfma-k32") for 16-bit storage (the product of two 16-bit values is exact
// in f32), and v_mfma_f32_16x16x4_f32 for f32 storage -- over k-blocks of 64
// (32 for f32) in increasing k; when K is split across workgroups, the
// partial sums are added in increasing split order by a second kernel
// (deterministic).
//
// 16-bit storage, whole k-blocks and strides of whole 16-byte vectors:
// 256 x 128 tiles (K of 768 or more, no split) or 256 x 256 (K of 3072 or
// more, three rounds of the CUs), eight waves a workgroup (two a SIMD, one
// workgroup a CU), each wave 64 x 64 or 128 x 64 as MFMAs of 32x32x16,
// operands loaded straight into LDS three (two) k-blocks deep (D16Loader),
// the fragments of each 16-k step read while the previous step's MFMAs run;
// 128 x 128 and 128 x 64 tiles the same way with four waves in two stages,
// two or three workgroups a CU, and 128 x 128 tiles of eight waves four
// stages deep for split weight gradients.  Operands off 16 bytes or partial
// k-blocks take four-wave tiles and the same MFMAs from register-staged
// operands; 128 x 96 tiles take the 16x16 MFMAs below.
//
// f32 storage, whole 32-deep k-blocks and strides of whole vectors: eight-wave
// tiles too (F32Loader), 256 x 128 and 256 x 96 three k-blocks deep, 128 x
// 128 four deep (split weight gradients among them) and 128 x 96 two deep
// (two workgroups a CU), each wave's
// 16x16x4 MFMAs taking the operands' roles exchanged so that its sums leave
// as 16-byte row stores from the registers.
//
// Workgroup: 256 threads (4 waves as 2x2; the eight-wave tiles 512, as 2x4
// or 4x2), tile (2*WM*16) x (2*WN*16), each wave WM x WN MFMA tiles of
// 16x16 (of 32x32 in the 16-bit direct tiles).  Operands are staged through LDS,
// double-buffered (one barrier per k-block), each as it lies in memory: a
// k-contiguous operand as [row][k], an m- or n-contiguous one as [k][row]
// (16-byte writes either way).  MFMA fragments hold consecutive k of one
// row: read directly from [row][k]; from [k][row] by gfx950's transposing
// LDS read (ds_read_b64_tr_b16: in each 16-lane group, lane i receives
// element i % 4 of the 8-byte chunks lanes i/4 + 4j read, so lanes reading
// k-rows kb + L/4 at columns 4*(L % 4) hand lane i four consecutive k of its
// column) for 16-bit types, by plain reads for f32 (one k a lane).  f32
// operands of whole k-blocks and aligned vectors skip the registers: each
// lane's 16 bytes go from global memory straight into an XOR-swizzled LDS
// tile (global_load_lds_dwordx4), the same products in the same order.
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "devfmt.hpp"
#include "gemm.hpp"

namespace presk {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));

constexpr int NT = 256;

// Storage traits: S = element in memory and LDS, BK = k-block, VEC = elements
// per 16-byte global load, KSTEP = k per MFMA, KPL = k per lane per MFMA.
template <int ST> struct St;
template <> struct St<kF32> {
    typedef float S;
    typedef f32x4 V;
    typedef float Frag;
    static constexpr int BK = 32, VEC = 4, PAD = 4, KSTEP = 4, KPL = 1;
};
template <> struct St<kBF16> {
    typedef unsigned short S;
    typedef u16x8 V;
    typedef u16x8 Frag;
    static constexpr int BK = 64, VEC = 8, PAD = 8, KSTEP = 32, KPL = 8;
};
template <> struct St<kF16> : St<kBF16> {};

__device__ __forceinline__ long long batch_offset(const GemmArgs& g, long long b, const long long* strides) {
    long long off = 0;
    for (int d = g.nbatch - 1; d >= 0; --d) {
        long long i = b % g.bdim[d];
        b /= g.bdim[d];
        off += i * strides[d];
    }
    return off;
}

// One operand's tile (ROWS x BK) staged into LDS as tile[row][k], k contiguous.
// `rs`/`ks` are the operand's element strides along its row axis (m or n) and k.
template <int ST, bool KCONTIG, int ROWS>
struct Loader {
    typedef typename St<ST>::S S;
    typedef typename St<ST>::V V;
    static constexpr int BK = St<ST>::BK, VEC = St<ST>::VEC, LD = BK + St<ST>::PAD;
    // KCONTIG: the tile is [ROWS][LD], BK/VEC threads per row -> ROWS/(NT/(BK/VEC))
    // rounds of one vector.  else: the tile is [BK][LDR], ROWS/VEC vectors per
    // k-row, BK k-rows over NT threads -> rounds.
    static constexpr int TPR = BK / VEC, RPR = NT / TPR, ROUNDS_K = ROWS / RPR;
    static constexpr int LDR = ROWS + 16, VPR = ROWS / VEC, ROUNDS_T = (BK * VPR + NT - 1) / NT;
    static constexpr bool PARTIAL_T = (BK * VPR) % NT != 0;  // the last round leaves threads idle
    static constexpr int NV = KCONTIG ? ROUNDS_K : ROUNDS_T;
    static constexpr int SIZE = KCONTIG ? ROWS * LD : BK * LDR;   // elements of one tile
    V r[NV];
    bool kin[NV];   // the vector's k lies below K; applied when it is stored, so
                    // that no use of the loaded registers waits for the loads
                    // before the MFMAs of the current k-block have been issued

    // Loads are unconditional 16-byte vectors from clamped addresses: a row
    // past the operand repeats its last row (the results of such rows are
    // never stored), a k past K reads k = K-1 and is zeroed by a select, so
    // the hot loop has no branches.  Needs the vector axis (k, or the rows
    // when the operand is transposed) to be a multiple of VEC and aligned;
    // the launcher checks, and otherwise uses the element-wise variant.
    __device__ __forceinline__ void load(const S* __restrict__ p, int rows, int K, int rs, int ks, int row0, int k0) {
        const int t = threadIdx.x;
        if (KCONTIG) {
            const int kc = (t % TPR) * VEC;
            const int k = k0 + kc;
            const bool in = k < K;
            const int kcl = in ? k : K - VEC;
#pragma unroll
            for (int q = 0; q < ROUNDS_K; ++q) {
                int row = row0 + (t / TPR) + q * RPR;
                row = row < rows ? row : rows - 1;
                r[q] = *(const V*)(p + (long long)row * rs + kcl);
                kin[q] = in;
            }
        } else {
#pragma unroll
            for (int q = 0; q < ROUNDS_T; ++q) {
                const int u = PARTIAL_T && t + q * NT >= BK * VPR ? BK * VPR - 1 : t + q * NT;
                int row = row0 + (u % VPR) * VEC;
                row = row + VEC <= rows ? row : rows - VEC;
                const int k = k0 + u / VPR;
                const bool in = k < K;
                r[q] = *(const V*)(p + (long long)(in ? k : K - 1) * ks + row);
                kin[q] = in;
            }
        }
    }

    // The element-wise variant for operands whose vector axis is ragged or
    // unaligned: every element bounds-checked.
    __device__ __forceinline__ void load_checked(const S* __restrict__ p, int rows, int K, int rs, int ks, int row0, int k0) {
        const int t = threadIdx.x;
        if (KCONTIG) {
            const int kc = (t % TPR) * VEC;
#pragma unroll
            for (int q = 0; q < ROUNDS_K; ++q) {
                const int row = row0 + (t / TPR) + q * RPR;
                for (int j = 0; j < VEC; ++j) {
                    const int k = k0 + kc + j;
                    r[q][j] = (row < rows && k < K) ? p[(long long)row * rs + (long long)k * ks] : (S)0;
                }
                kin[q] = true;
            }
        } else {
#pragma unroll
            for (int q = 0; q < ROUNDS_T; ++q) {
                const int u = PARTIAL_T && t + q * NT >= BK * VPR ? BK * VPR - 1 : t + q * NT;
                const int row = row0 + (u % VPR) * VEC, k = k0 + u / VPR;
                for (int j = 0; j < VEC; ++j)
                    r[q][j] = (k < K && row + j < rows) ? p[(long long)k * ks + (long long)(row + j) * rs] : (S)0;
                kin[q] = true;
            }
        }
    }

    __device__ __forceinline__ void store(S* tile) const {
        const int t = threadIdx.x;
        if (KCONTIG) {
            const int kc = (t % TPR) * VEC;
#pragma unroll
            for (int q = 0; q < ROUNDS_K; ++q) *(V*)(tile + ((t / TPR) + q * RPR) * LD + kc) = kin[q] ? r[q] : V{};
        } else {
#pragma unroll
            for (int q = 0; q < ROUNDS_T; ++q) {
                const int u = t + q * NT;
                if (PARTIAL_T && u >= BK * VPR) break;  // an idle thread of the last round
                *(V*)(tile + (u / VPR) * LDR + (u % VPR) * VEC) = kin[q] ? r[q] : V{};
            }
        }
    }
};

// f32 operand tiles loaded straight into LDS (global_load_lds_dwordx4: lane
// i of a wave's load writes bytes [16 i, 16 i + 16) of the wave's 1 KB LDS
// segment, from any global address it names), so that no register, wait or
// LDS write stands between the loads and the products.  No padding: 16-byte
// chunks are placed by an XOR swizzle that keeps the fragment reads free of
// bank conflicts (per 32 lanes, 32 distinct banks):
//   k-contiguous, [row][32 k]: chunk (r, kc) at slot r*8 + (kc ^ (r & 7))
//   m/n-contiguous, [k][ROWS]: chunk (k, cc) at slot k*(ROWS/4) + (cc ^ 4*(k & 1))
// Rows past the operand read its last row (their results are never stored).
// Nothing zeroes a k past K, so the launcher takes this path only when every
// k-block is whole (K % 32 == 0) and the operands hold aligned 16-byte
// vectors along their loaded axis.
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

template <bool KCONTIG, int ROWS>
struct DLoader {
    static constexpr int BK = 32, CPR = ROWS / 4;     // CPR: chunks per k-row of [k][ROWS]
    static constexpr int ROUNDS = ROWS * 8 / NT;      // chunks per thread
    static constexpr int SIZE = ROWS * BK;            // floats of one tile
    static_assert(ROWS * 8 % NT == 0, "whole rounds");
    __device__ __forceinline__ void load(const float* __restrict__ p, int rows, int rs, int ks, int row0, int k0,
                                         float* tile) const {
        const int t = threadIdx.x, wbase = t & ~63;
#pragma unroll
        for (int q = 0; q < ROUNDS; ++q) {
            const int slot = q * NT + t;
            const float* src;
            if (KCONTIG) {
                const int r = slot >> 3, kc = (slot & 7) ^ (r & 7);
                int row = row0 + r;
                row = row < rows ? row : rows - 1;
                src = p + (long long)row * rs + k0 + kc * 4;
            } else {
                const int k = slot / CPR, cc = (slot % CPR) ^ ((k & 1) * 4);
                int row = row0 + cc * 4;
                row = row + 4 <= rows ? row : rows - 4;
                src = p + (long long)(k0 + k) * ks + row;
            }
            // the wave's segment starts at its first slot; lane i fills slot + i
            __builtin_amdgcn_global_load_lds((glb_void_t*)src, (lds_void_t*)(tile + (q * NT + wbase) * 4), 16, 0, 0);
        }
    }
};

// f32 fragment (k = kk + (lane >> 4) of row base + (lane & 15)) from a swizzled tile
template <bool KC, int ROWS>
__device__ __forceinline__ float frag_dl(const float* xs, int base, int kk, int lane) {
    if constexpr (KC) {
        const int r = base + (lane & 15);
        return xs[r * 32 + (((kk >> 2) ^ (r & 7)) << 2) + (lane >> 4)];
    } else {
        const int k = kk + (lane >> 4), c = base + (lane & 15);
        return xs[k * ROWS + (((c >> 2) ^ ((k & 1) * 4)) << 2) + (c & 3)];
    }
}

typedef short v4i16 __attribute__((ext_vector_type(4)));

// 16-bit operand tiles (64 k) loaded straight into LDS, two or three stages
// deep, in 16-byte chunks placed by an XOR swizzle (lane i of a wave's load
// fills slot i of the wave's 1 KB segment; the swizzle picks which chunk each
// lane fetches):
//   k-contiguous, [row][8 chunks of 8 k]: chunk c of row r in slot
//     8 r + (c ^ ((r ^ (r >> 3)) & 7))
//   m/n-contiguous, [k][ROWS / 8 chunks of 8 rows]: chunk j of k-row r in slot
//     (ROWS / 8) r + (j ^ (2 (r & 3) ^ 8 (r & 1)))   (ROWS >= 128)
//     (ROWS / 8) r + (j ^ 2 (r & 3))                 (ROWS = 64)
// so that the 32x32x16 fragment reads below hit distinct banks in every
// 16-lane (and 32-lane) phase: 16-byte reads of 16 consecutive rows, and
// transposing 8-byte reads of 4 k-rows x 32 (64) bytes.  Rows past the
// operand read its last row (or last whole vector); the launcher takes this
// path only for whole k-blocks (K % 64 == 0) of aligned vectors.
//
// The loads (global_load_lds_dwordx4, saddr form: a wave-uniform base plus a
// 32-bit lane offset, the wave's LDS segment in m0) are issued by inline
// assembly: the compiler then tracks no LDS write for them and adds no
// vmcnt(0) before the barrier or the transposing reads, which would drain the
// blocks in flight; the kernel waits for them itself (wait_vm) before the
// barrier that precedes every read of a stage.  The lane offsets are fixed
// for the whole k-loop; a block moves the uniform base only.
template <bool KCONTIG, int ROWS, int NTH = NT>
struct D16Loader {
    static constexpr int BK = 64;
    static constexpr int CPR = KCONTIG ? 8 : ROWS / 8;    // chunks per LDS row
    static constexpr int SLOTS = ROWS * BK / 8;           // chunks per tile
    static constexpr int ROUNDS = SLOTS / NTH;            // loads per thread
    static constexpr int BYTES = SLOTS * 16;
    static_assert(SLOTS % NTH == 0, "whole rounds");
    unsigned voff[ROUNDS];      // byte offsets of this thread's chunks from the origin
    const char* origin;         // the operand's first k-block (uniform)
    long long block_bytes;      // how far one k-block moves the origin (uniform)
    unsigned lds0;              // this wave's segment of the stage-0 tile (uniform)

    // (a 64-row tile has 8 chunks a k-row: its swizzle stays below 8)
    __device__ static __forceinline__ int swz(int r) {
        return KCONTIG ? ((r ^ (r >> 3)) & 7) : ((2 * (r & 3)) ^ (ROWS >= 128 ? 8 * (r & 1) : 0));
    }
    __device__ __forceinline__ void init(const unsigned short* p, int rows, long long rs, long long ks, int row0, int k0,
                                         unsigned tile) {
        static_assert(KCONTIG || ROWS == 64 || ROWS % 128 == 0, "the swizzle stays inside a k-row");
        const int t = threadIdx.x;
        origin = (const char*)(p + (KCONTIG ? (long long)k0 : (long long)k0 * ks));
        block_bytes = KCONTIG ? 2LL * BK : 2LL * BK * ks;
#pragma unroll
        for (int q = 0; q < ROUNDS; ++q) {
            const int slot = q * NTH + t;
            const int r = slot / CPR, c = (slot % CPR) ^ swz(r);
            long long e;
            if (KCONTIG) {
                int row = row0 + r;
                row = row < rows ? row : rows - 1;
                e = row * rs + 8 * c;
            } else {
                int row = row0 + 8 * c;
                row = row + 8 <= rows ? row : rows - 8;
                e = r * ks + row;
            }
            voff[q] = (unsigned)(2 * e);
        }
        lds0 = __builtin_amdgcn_readfirstlane(tile + (unsigned)(t & ~63) * 16u);
    }
    // k-block kb into the tile `stage` bytes past the stage-0 tile
    __device__ __forceinline__ void issue(int kb, unsigned stage) const {
        const char* const src = origin + kb * block_bytes;
#pragma unroll
        for (int q = 0; q < ROUNDS; ++q)
            asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                         : : "v"(voff[q]), "s"(src), "s"(lds0 + stage + (unsigned)(q * NTH * 16)) : "memory", "m0");
    }
    // the 32x32x16 fragment: lane holds k = kk + 8 (lane >> 5) .. + 8 of row
    // base + (lane & 31) -- one 16-byte read from [row][k], or two
    // transposing reads from [k][row] (16-lane group g takes the 16 rows from
    // base + 16 (g & 1), k from kk + 8 (g >> 1))
    __device__ static __forceinline__ u16x8 frag(const unsigned char* xs, int base, int kk, int lane) {
        if constexpr (KCONTIG) {
            const int r = base + (lane & 31), c = (kk >> 3) + (lane >> 5);
            return *(const u16x8*)(xs + (r * 8 + (c ^ swz(r))) * 16);
        } else {
            const int L = lane & 15, g = lane >> 4;
            const int r = kk + 8 * (g >> 1) + (L >> 2), col = base + 16 * (g & 1) + 4 * (L & 3);
            const int off = r * ROWS * 2 + (((col >> 3) ^ swz(r)) << 4) + (col & 7) * 2;
            typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
            // k-row r + 4 has r's swizzle
            const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(xs + off));
            const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(xs + off + 4 * ROWS * 2));
            u16x8 f;
            f[0] = (unsigned short)lo[0]; f[1] = (unsigned short)lo[1]; f[2] = (unsigned short)lo[2]; f[3] = (unsigned short)lo[3];
            f[4] = (unsigned short)hi[0]; f[5] = (unsigned short)hi[1]; f[6] = (unsigned short)hi[2]; f[7] = (unsigned short)hi[3];
            return f;
        }
    }
};

// f32 operand tiles (32 k) loaded straight into LDS for the eight-wave tiles,
// in DLoader's swizzled layout (frag_dl reads them), by the same saddr-form
// inline assembly as D16Loader: the kernel waits for its own loads, so two
// k-blocks stay in flight while one is multiplied.  A tile of SLOTS chunks
// that is not a whole number of the workgroup's rounds (96 rows: 1.5) has its
// last round issued by the first SLOTS % NTH / 64 waves only, so those waves
// count one load more a block (loads_of).  Byte offsets from the uniform base
// are 32-bit: the launcher takes these tiles only for operands whose rows
// span less than 4 GiB.
template <bool KCONTIG, int ROWS, int NTH>
struct F32Loader {
    static constexpr int BK = 32;
    static constexpr int CPR = KCONTIG ? 8 : ROWS / 4;    // chunks per LDS row
    static constexpr int SLOTS = ROWS * BK / 4;           // chunks per tile
    static constexpr int FULL = SLOTS / NTH;              // rounds every wave issues
    static constexpr int PW = SLOTS % NTH / 64;           // waves issuing one round more
    static constexpr int ROUNDS = FULL + (PW > 0 ? 1 : 0);
    static constexpr int BYTES = SLOTS * 16;
    static_assert(SLOTS % 64 == 0, "whole waves a round");
    static_assert(KCONTIG || ROWS % 8 == 0, "the swizzle stays inside a k-row");
    unsigned voff[ROUNDS];
    const char* origin;
    long long block_bytes;
    unsigned lds0;
    int wave;                   // this wave's index (uniform)

    __device__ static constexpr int loads_of(bool extra) { return FULL + (extra ? 1 : 0); }
    __device__ __forceinline__ void init(const float* p, int rows, long long rs, long long ks, int row0, int k0,
                                         unsigned tile) {
        const int t = threadIdx.x;
        wave = __builtin_amdgcn_readfirstlane(t >> 6);
        origin = (const char*)(p + (KCONTIG ? (long long)k0 : (long long)k0 * ks));
        block_bytes = KCONTIG ? 4LL * BK : 4LL * BK * ks;
#pragma unroll
        for (int q = 0; q < ROUNDS; ++q) {
            const int slot = q * NTH + t;
            long long e;
            if (KCONTIG) {
                const int r = slot >> 3, kc = (slot & 7) ^ (r & 7);
                int row = row0 + r;
                row = row < rows ? row : rows - 1;
                e = row * rs + kc * 4;
            } else {
                const int k = slot / CPR, cc = (slot % CPR) ^ ((k & 1) * 4);
                int row = row0 + cc * 4;
                row = row + 4 <= rows ? row : rows - 4;
                e = k * ks + row;
            }
            voff[q] = (unsigned)(4 * e);
        }
        lds0 = __builtin_amdgcn_readfirstlane(tile + (unsigned)(t & ~63) * 16u);
    }
    __device__ __forceinline__ void issue(int kb, unsigned stage) const {
        const char* const src = origin + kb * block_bytes;
#pragma unroll
        for (int q = 0; q < ROUNDS; ++q)
            if (q < FULL || wave < PW)
                asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                             : : "v"(voff[q]), "s"(src), "s"(lds0 + stage + (unsigned)(q * NTH * 16)) : "memory", "m0");
    }
};

// wait until at most N of this thread's vector-memory operations are
// outstanding (expcnt and lgkmcnt not waited on)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One MFMA operand fragment: k = kk + (lane >> 4) * KPL .. + KPL of row
// base + (lane & 15), from a tile laid out [row][k] (KC) or [k][row].
template <int ST, bool KC, int LDX>
__device__ __forceinline__ typename St<ST>::Frag frag(const typename St<ST>::S* xs, int base, int kk, int lane) {
    typedef typename St<ST>::Frag Frag;
    if constexpr (KC) {
        return *(const Frag*)&xs[(base + (lane & 15)) * LDX + kk + (lane >> 4) * St<ST>::KPL];
    } else if constexpr (ST == kF32) {
        return xs[(kk + (lane >> 4)) * LDX + base + (lane & 15)];
    } else {
        // two transposing reads of 4 k each: lane L of a 16-lane group reads
        // k-row kb + L/4 at columns 4*(L % 4); lane i then holds k kb..kb+3
        // of column base + i
        const int L = lane & 15, r = kk + 8 * (lane >> 4) + (L >> 2), c = base + 4 * (L & 3);
        typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(xs + r * LDX + c));
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(xs + (r + 4) * LDX + c));
        Frag f;
        f[0] = (unsigned short)lo[0]; f[1] = (unsigned short)lo[1]; f[2] = (unsigned short)lo[2]; f[3] = (unsigned short)lo[3];
        f[4] = (unsigned short)hi[0]; f[5] = (unsigned short)hi[1]; f[6] = (unsigned short)hi[2]; f[7] = (unsigned short)hi[3];
        return f;
    }
}

// A 16-bit operand fragment of the 32x32x16 MFMA from a padded register-staged
// tile: k = kk + 8 * (lane >> 5) .. + 8 of row base + (lane & 31), from
// [row][k] (KC) by one 16-byte read, or from [k][row] by two transposing
// reads a 16-lane group (group g takes the 16 rows from base + 16 * (g & 1),
// k from kk + 8 * (g >> 1)).
template <bool KC, int LDX>
__device__ __forceinline__ u16x8 frag32(const unsigned short* xs, int base, int kk, int lane) {
    if constexpr (KC) {
        return *(const u16x8*)&xs[(base + (lane & 31)) * LDX + kk + (lane >> 5) * 8];
    } else {
        const int L = lane & 15;
        const int r = kk + 8 * (lane >> 5) + (L >> 2), c = base + 16 * ((lane >> 4) & 1) + 4 * (L & 3);
        typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(xs + r * LDX + c));
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(xs + (r + 4) * LDX + c));
        u16x8 f;
        f[0] = (unsigned short)lo[0]; f[1] = (unsigned short)lo[1]; f[2] = (unsigned short)lo[2]; f[3] = (unsigned short)lo[3];
        f[4] = (unsigned short)hi[0]; f[5] = (unsigned short)hi[1]; f[6] = (unsigned short)hi[2]; f[7] = (unsigned short)hi[3];
        return f;
    }
}

template <int ST>
__device__ __forceinline__ f32x16 mfma32(u16x8 a, u16x8 b, f32x16 acc) {
    if constexpr (ST == kBF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
}

template <int ST>
__device__ __forceinline__ f32x4 mfma(typename St<ST>::Frag a, typename St<ST>::Frag b, f32x4 acc);
template <>
__device__ __forceinline__ f32x4 mfma<kBF16>(u16x8 a, u16x8 b, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma<kF16>(u16x8 a, u16x8 b, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma<kF32>(float a, float b, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
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

// The stored value of an output element (as store_out computes it).
template <int ST>
__device__ __forceinline__ typename St<ST>::S round_out(float sum, bool has_bias, float bias, bool& ovf) {
    if constexpr (ST == kF32) {
        return has_bias ? sum + bias : sum;
    } else if constexpr (ST == kBF16) {
        unsigned short h = pk_f32_to_bf16(sum);
        if (has_bias) h = pk_f32_to_bf16(pk_bf16_to_f32(h) + bias);
        return h;
    } else {
        ovf |= pk_overflows_f16(sum);
        unsigned short h = pk_f32_to_f16(sum);
        if (has_bias) {
            const float v = pk_f16_to_f32(h) + bias;
            ovf |= pk_overflows_f16(v);
            h = pk_f32_to_f16(v);
        }
        return h;
    }
}

template <int ST>
__device__ __forceinline__ float load_bias(const void* p, long long off) {
    if (ST == kF32) return ((const float*)p)[off];
    if (ST == kBF16) return pk_bf16_to_f32(((const unsigned short*)p)[off]);
    return pk_f16_to_f32(((const unsigned short*)p)[off]);
}

// Wait until the k-block a stage is about to be read from has landed, with
// `later` blocks issued after it (NL loads a thread each) still in flight.
template <int NL, int L>
__device__ __forceinline__ void wait_blocks(int later) {
    if constexpr (L == 0) {
        wait_vm<0>();
    } else {
        if (later >= L) wait_vm<L * NL>();
        else wait_blocks<NL, L - 1>(later);
    }
}

// Blocks kt .. kt + sizeof(I) - 1 in stages I (straight-line, so that the
// accumulators stay in place); the tail takes only the blocks below n.
template <typename F, int... I>
__device__ __forceinline__ void stage_round(F& f, int kt, std::integer_sequence<int, I...>) {
    (f(kt + I, std::integral_constant<int, I>{}), ...);
}
template <typename F, int... I>
__device__ __forceinline__ void stage_tail(F& f, int kt, int n, std::integer_sequence<int, I...>) {
    ((kt + I < n ? f(kt + I, std::integral_constant<int, I>{}) : void()), ...);
}

// Workgroups of NW waves (4, or 8: two a SIMD), WAN of them along the tile's
// columns, each wave WM x WN MFMA tiles of MF x MF.
template <int ST, bool AK, bool BK_, int WM, int WN, bool SAFE, bool DL, int MF, int NW = 4, int WAN = 2>
__global__ void __launch_bounds__(64 * NW) gemm_kernel(GemmArgs g) {
    static_assert(!DL || !SAFE, "direct loads: whole vectors");
    static_assert(MF == 16 || ST != kF32, "32x32 tiles: 16-bit storage");
    constexpr bool D16 = DL && MF == 32;
    // f32 eight-wave tiles (two waves a SIMD): operands straight into LDS,
    // three stages deep like the 16-bit ones
    constexpr bool F8 = ST == kF32 && DL && MF == 16 && NW == 8;
    static_assert(NW == 4 || D16 || F8, "eight waves: tiles loaded straight into LDS");
    constexpr int NTH = 64 * NW, WAM = NW / WAN;
    // f32 storage: the MFMAs take the operands' roles exchanged (D = B^T A^T,
    // the same products over the same k-steps, so the same sums bit for
    // bit), and a lane then holds four consecutive columns of one output
    // row, which leave as one 16-byte store straight from the registers
    constexpr bool SWAP = ST == kF32 && MF == 16;
    typedef typename St<ST>::S S;
    typedef typename St<ST>::Frag Frag;
    typedef typename std::conditional<MF == 32, f32x16, f32x4>::type Acc;
    constexpr int BK = St<ST>::BK, LD = BK + St<ST>::PAD, KSTEP = MF == 32 ? 16 : St<ST>::KSTEP, KPL = St<ST>::KPL;
    constexpr int BM = WAM * WM * MF, BN = WAN * WN * MF;
    // LDS: the double-buffered operand tiles, reused by the epilogue for the
    // tile's f32 sums
    typedef Loader<ST, AK, BM> LA;
    typedef Loader<ST, BK_, BN> LB;
    typedef DLoader<AK, BM> DA;
    typedef DLoader<BK_, BN> DB;
    constexpr int ASZ = DL ? DA::SIZE : LA::SIZE, BSZ = DL ? DB::SIZE : LB::SIZE;
    constexpr int LDA = AK ? LD : LA::LDR, LDB = BK_ ? LD : LB::LDR;
    constexpr int CLD = BN + 4;
    typedef typename std::conditional<F8, F32Loader<AK, BM, NTH>, D16Loader<AK, BM, NTH>>::type QA;
    typedef typename std::conditional<F8, F32Loader<BK_, BN, NTH>, D16Loader<BK_, BN, NTH>>::type QB;
    constexpr int STAGE = QA::BYTES + QB::BYTES;
    // straight-into-LDS stages: three where they fit (256 x 128 tiles, 144 KB),
    // else two (256 x 256, 128 KB); two for 128-row tiles (64 or 48 KB), so
    // that two workgroups share a CU
    // f32 eight-wave tiles: as many stages as fit, at most four (128 x 128: 4
    // x 32 KB; 256 x 128 and 256 x 96: 3 x 48 and 3 x 44 KB), but two for
    // 128 x 96 (2 x 28 KB: two workgroups a CU, four waves a SIMD)
    // 16-bit: two stages for four-wave 128-row tiles (two workgroups a CU),
    // four for eight-wave ones (one a CU), else three where they fit
    constexpr int NS = F8 ? (BM == 128 && BN == 96 ? 2 : 4 * STAGE <= 150 * 1024 ? 4 : 3)
                          : BM == 128 ? (NW == 8 ? 4 : 2) : 3 * STAGE <= 150 * 1024 ? 3 : 2;
    // the epilogue stages the tile's f32 sums in LDS whole, or in two halves
    // of rows when the whole would not fit beside nothing else (256 x 256)
    constexpr int EH = BM * CLD * 4 <= 150 * 1024 ? 1 : 2, EROWS = BM / EH;
    constexpr int OPER = D16 || F8 ? NS * STAGE : 2 * (ASZ + BSZ) * (int)sizeof(S), CTILE = EROWS * CLD * 4;
    static_assert(EH == 1 || (WM * MF) % EROWS == 0, "each wave's rows lie in one half");
    // (the exchanged-roles f32 tiles store their sums from the registers)
    __shared__ __attribute__((aligned(16))) char smem[SWAP || OPER > CTILE ? OPER : CTILE];
    S* const As0 = (S*)smem;
    S* const Bs0 = As0 + 2 * ASZ;

    // Work order.  The grid is one line of (split, batch, tile) items.  The
    // hardware deals workgroups to the 8 XCDs round robin (id mod 8).  Each
    // XCD is given one contiguous run of items, so the tiles of one batch
    // entry and neighbouring row-tiles share its L2 -- but for the four-wave
    // tiles with a k-split, whose k-ranges' panels outgrow an L2, spreading
    // each range over all XCDs measures faster: their items go in plain
    // order.  (The eight-wave split tiles, one workgroup a CU and each XCD's
    // tiles streaming one k-range together, keep the runs: 1-3 % faster in
    // f32, up to 20 % in bf16.)  Within a run, tiles go GROUP row-tiles at a
    // time across the columns, so that concurrent tiles share A rows: 8 for
    // 128-row tiles (64 a XCD at once, 8 x 8), 4 for 256-row ones (32 at
    // once: 4 x 8, a block of the output as tall as it is wide for 256 x 128
    // tiles).
    // The arithmetic is 32-bit: the launcher keeps the items below 2^31 and
    // the plan the batch below 2^16 (64-bit divisions cost hundreds of scalar
    // instructions a wave, before the first load is issued).
    const unsigned tiles = (unsigned)g.tiles_m * (unsigned)g.tiles_n;
    const unsigned total = gridDim.x;
    const unsigned nb = (unsigned)g.batch;
    const unsigned xcd = blockIdx.x % 8, local = blockIdx.x / 8;
    const unsigned q8 = total / 8, r8 = total % 8;
    const unsigned item = g.splits > 1 && NW == 4 ? blockIdx.x : xcd * q8 + (xcd < r8 ? xcd : r8) + local;
    const unsigned tb = item / tiles;
    const int split = (int)(tb / nb);
    const unsigned batch = tb - (unsigned)split * nb;
    const unsigned bid = item - tb * tiles;
    constexpr unsigned GROUP = BM == 256 ? 4 : 8;
    const unsigned tiles_m = (unsigned)g.tiles_m;
    const unsigned group_size = GROUP * (unsigned)g.tiles_n;
    const unsigned grp = bid / group_size;
    const unsigned first_m = grp * GROUP;
    const unsigned gm = (tiles_m - first_m) < GROUP ? (tiles_m - first_m) : GROUP;
    const unsigned in_grp = bid - grp * group_size;
    const unsigned tn_idx = in_grp / gm;
    const unsigned tm_idx = first_m + (in_grp - tn_idx * gm);
    const long long m0 = (long long)tm_idx * BM, n0 = (long long)tn_idx * BN;

    // the batch entry's offsets in A, B and C, one decomposition for all three
    long long a_off = 0, b_off = 0, c_off = 0;
    {
        unsigned rest = batch;
        for (int d = g.nbatch - 1; d >= 0; --d) {
            const unsigned dim = (unsigned)g.bdim[d], q = rest / dim, i = rest - q * dim;
            rest = q;
            a_off += (long long)i * g.sa_b[d];
            b_off += (long long)i * g.sb_b[d];
            c_off += (long long)i * g.sc_b[d];
        }
    }
    const S* A = (const S*)g.A + a_off;
    const S* B = (const S*)g.B + b_off;
    // split s of S takes k-blocks [s*nkb/S, (s+1)*nkb/S)
    const unsigned nkb = (unsigned)((g.K + BK - 1) / BK), ns = (unsigned)g.splits;
    const int kbeg = (int)((unsigned)split * nkb / ns * BK);
    int kend = (int)(((unsigned)split + 1) * nkb / ns * BK);
    if (kend > (int)g.K) kend = (int)g.K;
    const int M = (int)g.M, N = (int)g.N;
    const int sa_m = (int)g.sa_m, sa_k = (int)g.sa_k, sb_k = (int)g.sb_k, sb_n = (int)g.sb_n;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave / WAN) * (WM * MF), wn = (wave % WAN) * (WN * MF);
    Acc acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = Acc{};

    const int nk = (kend - kbeg + BK - 1) / BK;
    if constexpr (D16) {
        // NS stages: blocks kt + 1 .. kt + NS - 1 stream into LDS while block
        // kt is multiplied.  The fragments of each 16-k step are read while
        // the previous step's MFMAs run; before the last step of a block, the
        // next block's first fragments are read once this thread's loads of
        // that block have landed (those of the blocks after it may still be
        // in flight) and a barrier has seen every thread's -- the barrier
        // also retires every read of the stage the next loads overwrite.
        constexpr int NL = QA::ROUNDS + QB::ROUNDS;   // loads a thread issues per block
        constexpr int LA = NS - 1;                    // blocks in flight ahead
        static_assert((LA - 1) * NL < 64, "vmcnt holds the loads in flight");
        const int nd = (kend - kbeg) / BK;            // whole blocks (the launcher checks)
        QA qa;
        QB qb;
        unsigned char* const st0 = (unsigned char*)smem;
        const unsigned lds = (unsigned)(size_t)(lds_void_t*)st0;
        qa.init((const unsigned short*)A, M, sa_m, sa_k, (int)m0, kbeg, lds);
        qb.init((const unsigned short*)B, N, sb_n, sb_k, (int)n0, kbeg, lds + QA::BYTES);
        auto fetch = [&](int kb, int s) {
            qa.issue(kb, (unsigned)(s * STAGE));
            qb.issue(kb, (unsigned)(s * STAGE));
        };
        u16x8 a[WM], b[WN];
        auto read = [&](const unsigned char* st, int kk) {
#pragma unroll
            for (int i = 0; i < WM; ++i) a[i] = QA::frag(st, wm + i * 32, kk, lane);
#pragma unroll
            for (int j = 0; j < WN; ++j) b[j] = QB::frag(st + QA::BYTES, wn + j * 32, kk, lane);
        };
        if (nd > 0) {
            const int pre = nd < LA ? nd : LA;
            for (int kb = 0; kb < pre; ++kb) fetch(kb, kb);
            wait_blocks<NL, LA - 1>(pre - 1);
            __syncthreads();
            read(st0, 0);
        }
        auto block = [&](int kt, auto stage) {
            constexpr int S = decltype(stage)::value;
            if (kt + LA < nd) fetch(kt + LA, (S + LA) % NS);
            const unsigned char* const st = st0 + S * STAGE;
#pragma unroll
            for (int kk = 0; kk < BK; kk += KSTEP) {
                u16x8 ca[WM], cb[WN];
#pragma unroll
                for (int i = 0; i < WM; ++i) ca[i] = a[i];
#pragma unroll
                for (int j = 0; j < WN; ++j) cb[j] = b[j];
                if (kk + KSTEP < BK) {
                    read(st, kk + KSTEP);
                } else if (kt + 1 < nd) {
                    const int last = kt + LA < nd - 1 ? kt + LA : nd - 1;   // the last block issued
                    wait_blocks<NL, LA - 1>(last - (kt + 1));
                    __syncthreads();
                    read(st0 + ((S + 1) % NS) * STAGE, 0);
                }
                // the reads stay ahead of this step's MFMAs (the scheduler
                // would otherwise pair each read with the MFMA that uses it)
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int j = 0; j < WN; ++j) acc[i][j] = mfma32<ST>(ca[i], cb[j], acc[i][j]);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        // whole rounds of the stages, then the last blocks
        int kt = 0;
        for (; kt + NS <= nd; kt += NS) stage_round(block, kt, std::make_integer_sequence<int, NS>{});
        stage_tail(block, kt, nd, std::make_integer_sequence<int, NS - 1>{});
    } else if constexpr (F8) {
        // The 16-bit stages' order of loads, waits and barriers over 32-deep
        // f32 blocks: blocks kt + 1 .. kt + NS - 1 (two or three) stream into
        // LDS while block kt is multiplied; each 4-k step's fragments are
        // read while the previous step's MFMAs run.  A's tile is whole rounds of loads; a
        // 96-row B tile's last round is issued by the first waves only, which
        // then count one load more a block.
        static_assert(QA::PW == 0, "A: whole rounds");
        constexpr int NLL = QA::FULL + QB::FULL, NLH = NLL + (QB::PW > 0 ? 1 : 0);
        constexpr int LA = NS - 1;
        static_assert((LA - 1) * NLH < 64, "vmcnt holds the loads in flight");
        const int nd = (kend - kbeg) / BK;
        QA qa;
        QB qb;
        unsigned char* const st0 = (unsigned char*)smem;
        const unsigned lds = (unsigned)(size_t)(lds_void_t*)st0;
        qa.init((const float*)A, M, sa_m, sa_k, (int)m0, kbeg, lds);
        qb.init((const float*)B, N, sb_n, sb_k, (int)n0, kbeg, lds + QA::BYTES);
        auto fetch = [&](int kb, int s) {
            qa.issue(kb, (unsigned)(s * STAGE));
            qb.issue(kb, (unsigned)(s * STAGE));
        };
        auto wait_for = [&](int later) {
            if (NLH != NLL && qb.wave < QB::PW) wait_blocks<NLH, LA - 1>(later);
            else wait_blocks<NLL, LA - 1>(later);
        };
        float a[WM], b[WN];
        auto read = [&](const unsigned char* st, int kk) {
#pragma unroll
            for (int i = 0; i < WM; ++i) a[i] = frag_dl<AK, BM>((const float*)st, wm + i * 16, kk, lane);
#pragma unroll
            for (int j = 0; j < WN; ++j) b[j] = frag_dl<BK_, BN>((const float*)(st + QA::BYTES), wn + j * 16, kk, lane);
        };
        if (nd > 0) {
            const int pre = nd < LA ? nd : LA;
            for (int kb = 0; kb < pre; ++kb) fetch(kb, kb);
            wait_for(pre - 1);
            __syncthreads();
            read(st0, 0);
        }
        auto block = [&](int kt, auto stage) {
            constexpr int S = decltype(stage)::value;
            if (kt + LA < nd) fetch(kt + LA, (S + LA) % NS);
            const unsigned char* const st = st0 + S * STAGE;
#pragma unroll
            for (int kk = 0; kk < BK; kk += KSTEP) {
                float ca[WM], cb[WN];
#pragma unroll
                for (int i = 0; i < WM; ++i) ca[i] = a[i];
#pragma unroll
                for (int j = 0; j < WN; ++j) cb[j] = b[j];
                if (kk + KSTEP < BK) {
                    read(st, kk + KSTEP);
                } else if (kt + 1 < nd) {
                    const int last = kt + LA < nd - 1 ? kt + LA : nd - 1;
                    wait_for(last - (kt + 1));
                    __syncthreads();
                    read(st0 + ((S + 1) % NS) * STAGE, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int j = 0; j < WN; ++j) acc[i][j] = mfma<ST>(cb[j], ca[i], acc[i][j]);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        int kt = 0;
        for (; kt + NS <= nd; kt += NS) stage_round(block, kt, std::make_integer_sequence<int, NS>{});
        stage_tail(block, kt, nd, std::make_integer_sequence<int, NS - 1>{});
    } else if constexpr (DL && MF == 16) {
        // One k-block ahead: block kt+1 streams into one LDS buffer while
        // block kt is multiplied out of the other; a block ends with this
        // wave's loads complete, then a barrier for every wave's.
        const DA da{};
        const DB db{};
        auto fetch = [&](int k0, int buf) {
            da.load((const float*)A, M, sa_m, sa_k, (int)m0, k0, (float*)As0 + buf * ASZ);
            db.load((const float*)B, N, sb_n, sb_k, (int)n0, k0, (float*)Bs0 + buf * BSZ);
        };
        if (nk > 0) fetch(kbeg, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        for (int kt = 0; kt < nk; ++kt) {
            const int cur = kt & 1;
            if (kt + 1 < nk) fetch(kbeg + (kt + 1) * BK, cur ^ 1);
            const float* as = (const float*)As0 + cur * ASZ;
            const float* bs = (const float*)Bs0 + cur * BSZ;
#pragma unroll
            for (int kk = 0; kk < BK; kk += KSTEP) {
                Frag a[WM], b[WN];
#pragma unroll
                for (int i = 0; i < WM; ++i) a[i] = frag_dl<AK, BM>(as, wm + i * 16, kk, lane);
#pragma unroll
                for (int j = 0; j < WN; ++j) b[j] = frag_dl<BK_, BN>(bs, wn + j * 16, kk, lane);
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int j = 0; j < WN; ++j) acc[i][j] = SWAP ? mfma<ST>(b[j], a[i], acc[i][j]) : mfma<ST>(a[i], b[j], acc[i][j]);
            }
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
    } else {
        // One k-block ahead: block kt+1 is loaded into registers while block kt
        // is multiplied out of one LDS buffer, then stored to the other.  (Two
        // blocks ahead, a second register set, measured no faster.)
        LA la;
        LB lb;
        auto fetch = [&](int k0) {
            if (SAFE) {
                la.load_checked(A, M, kend, sa_m, sa_k, (int)m0, k0);
                lb.load_checked(B, N, kend, sb_n, sb_k, (int)n0, k0);
            } else {
                la.load(A, M, kend, sa_m, sa_k, (int)m0, k0);
                lb.load(B, N, kend, sb_n, sb_k, (int)n0, k0);
            }
        };
        if (nk > 0) {
            fetch(kbeg);
            la.store(As0);
            lb.store(Bs0);
        }
        __syncthreads();
        for (int kt = 0; kt < nk; ++kt) {
            const int cur = kt & 1;
            if (kt + 1 < nk) fetch(kbeg + (kt + 1) * BK);
            const S* as = As0 + cur * ASZ;
            const S* bs = Bs0 + cur * BSZ;
#pragma unroll
            for (int kk = 0; kk < BK; kk += KSTEP) {
                if constexpr (MF == 32) {
                    u16x8 a[WM], b[WN];
#pragma unroll
                    for (int i = 0; i < WM; ++i) a[i] = frag32<AK, LDA>((const unsigned short*)as, wm + i * 32, kk, lane);
#pragma unroll
                    for (int j = 0; j < WN; ++j) b[j] = frag32<BK_, LDB>((const unsigned short*)bs, wn + j * 32, kk, lane);
#pragma unroll
                    for (int i = 0; i < WM; ++i)
#pragma unroll
                        for (int j = 0; j < WN; ++j) acc[i][j] = mfma32<ST>(a[i], b[j], acc[i][j]);
                } else {
                    Frag a[WM], b[WN];
#pragma unroll
                    for (int i = 0; i < WM; ++i) a[i] = frag<ST, AK, LDA>(as, wm + i * 16, kk, lane);
#pragma unroll
                    for (int j = 0; j < WN; ++j) b[j] = frag<ST, BK_, LDB>(bs, wn + j * 16, kk, lane);
#pragma unroll
                    for (int i = 0; i < WM; ++i)
#pragma unroll
                        for (int j = 0; j < WN; ++j) acc[i][j] = SWAP ? mfma<ST>(b[j], a[i], acc[i][j]) : mfma<ST>(a[i], b[j], acc[i][j]);
                }
            }
            if (kt + 1 < nk) {
                la.store(As0 + (cur ^ 1) * ASZ);
                lb.store(Bs0 + (cur ^ 1) * BSZ);
            }
            __syncthreads();
        }
    }

    if constexpr (SWAP) {
        // lane holds row (lane & 15) and columns 4 (lane >> 4) .. + 3 of each
        // 16 x 16 tile; no overflow guard in f32.  A per-column bias is read
        // once a column group, for every row the lane stores.  A row's column
        // tiles are stored one after another, so that the two 64-byte halves
        // of each 128-byte line leave together (stored a column tile at a
        // time, the 256 x 128 tiles wrote 21 % more than their output)
        float* const C = (float*)g.C + c_off;
        const bool cvec = g.sc_m % 4 == 0 && (uintptr_t)C % 16 == 0;
        const bool wvec = N % 4 == 0;
        const bool has_bias = g.bias && g.splits <= 1;
        const float bscalar = has_bias && g.bias_kind == 3 ? load_bias<ST>(g.bias, 0) : 0.f;
        f32x4 bcs[WN];
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const int n = (int)n0 + wn + j * 16 + 4 * (lane >> 4);
            bcs[j] = f32x4{bscalar, bscalar, bscalar, bscalar};
            if (n < N && has_bias && g.bias_kind == 1) {
                if (n + 4 <= N && (uintptr_t)g.bias % 16 == 0) {
                    bcs[j] = *(const f32x4*)((const float*)g.bias + n);
                } else {
                    for (int e = 0; e < 4 && n + e < N; ++e) bcs[j][e] = load_bias<ST>(g.bias, n + e);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int m = (int)m0 + wm + i * 16 + (lane & 15);
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const int n = (int)n0 + wn + j * 16 + 4 * (lane >> 4);
                if (n >= N) continue;
                const bool full = n + 4 <= N;
                const f32x4 bc = bcs[j];
                f32x4 v = acc[i][j];
                if (g.splits > 1) {
                    float* w = g.work + ((long long)split * M + m) * N + n;
                    if (full && wvec) {
                        *(f32x4*)w = v;
                    } else {
                        for (int e = 0; e < 4 && n + e < N; ++e) w[e] = v[e];
                    }
                    continue;
                }
                if (has_bias) {
                    if (g.bias_kind == 2) {
                        for (int e = 0; e < 4 && n + e < N; ++e) v[e] = v[e] + load_bias<ST>(g.bias, (long long)m * N + n + e);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = v[e] + bc[e];
                    }
                }
                float* c = C + (long long)m * g.sc_m + n;
                if (full && cvec) {
                    *(f32x4*)c = v;
                } else {
                    for (int e = 0; e < 4 && n + e < N; ++e) c[e] = v[e];
                }
            }
        }
        return;
    } else {
    // The tile's sums go through LDS (lane holds column lane & 15, rows
    // 4*(lane >> 4) + r of each 16x16 tile) so that each thread then stores
    // 16 contiguous bytes of one output row.
    float* const cs = (float*)smem;
    constexpr int OV = 16 / (int)sizeof(S);  // output elements per 16-byte store
    constexpr int TPR = BN / OV, RPR = NTH / TPR;  // threads past TPR*RPR store nothing
    bool ovf = false;
    const long long cbase = c_off;
    S* C = (S*)g.C + cbase;
    const int nl = (threadIdx.x % TPR) * OV;
    const int n = (int)n0 + nl;
    const bool cvec = N % OV == 0 && g.sc_m % OV == 0 && (uintptr_t)C % 16 == 0;
    const bool wvec = N % 4 == 0;
    // a per-column bias is the same for every row this thread stores
    float bcol[OV];
#pragma unroll
    for (int e = 0; e < OV; ++e)
        bcol[e] = g.bias && g.bias_kind == 1 && g.splits <= 1 && n + e < N ? load_bias<ST>(g.bias, n + e) : 0.f;
    const float bscalar = g.bias && g.bias_kind == 3 && g.splits <= 1 ? load_bias<ST>(g.bias, 0) : 0.f;
#pragma unroll 1
    for (int h = 0; h < EH; ++h) {
    // the waves whose rows lie in this half stage their sums
    __syncthreads();
    if (EH == 1 || wm / EROWS == h) {
        const int w0 = wm - h * EROWS;
        if constexpr (MF == 32) {
            // a 32x32 tile: lane holds column lane & 31, rows 8 * (r >> 2) +
            // 4 * (lane >> 5) + (r & 3), r = 0 .. 15
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        cs[(w0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * CLD + wn + j * 32 + (lane & 31)] =
                            acc[i][j][r];
        } else {
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        cs[(w0 + i * 16 + (lane >> 4) * 4 + r) * CLD + wn + j * 16 + (lane & 15)] = acc[i][j][r];
        }
    }
    __syncthreads();
    for (int rr = threadIdx.x < TPR * RPR ? (int)threadIdx.x / TPR : EROWS; rr < EROWS; rr += RPR) {
        const int m = (int)m0 + h * EROWS + rr;
        if (m >= M || n >= N) continue;
        float v[OV];
#pragma unroll
        for (int e = 0; e < OV; e += 4) {
            const f32x4 q = *(const f32x4*)&cs[rr * CLD + nl + e];
            v[e] = q[0];
            v[e + 1] = q[1];
            v[e + 2] = q[2];
            v[e + 3] = q[3];
        }
        const bool full = n + OV <= N;
        if (g.splits > 1) {
            float* w = g.work + ((long long)split * M + m) * N + n;
            if (full && wvec) {
#pragma unroll
                for (int e = 0; e < OV; e += 4) *(f32x4*)(w + e) = f32x4{v[e], v[e + 1], v[e + 2], v[e + 3]};
            } else {
                for (int e = 0; e < OV && n + e < N; ++e) w[e] = v[e];
            }
            continue;
        }
        S out[OV];
#pragma unroll
        for (int e = 0; e < OV; ++e) {
            float b = g.bias_kind == 1 ? bcol[e] : bscalar;
            if (g.bias && g.bias_kind == 2 && n + e < N) b = load_bias<ST>(g.bias, (long long)m * N + n + e);
            out[e] = round_out<ST>(v[e], g.bias != nullptr, b, ovf);
        }
        S* c = C + (long long)m * g.sc_m + n;
        if (full && cvec) {
            typename St<ST>::V w;
            __builtin_memcpy(&w, out, 16);
            *(typename St<ST>::V*)c = w;
        } else {
            for (int e = 0; e < OV && n + e < N; ++e) c[e] = out[e];
        }
    }
    }
    if (ovf && g.flag) atomicOr(g.flag, 1u);
    }
}

// The split partial sums added in increasing split order, then the epilogue.
template <int ST>
__global__ void __launch_bounds__(256) split_reduce_kernel(GemmArgs g) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= g.M * g.N) return;
    // M * N < 2^31 (the plan's bound): 32-bit division
    const unsigned nn = (unsigned)g.N, mq = (unsigned)idx / nn;
    const long long m = mq, n = (unsigned)idx - mq * nn;
    // the partials in increasing split order, eight loads in flight
    const long long mn = g.M * g.N;
    float s = g.work[idx];
    int p = 1;
    for (; p + 8 <= g.splits; p += 8) {
        float w[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) w[q] = g.work[(long long)(p + q) * mn + idx];
#pragma unroll
        for (int q = 0; q < 8; ++q) s = s + w[q];
    }
    for (; p < g.splits; ++p) s = s + g.work[(long long)p * mn + idx];
    bool ovf = false;
    float b = 0.f;
    // an e8m15 plan keeps bias_kind but passes no bias here: its own last
    // kernel adds the bias after narrowing the sum
    if (g.bias) {
        if (g.bias_kind == 1) b = load_bias<ST>(g.bias, n);
        else if (g.bias_kind == 2) b = load_bias<ST>(g.bias, idx);
        else if (g.bias_kind == 3) b = load_bias<ST>(g.bias, 0);
    }
    store_out<ST>(g.C, m * g.sc_m + n, s, g.bias != nullptr, b, ovf);
    if (ovf && g.flag) atomicOr(g.flag, 1u);
}

// Products with K of at most two k-blocks (the attention's scores: K 64 or
// 128 in 16-bit storage, 32 or 64 in f32), both operands k-contiguous: a
// workgroup keeps its 128-row panel of A in LDS for the whole K and streams
// the 64-column tiles of B across it.  Each tile's B is loaded into
// registers while the previous tile is multiplied and stored, and the
// output leaves through the B buffer the tile has finished with (in f32 in
// two halves of 64 rows), so a workgroup's loads, MFMAs and stores overlap
// across its tiles instead of each tile paying its own prologue and
// epilogue.  The products are the 128 x 64 tiles' own: the same MFMAs
// (32x32x16 for 16-bit storage, 16x16x4 for f32) over the same k-steps in
// the same order, with the operands' roles exchanged (D = B A^T: a lane
// then holds four consecutive columns of one output row, which leave as one
// LDS write).  The launcher takes it only where every tile is whole (M %
// 128, N % 64, K a whole number of k-blocks) and no bias or split applies.
template <int ST, int NK>
__global__ void __launch_bounds__(NT) stream_kernel(GemmArgs g, int tiles_per_item, int chunks) {
    typedef typename St<ST>::S S;
    typedef Loader<ST, true, 128> LA;
    typedef Loader<ST, true, 64> LB;
    constexpr bool F32 = ST == kF32;
    constexpr int BK = St<ST>::BK, LD = LA::LD, ASZ = LA::SIZE, BSZ = LB::SIZE;
    constexpr int CLD = 64 + (F32 ? 4 : 8);           // the staged output's row stride (elements)
    constexpr int HALVES = F32 ? 2 : 1, HROWS = 128 / HALVES;
    constexpr int EPC = 16 / (int)sizeof(S), CPR = 64 / EPC;   // elements a 16-byte chunk, chunks a row
    static_assert(HROWS * CLD <= 2 * BSZ, "a tile's output (or half of it) fits the B buffer it finished with");
    static_assert(HROWS * CPR == 4 * NT, "four 16-byte chunks a thread a half");
    __shared__ __attribute__((aligned(16))) S smem[2 * ASZ + 4 * BSZ];
    S* const As = smem;                              // A's k-blocks, [2][128][LD]
    S* const Bs = smem + 2 * ASZ;                    // two buffers of B's k-blocks, [2][2][64][LD]

    // the item: a batch entry, a 128-row panel, a run of column tiles;
    // each XCD (workgroup id mod 8) takes a contiguous run of items, so the
    // panels of one batch entry share its L2 and B
    const unsigned total = gridDim.x, xcd = blockIdx.x % 8, local = blockIdx.x / 8;
    const unsigned q8 = total / 8, r8 = total % 8;
    const unsigned item = xcd * q8 + (xcd < r8 ? xcd : r8) + local;
    const unsigned tiles_m = (unsigned)(g.M / 128), tiles_n = (unsigned)(g.N / 64);
    const unsigned chunk = item % (unsigned)chunks, panel = item / (unsigned)chunks;
    const unsigned tm = panel % tiles_m, batch = panel / tiles_m;
    long long a_off = 0, b_off = 0, c_off = 0;
    {
        unsigned rest = batch;
        for (int d = g.nbatch - 1; d >= 0; --d) {
            const unsigned dim = (unsigned)g.bdim[d], q = rest / dim, i = rest - q * dim;
            rest = q;
            a_off += (long long)i * g.sa_b[d];
            b_off += (long long)i * g.sb_b[d];
            c_off += (long long)i * g.sc_b[d];
        }
    }
    const S* A = (const S*)g.A + a_off;
    const S* B = (const S*)g.B + b_off;
    S* C = (S*)g.C + c_off;
    const int M = (int)g.M, N = (int)g.N, K = (int)g.K;
    const int sa_m = (int)g.sa_m, sb_n = (int)g.sb_n;
    const int m0 = (int)tm * 128;
    const unsigned t_first = chunk * (unsigned)tiles_per_item;
    const unsigned t_end = t_first + (unsigned)tiles_per_item < tiles_n ? t_first + (unsigned)tiles_per_item : tiles_n;
    if (t_first >= t_end) return;                    // the whole workgroup: no barrier is skipped by some threads
    // the item's tiles from a rotated start (panel p begins at its p-th
    // tile): workgroups that run side by side then write different column
    // blocks of their rows rather than all the same 128-byte strip of every
    // row at once
    const unsigned cnt = t_end - t_first, rot = panel % cnt;
    auto tile_of = [&](unsigned i) { return t_first + (i + rot) % cnt; };

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 32;

    // A's panel, and the first tile's B, once
    {
        LA la;
        LB lb;
#pragma unroll
        for (int kb = 0; kb < NK; ++kb) {
            la.load(A, M, K, sa_m, 1, m0, kb * BK);
            la.store(As + kb * ASZ);
            lb.load(B, N, K, sb_n, 1, (int)tile_of(0) * 64, kb * BK);
            lb.store(Bs + kb * BSZ);
        }
    }
    __syncthreads();

    bool ovf = false;
    LB next[NK];
    for (unsigned i = 0; i < cnt; ++i) {
        const unsigned t = tile_of(i);
        const int cur = (int)(i & 1);
        S* const bcur = Bs + cur * 2 * BSZ;
        const bool more = i + 1 < cnt;
        if (more) {
#pragma unroll
            for (int kb = 0; kb < NK; ++kb) next[kb].load(B, N, K, sb_n, 1, (int)tile_of(i + 1) * 64, kb * BK);
        }
        // 16-bit: acc16[i] holds output row wm + 32 i + (lane & 31), columns
        // wn + 8 q + 4 (lane >> 5) + e at element 4 q + e; f32: acc32[i][j]
        // row wm + 16 i + (lane & 15), columns wn + 16 j + 4 (lane >> 4) + e
        f32x16 acc16[2] = {f32x16{}, f32x16{}};
        f32x4 acc32[4][2] = {};
#pragma unroll
        for (int kb = 0; kb < NK; ++kb) {
            const S* as = As + kb * ASZ;
            const S* bs = bcur + kb * BSZ;
            if constexpr (F32) {
#pragma unroll
                for (int kk = 0; kk < BK; kk += 4) {
                    float bf[2], af[4];
#pragma unroll
                    for (int j = 0; j < 2; ++j) bf[j] = frag<ST, true, LD>(bs, wn + 16 * j, kk, lane);
#pragma unroll
                    for (int q = 0; q < 4; ++q) af[q] = frag<ST, true, LD>(as, wm + 16 * q, kk, lane);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int j = 0; j < 2; ++j) acc32[q][j] = mfma<ST>(bf[j], af[q], acc32[q][j]);
                }
            } else {
#pragma unroll
                for (int kk = 0; kk < BK; kk += 16) {
                    const u16x8 b = frag32<true, LD>((const unsigned short*)bs, wn, kk, lane);
                    const u16x8 a0 = frag32<true, LD>((const unsigned short*)as, wm, kk, lane);
                    const u16x8 a1 = frag32<true, LD>((const unsigned short*)as, wm + 32, kk, lane);
                    acc16[0] = mfma32<ST>(b, a0, acc16[0]);
                    acc16[1] = mfma32<ST>(b, a1, acc16[1]);
                }
            }
        }
        // the tile's outputs, rounded, through the B buffer, half by half
        S* const cs = bcur;
        const int n0 = (int)t * 64;
#pragma unroll
        for (int h = 0; h < HALVES; ++h) {
            __syncthreads();                         // every wave is done with this tile's B (or the last half's reads)
            if (HALVES == 1 || wm / HROWS == h) {
                if constexpr (F32) {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            *(f32x4*)&cs[(wm - h * HROWS + 16 * q + (lane & 15)) * CLD + wn + 16 * j + 4 * (lane >> 4)] = acc32[q][j];
                } else {
#pragma unroll
                    for (int q2 = 0; q2 < 2; ++q2)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            u16x4 w;
#pragma unroll
                            for (int e = 0; e < 4; ++e) w[e] = round_out<ST>(acc16[q2][4 * q + e], false, 0.f, ovf);
                            *(u16x4*)&cs[(wm + 32 * q2 + (lane & 31)) * CLD + wn + 8 * q + 4 * (lane >> 5)] = w;
                        }
                }
            }
            __syncthreads();
            // 16 contiguous bytes of one output row a thread, four chunks
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = threadIdx.x + u * NT, row = c / CPR, col = (c % CPR) * EPC;
                *(uint4*)&C[(long long)(m0 + h * HROWS + row) * g.sc_m + n0 + col] = *(const uint4*)&cs[row * CLD + col];
            }
        }
        if (more) {
            // the next tile's B into the other buffer (its last reads, the
            // previous tile's outputs, finished before the barriers above)
            S* const bnext = Bs + (cur ^ 1) * 2 * BSZ;
#pragma unroll
            for (int kb = 0; kb < NK; ++kb) next[kb].store(bnext + kb * BSZ);
        }
        __syncthreads();
    }
    if (ovf && g.flag) atomicOr(g.flag, 1u);
}

// every batch entry's output starts on a 16-byte boundary
bool sc_b_whole(const GemmArgs& g) {
    for (int d = 0; d < g.nbatch; ++d)
        if (g.sc_b[d] % 8) return false;
    return true;
}

// Whether stream_kernel computes `g` (the tiles the plan chose, every tile
// whole, at most two k-blocks, k-contiguous aligned operands, no bias, no
// split, a 16-byte aligned output)
bool stream_fits(const GemmArgs& g) {
    const int bk = g.storage == kF32 ? St<kF32>::BK : St<kBF16>::BK;
    return g.stream && g.bm == 128 && g.bn == 64 && g.splits <= 1 && !g.bias &&
           g.a_kcontig && g.b_kcontig && g.a_vec && g.b_vec && g.K > 0 && g.K % bk == 0 && g.K <= 2 * bk &&
           g.M > 0 && g.M % 128 == 0 && g.N > 0 && g.N % 64 == 0 && g.sc_m % 8 == 0 &&
           (uintptr_t)g.C % 16 == 0 && g.batch * (g.M / 128) < 0x7fffffffLL && sc_b_whole(g);
}

template <int ST>
hipError_t stream_launch(const GemmArgs& g, hipStream_t stream) {
    const long long panels = g.batch * (g.M / 128), tiles_n = g.N / 64;
    // enough items to fill two workgroups a CU: each panel's columns split
    // into `chunks` runs where there are fewer panels than that
    long long chunks = panels >= 512 ? 1 : (512 + panels - 1) / panels;
    if (chunks > tiles_n) chunks = tiles_n;
    const long long per = (tiles_n + chunks - 1) / chunks;
    chunks = (tiles_n + per - 1) / per;
    const long long items = panels * chunks;
    if (items > 0x7fffffffLL) return hipErrorInvalidValue;
    if (g.K == St<ST>::BK)
        stream_kernel<ST, 1><<<(unsigned)items, NT, 0, stream>>>(g, (int)per, (int)chunks);
    else
        stream_kernel<ST, 2><<<(unsigned)items, NT, 0, stream>>>(g, (int)per, (int)chunks);
    return hipGetLastError();
}

template <int ST, int WM, int WN, bool SAFE, bool DL = false, int MF = 16, int NW = 4, int WAN = 2>
hipError_t launch_shape(const GemmArgs& g, hipStream_t stream) {
    const long long items = (long long)g.tiles_m * g.tiles_n * g.batch * g.splits;
    if (items <= 0) return hipSuccess;
    if (items > 0x7fffffffLL) return hipErrorInvalidValue;
    dim3 grid((unsigned)items, 1, 1);
    constexpr int T = 64 * NW;
    if (g.a_kcontig && g.b_kcontig) gemm_kernel<ST, true, true, WM, WN, SAFE, DL, MF, NW, WAN><<<grid, T, 0, stream>>>(g);
    else if (g.a_kcontig) gemm_kernel<ST, true, false, WM, WN, SAFE, DL, MF, NW, WAN><<<grid, T, 0, stream>>>(g);
    else if (g.b_kcontig) gemm_kernel<ST, false, true, WM, WN, SAFE, DL, MF, NW, WAN><<<grid, T, 0, stream>>>(g);
    else gemm_kernel<ST, false, false, WM, WN, SAFE, DL, MF, NW, WAN><<<grid, T, 0, stream>>>(g);
    return hipGetLastError();
}

template <int ST>
hipError_t launch_typed(const GemmArgs& g, hipStream_t stream) {
    // the clamped vector loads need each operand's vector axis (k when it is
    // contiguous, else the rows) to hold whole aligned vectors
    const bool fast = g.a_vec && g.b_vec;
    hipError_t e;
    if (stream_fits(g)) return stream_launch<ST>(g, stream);
    if constexpr (ST == kF32) {
    if (g.bm == 256 || g.eight) {
        // 256 x 128 or 256 x 96 tiles of eight waves (4 x 2 waves of 64 x 64
        // or 64 x 48), three stages straight into LDS, 128 x 128 ones (4 x 2
        // waves of 32 x 64) four stages deep, or 128 x 96 ones (32 x 48) two
        // stages deep, two workgroups a CU; operands that do not allow it
        // (alignment is known only here) take the four-wave 128-row tiles of
        // the same columns and split -- the same MFMAs over the same k-steps
        if (gemm_f32_wide_fits(g)) {
            if (g.bm == 256 && g.bn == 96) e = launch_shape<ST, 4, 3, false, true, 16, 8, 2>(g, stream);
            else if (g.bm == 256 && g.bn == 128) e = launch_shape<ST, 4, 4, false, true, 16, 8, 2>(g, stream);
            else if (g.bm == 128 && g.bn == 128) e = launch_shape<ST, 2, 4, false, true, 16, 8, 2>(g, stream);
            else if (g.bm == 128 && g.bn == 96) e = launch_shape<ST, 2, 3, false, true, 16, 8, 2>(g, stream);
            else return hipErrorInvalidValue;
            if (e != hipSuccess || g.splits <= 1) return e;
            split_reduce_kernel<ST><<<(unsigned)((g.M * g.N + 255) / 256), 256, 0, stream>>>(g);
            return hipGetLastError();
        }
        GemmArgs h = g;
        h.bm = 128;
        h.eight = false;
        h.tiles_m = (int)((g.M + 127) / 128);
        return launch_typed<ST>(h, stream);
    }
    }
    if (ST == kF32 && fast && g.K % St<kF32>::BK == 0) {
        // whole k-blocks of whole vectors: the f32 tiles load straight into LDS
        if (g.bn == 96) e = launch_shape<ST, 4, 3, false, ST == kF32>(g, stream);
        else if (g.bn == 64) e = launch_shape<ST, 4, 2, false, ST == kF32>(g, stream);
        else e = launch_shape<ST, 4, 4, false, ST == kF32>(g, stream);
    } else if (ST != kF32 && g.bm == 256) {
        // 256 x 128 tiles of 32x32x16 MFMAs (a wave 128 x 64), operands
        // straight into LDS (the plan takes these tiles for whole k-blocks);
        // operand pointers off 16 bytes: the same products from
        // register-staged tiles, element-wise loads
        if constexpr (ST != kF32) {
            const bool whole = fast && g.K % St<ST>::BK == 0 && (g.splits <= 1 || g.k_per_split % St<ST>::BK == 0);
            // whole k-blocks: eight waves (two a SIMD), a wave 128 x 64 of
            // the 256 x 256 tiles (2 x 4 waves) or 64 x 64 of the 256 x 128
            // ones (4 x 2); else four waves of register-staged operands
            if (g.bn == 256)
                e = whole ? launch_shape<ST, 4, 2, false, true, 32, 8, 4>(g, stream) : launch_shape<ST, 4, 4, true, false, 32>(g, stream);
            else
                e = whole ? launch_shape<ST, 2, 2, false, true, 32, 8, 2>(g, stream) : launch_shape<ST, 4, 2, true, false, 32>(g, stream);
        } else {
            e = hipErrorInvalidValue;
        }
    } else if (ST != kF32 && (g.bn == 128 || g.bn == 64)) {
        // 128 x 128 and 128 x 64 tiles of 32x32x16 MFMAs (a wave 64 x 64 or
        // 64 x 32), operands straight into LDS in two stages (two workgroups
        // a CU), or 128 x 128 tiles of eight waves (a wave 32 x 64, four
        // stages, one workgroup a CU: the split weight gradients); operands
        // off 16 bytes or partial k-blocks: the same products from
        // register-staged tiles.  Measured 10-20 % faster than the
        // register-staged 16x16x32 tiles at K 128-1536 (the course step's,
        // the MLP block's and the Llama attention scores' shapes).
        if constexpr (ST != kF32) {
            const bool whole = fast && g.K % St<ST>::BK == 0 && (g.splits <= 1 || g.k_per_split % St<ST>::BK == 0);
            if (g.bn == 128 && g.eight && whole)
                e = launch_shape<ST, 1, 2, false, true, 32, 8, 2>(g, stream);
            else if (g.bn == 128)
                e = whole ? launch_shape<ST, 2, 2, false, true, 32>(g, stream) : launch_shape<ST, 2, 2, true, false, 32>(g, stream);
            else
                e = whole ? launch_shape<ST, 2, 1, false, true, 32>(g, stream) : launch_shape<ST, 2, 1, true, false, 32>(g, stream);
        } else {
            e = hipErrorInvalidValue;
        }
    } else if (g.bn == 96) {
        e = fast ? launch_shape<ST, 4, 3, false>(g, stream) : launch_shape<ST, 4, 3, true>(g, stream);
    } else if (g.bn == 64) {
        e = fast ? launch_shape<ST, 4, 2, false>(g, stream) : launch_shape<ST, 4, 2, true>(g, stream);
    } else {
        e = fast ? launch_shape<ST, 4, 4, false>(g, stream) : launch_shape<ST, 4, 4, true>(g, stream);
    }
    if (e != hipSuccess || g.splits <= 1) return e;
    const long long n = g.M * g.N;
    split_reduce_kernel<ST><<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(g);
    return hipGetLastError();
}

__global__ void __launch_bounds__(256) e8_widen_kernel(const unsigned char* __restrict__ src, float* __restrict__ dst,
                                                       long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = pk_e8m15_to_f32(pk_ld24(src, i));
}

__global__ void __launch_bounds__(256) e8_narrow_kernel(GemmArgs g, unsigned char* __restrict__ out,
                                                        const unsigned char* __restrict__ bias) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= g.batch * g.M * g.N) return;
    const long long n = idx % g.N, m = (idx / g.N) % g.M, b = idx / (g.N * g.M);
    const long long off = batch_offset(g, b, g.sc_b) + m * g.sc_m + n;
    const float sum = ((const float*)g.C)[off];
    bool ovf = pk_overflows_e8m15(sum);
    unsigned h = pk_f32_to_e8m15(sum);
    if (bias) {
        const long long bo = g.bias_kind == 1 ? n : g.bias_kind == 2 ? m * g.N + n : 0;
        const float v = pk_e8m15_to_f32(h) + pk_e8m15_to_f32(pk_ld24(bias, bo));
        ovf |= pk_overflows_e8m15(v);
        h = pk_f32_to_e8m15(v);
    }
    pk_st24(out, off, h);
    if (ovf && g.flag) atomicOr(g.flag, 1u);
}

__global__ void __launch_bounds__(256) widen_kernel(WidenArgs w) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= w.n) return;
    float v;
    if (w.kind == 1) {
        v = pk_bf16_to_f32(((const unsigned short*)w.src)[i]);
    } else if (w.kind == 2) {
        v = pk_f16_to_f32(((const unsigned short*)w.src)[i]);
    } else if (w.kind == 3) {
        v = pk_e8m15_to_f32(pk_ld24((const unsigned char*)w.src, i));
    } else {
        // the element's scale: its index with the span axes' strides zero
        long long rest = i, s = 0;
        for (int d = w.ndims - 1; d >= 0; --d) {
            const long long q = rest / w.dims[d];
            s += (rest - q * w.dims[d]) * w.sstride[d];
            rest = q;
        }
        const int q = w.kind == 4 ? (int)((const signed char*)w.src)[i] : pk_nibble((const unsigned char*)w.src, i);
        v = (float)q * w.scales[s];
    }
    w.dst[i] = v;
}

template <int ST>
__global__ void __launch_bounds__(256) narrow16_kernel(GemmArgs g, unsigned short* __restrict__ out,
                                                       const unsigned short* __restrict__ bias) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= g.batch * g.M * g.N) return;
    const long long n = idx % g.N, m = (idx / g.N) % g.M, b = idx / (g.N * g.M);
    const long long off = batch_offset(g, b, g.sc_b) + m * g.sc_m + n;
    const float sum = ((const float*)g.C)[off];
    bool ovf = false;
    auto narrow = [&](float v) -> unsigned short {
        if (ST == kBF16) return pk_f32_to_bf16(v);
        ovf |= pk_overflows_f16(v);
        return pk_f32_to_f16(v);
    };
    auto widen = [](unsigned short h) { return ST == kBF16 ? pk_bf16_to_f32(h) : pk_f16_to_f32(h); };
    unsigned short h = narrow(sum);
    if (bias) {
        const long long bo = g.bias_kind == 1 ? n : g.bias_kind == 2 ? m * g.N + n : 0;
        h = narrow(widen(h) + widen(bias[bo]));
    }
    out[off] = h;
    if (ovf && g.flag) atomicOr(g.flag, 1u);
}

}  // namespace

hipError_t gemm_widen(const WidenArgs& w, hipStream_t stream) {
    if (w.n <= 0) return hipSuccess;
    if (w.kind < 1 || w.kind > 5 || (w.kind >= 4 && (!w.scales || w.ndims < 1 || w.ndims > 8))) return hipErrorInvalidValue;
    widen_kernel<<<(unsigned)((w.n + 255) / 256), 256, 0, stream>>>(w);
    return hipGetLastError();
}

hipError_t gemm_narrow16(const GemmArgs& g, int st, void* out, const void* bias, hipStream_t stream) {
    const long long n = g.batch * g.M * g.N;
    if (n <= 0) return hipSuccess;
    const unsigned grid = (unsigned)((n + 255) / 256);
    if (st == kBF16)
        narrow16_kernel<kBF16><<<grid, 256, 0, stream>>>(g, (unsigned short*)out, (const unsigned short*)bias);
    else if (st == kF16)
        narrow16_kernel<kF16><<<grid, 256, 0, stream>>>(g, (unsigned short*)out, (const unsigned short*)bias);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t gemm_e8_widen(const void* src, float* dst, long long n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    e8_widen_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>((const unsigned char*)src, dst, n);
    return hipGetLastError();
}

hipError_t gemm_e8_narrow(const GemmArgs& g, void* out, const void* bias, hipStream_t stream) {
    const long long n = g.batch * g.M * g.N;
    if (n <= 0) return hipSuccess;
    e8_narrow_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(g, (unsigned char*)out, (const unsigned char*)bias);
    return hipGetLastError();
}

int gemm_block_k(int storage) { return storage == kF32 ? St<kF32>::BK : St<kBF16>::BK; }
int gemm_tile_m() { return 128; }
bool gemm_f32_wide_fits(const GemmArgs& g) {
    if (g.storage != kF32 || !g.a_vec || !g.b_vec || g.K % St<kF32>::BK) return false;
    // the loads' 32-bit byte offsets from a k-block's base: rows x row stride
    // (k-contiguous), else 32 k-rows x k stride plus the rows
    auto span = [](bool kc, long long rows, long long rs, long long ks) {
        return kc ? (double)rows * (double)rs + 32.0 : 32.0 * (double)ks + (double)rows;
    };
    return 4.0 * span(g.a_kcontig, g.M, g.sa_m, g.sa_k) < 4294967296.0 &&
           4.0 * span(g.b_kcontig, g.N, g.sb_n, g.sb_k) < 4294967296.0;
}
int gemm_tile_m_of(const GemmArgs& g) { return g.bm == 256 ? 256 : 128; }

hipError_t gemm_launch(const GemmArgs& g, hipStream_t stream) {
    switch (g.storage) {
        case kF32: return launch_typed<kF32>(g, stream);
        case kBF16: return launch_typed<kBF16>(g, stream);
        case kF16: return launch_typed<kF16>(g, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace presk
