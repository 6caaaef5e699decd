// The MFMA contraction kernel's launch description (gemm.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace presk {

enum Storage { kF32 = 0, kBF16 = 1, kF16 = 2 };

struct GemmArgs {
    const void* A;        // operand 0, element (b, m, k) at A + batch + m*sa_m + k*sa_k
    const void* B;        // operand 1, element (b, k, n) at B + batch + k*sb_k + n*sb_n
    const void* bias;     // the epilogue's operand or null
    void* C;              // output, element (b, m, n) at C + batch + m*sc_m + n
    float* work;          // split-K partials [splits][M][N] (splits > 1)
    unsigned* flag;       // overflow guard (f16 output) or null
    long long M, N, K;
    long long sa_m, sa_k, sb_k, sb_n;
    long long sc_m;                 // output row stride: N, or wider when an `ein` puts batch axes inside a row
    int nbatch;                     // batch axes (outer axes of an `ein`), at most 3
    long long bdim[3], sa_b[3], sb_b[3], sc_b[3];
    long long batch;                // product of bdim
    // bias element of (m, n): kind 1 bias[n], 2 bias[m*N + n], 3 bias[0]
    int bias_kind;
    int storage;                    // Storage
    bool a_kcontig, b_kcontig;      // sa_k == 1 / sb_k == 1
    bool a_vec, b_vec;              // whole aligned 16-byte vectors along the loaded axis
    int splits;
    long long k_per_split;
    int tiles_m, tiles_n;
    int bm;                         // tile rows: 128, or 256 (eight-wave tiles)
    int bn;                         // tile columns: 256, 128, 96 or 64
    bool eight;                     // 128-row tiles of eight waves: 128 x 128, or 128 x 96 in f32 (256-row tiles always have eight)
    bool stream;                    // K of at most two k-blocks may stream B's tiles across a kept A panel
};

hipError_t gemm_launch(const GemmArgs& g, hipStream_t stream);

// e8m15 contractions (the f32 kernel on exact widenings): an e8m15 code is
// the top 24 bits of its f32, so the n codes at src widen to dst exactly
hipError_t gemm_e8_widen(const void* src, float* dst, long long n, hipStream_t stream);
// the e8m15 output of every element g's M, N and batch cover (C's layout):
// the f32 sum at g.C rounded (overflow guard at g.flag), then, with a bias,
// read back, the bias added in f32 and rounded again (lower.rs:1053-1060)
hipError_t gemm_e8_narrow(const GemmArgs& g, void* out, const void* bias, hipStream_t stream);
// Operands multiplied on the f32 kernel from f32 copies: `kind` 1 bf16 and
// 2 f16 values widened exactly, 3 e8m15 codes widened exactly, 4 int8 and 5
// int4 integer weights loaded as a Quant input is (f32(q) * s, one f32
// multiplication, crates/presk-rt/src/quant.rs:248-252), the scale of
// element ix at sum ix_a * sstride_a over the buffer's `ndims` axes.
struct WidenArgs {
    const void* src;
    float* dst;
    long long n;
    int kind;
    const float* scales;
    int ndims;
    long long dims[8], sstride[8];
};
hipError_t gemm_widen(const WidenArgs& w, hipStream_t stream);
// the bf16 or f16 (`st`) output of every element g's M, N and batch cover:
// the f32 sum at g.C stored rounded (the guard at g.flag for f16), then,
// with a bias, read back, the bias added in f32 and rounded again
// (lower.rs:1053-1060)
hipError_t gemm_narrow16(const GemmArgs& g, int st, void* out, const void* bias, hipStream_t stream);
int gemm_block_k(int storage);
int gemm_tile_m();
int gemm_tile_m_of(const GemmArgs& g);
// f32 operands the eight-wave tiles can take: whole aligned vectors, whole
// 32-deep k-blocks (a k-split's ranges are whole blocks), 32-bit byte
// offsets within a k-block
bool gemm_f32_wide_fits(const GemmArgs& g);

}  // namespace presk
