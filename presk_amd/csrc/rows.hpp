// Launch description of the row-nest class (rows.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace presk {

enum RowOp {
    kRowMean = 0, kRowSum, kSoftmax3, kSoftmax2, kMaskedSoftmax3, kMaskedSoftmax2, kCrossEntropy, kCrossEntropyVjp,
    kSumToRows
};

struct RowArgs {
    const void* x;        // [rows][n]
    const void* mask;     // i64 [mask_rows][n] (masked softmax)
    const void* y;        // i64 [rows] (cross entropy)
    const void* ct;       // [rows] (cross_entropy_vjp)
    void* out;
    unsigned* flag;
    long long rows, n, mask_rows;
    long long mask_row0;  // the mask row of row 0 (a launch over a range of rows)
    float n_real;         // n as the nest's f32 constant (mean)
    int op, storage;      // RowOp; 0 f32, 1 bf16, 2 f16
    unsigned* mbits;      // masked softmax over long rows: the mask as bits, [mask_rows][mask_words(n)]
};

hipError_t rows_launch(const RowArgs& a, hipStream_t stream);

// The mask of a masked softmax packed to bits in `mbits` (rows_mask_words(n)
// 32-bit words a mask row, bit c of a row its column c).
hipError_t rows_pack_mask(const RowArgs& a, hipStream_t stream);

// FAST mode's row nests (wrows.hip): the same nests with their sums in the
// `lanes64-tree` order and FAST mode's exponential.  wrows_ok: the shape is
// one it holds (the op, rows of at most 16 blocks a lane); wrows_vec: the
// elements of a block (the order's block width); wrows_fits: also the
// buffers' alignment for 16-byte blocks; a masked softmax needs `mbits`.
bool wrows_ok(const RowArgs& a);
int wrows_vec(const RowArgs& a);
bool wrows_fits(const RowArgs& a);
hipError_t wrows_launch(const RowArgs& a, hipStream_t stream);

// Whether a launch of these arguments reads the mask as bits (a workspace
// of mask_rows * mask_words(n) words the caller provides in `mbits`).
bool rows_need_mask_bits(const RowArgs& a);
long long rows_mask_words(long long n);

}  // namespace presk
