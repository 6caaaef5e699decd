// Launch descriptions of the reduction classes (reduce.hip, rows.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace presk {

struct ColSumArgs {
    const void* x;        // [rows][cols] in the storage type
    void* out;            // [cols]
    float* work;          // [nchunks][cols] chunk sums
    unsigned* flag;       // overflow guard (f16) or null
    long long rows, cols, chunk, nchunks;
    long long ld;         // x's row stride in elements (cols, or wider for a range of columns)
    float div;            // mean: the total divided by this (the nest's f32 count), else 0
    int storage;          // 0 f32, 1 bf16, 2 f16
    int square;           // 1: each term is x * x (rounded), `sum_squares`
};

hipError_t colsum_launch(const ColSumArgs& a, hipStream_t stream);

}  // namespace presk
