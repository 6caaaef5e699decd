// Launch description of the token-scatter class (scatter.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace presk {

struct ScatterArgs {
    const long long* idx;  // i64 [tokens]: the table row each token reads
    const void* ct;        // [tokens][d]: the cotangent of each token's row
    void* out;             // [vocab][d]
    unsigned* flag;
    long long tokens, vocab, d;
    int storage;           // 0 f32, 1 bf16, 2 f16
};

hipError_t embed_vjp_launch(const ScatterArgs& a, hipStream_t stream);

}  // namespace presk
