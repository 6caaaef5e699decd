// The generic path: any PSK-Kernel nest printed as HIP source for gfx950 and
// built with hiprtc -- the executor's counterpart of the reference's LLVM
// backend, which prints a kernel as C and builds it with clang
// (crates/presk-llvm/src/lib.rs:240-304, after the C printer of
// crates/presk-export-c/src/lib.rs:291-369).
//
// Each printed kernel performs exactly the operations of the kernel
// interpreter (crates/presk-kernel/src/exec.rs:619-869) in the same order:
// f32 arithmetic for f32/bf16/f16/e8m15 storage, f64 for f64, exact widening
// loads, stores rounded once, the overflow guard, the fdlibm-method
// functions.  It is parallel only over loops whose iterations write disjoint
// output elements (`Kernel::parallel_at`, ir.rs:375-492) and carry no scalar
// from one iteration to the next, so every output element is computed by the
// same statements in the same order: bit-identical to the interpreter.
#pragma once

#include <string>
#include <vector>

#include "ir.hpp"

namespace presk {

constexpr int kMaxBufs = 24;

// What one launch of a printed phase needs: the parallel loops mapped to the
// grid (outermost first) and whether the outermost takes the [lo, hi) split.
struct Phase {
    std::string fn;                   // the __global__ function's name
    std::vector<int64_t> bounds;      // parallel loop bounds, outermost first (empty: one thread)
    bool split = false;               // bounds[0] is the KernelFn split loop
};

struct Generated {
    std::string src;
    std::vector<Phase> phases;
    bool fast_fns = false;            // an f32 exp or erf printed as FAST mode's function
};

// Prints `k`.  Returns false and sets `err` for a kernel the printer refuses.
// `fast_fns` (FAST mode): f32 exp and erf as pk_expf_fast / pk_erff_fast,
// whose results lie within a stated bound of the interpreter's, in place of
// its bits.
bool generate_hip(const Kernel& k, Generated* out, std::string* err, bool fast_fns = false);

// The argument block every printed phase takes (by value).
struct PhaseArgs {
    void* buf[kMaxBufs];
    unsigned* flag;
    long long lo, hi;
};

}  // namespace presk
