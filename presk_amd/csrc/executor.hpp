// Internal interfaces of the executor library (libpresk_hip.so).
#pragma once

#include <hip/hip_runtime.h>

#include <memory>
#include <string>
#include <vector>

#include "hipgen.hpp"
#include "ir.hpp"

namespace presk {

// A hand-written kernel chosen for a nest (classes.hip).  `launch` enqueues it
// on `stream` over the KernelFn pointer table, for the iterations [lo, hi)
// of the nest's split loop.  `nest` is that loop's bound (`parallel_outer`,
// -1 when the nest has none: then the whole call is (0, 0)); `split` is the
// bound the plan honours partial ranges of: `nest`, or -1 when the plan
// computes only whole calls.  `work` is device memory of at least
// `workspace_bytes()` bytes (null when that is 0) that the launch may use as
// scratch: the caller provides it and keeps it until the launch has run;
// nothing in it needs to be zero, and a partial range needs no more than
// the whole.
struct ClassPlan {
    virtual ~ClassPlan() = default;
    virtual const char* kind() const = 0;
    virtual std::string order() const = 0;
    virtual hipError_t launch(void* const* bufs, int64_t lo, int64_t hi, void* work, hipStream_t stream) const = 0;
    virtual size_t workspace_bytes() const { return 0; }
    int64_t nest = -1, split = -1;

    // (first, count) of the split loop's iterations a launch covers, count
    // -1 for the whole call; false when [lo, hi) is not a range the plan runs.
    // A plan that computes only whole calls (split -1, which the kernel's
    // info reports as its split bound) takes (0, 0) as the whole call, as the
    // ABI states, whatever the nest's own bound.
    bool range(int64_t lo, int64_t hi, int64_t* first, int64_t* count) const {
        *first = 0;
        *count = -1;
        if (lo == 0 && (hi == nest || ((nest < 0 || split < 0) && hi == 0))) return true;
        if (split < 0 || lo < 0 || hi > split || lo > hi) return false;
        *first = lo;
        *count = hi - lo;
        return true;
    }
};

// The hand-written kernel for `k` under `mode` (PRESK_HIP_EXACT/FAST), or
// nullptr when the nest is left to the generic printer.
std::unique_ptr<ClassPlan> classify(const Kernel& k, int mode);

// PRESK_HIP_GEMM_TILE=<bm>x<bn>[/<splits>] (e.g. "256x256", "128x64/4"):
// the contraction tiles, and the k splits of a single-entry contraction, that
// every contraction takes where they apply, in place of the plan's choice.
// bm 128 takes bn 64, 96 or 128; bm 256 (16-bit storage, no k split) takes
// bn 128 or 256; splits 1 to 64.  Where an override does not apply (bm 256
// on f32, splits on a batched `ein`, more splits than k-blocks), that part
// is left to the plan.  False with a message when the variable is set and
// malformed; an unset or empty variable is no override (bm 0).
struct TileOverride {
    int bm = 0, bn = 0, splits = 0;
    bool eight = false;     // 128-row tiles of eight waves (128 x 128, or 128 x 96 in f32)
};
bool tile_override(TileOverride* t, std::string* err);

// The algorithmic bytes of a launch (inputs once + output once at storage
// width, crates/presk-kernel/src/cost.rs:26-95) and the contraction flops.
double kernel_bytes(const Kernel& k);
double kernel_flops(const Kernel& k);

// hiprtc build of generated source, cached by content (in memory and on disk).
bool build_code_object(const std::string& src, std::vector<char>* code, std::string* err);

// Device self-test of the scalar functions (selftest.hip).
hipError_t scalar_digest(int fn, uint64_t lo, uint64_t hi, uint64_t* digest);

}  // namespace presk
