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
// on `stream` over the KernelFn pointer table.
struct ClassPlan {
    virtual ~ClassPlan() = default;
    virtual const char* kind() const = 0;
    virtual std::string order() const = 0;
    virtual hipError_t launch(void* const* bufs, int64_t lo, int64_t hi, hipStream_t stream) const = 0;
    // allocate what a full-range launch would allocate on first use (its
    // workspace), so that a recorded sequence can be captured into a graph
    virtual hipError_t prepare() const { return hipSuccess; }
};

// The hand-written kernel for `k` under `mode` (PRESK_HIP_EXACT/FAST), or
// nullptr when the nest is left to the generic printer.
std::unique_ptr<ClassPlan> classify(const Kernel& k, int mode);

// The algorithmic bytes of a launch (inputs once + output once at storage
// width, crates/presk-kernel/src/cost.rs:26-95) and the contraction flops.
double kernel_bytes(const Kernel& k);
double kernel_flops(const Kernel& k);

// hiprtc build of generated source, cached by content (in memory and on disk).
bool build_code_object(const std::string& src, std::vector<char>* code, std::string* err);

// Device self-test of the scalar functions (selftest.hip).
hipError_t scalar_digest(int fn, uint64_t lo, uint64_t hi, uint64_t* digest);

}  // namespace presk
