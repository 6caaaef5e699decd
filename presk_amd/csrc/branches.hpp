// Parallel graph branches: which steps of a recorded launch sequence may run
// side by side in one HIP graph.  Host code only, with no HIP call, so that a
// CPU test runs it under AddressSanitizer on a whole recorded sequence.
#pragma once

#include <cstdint>
#include <utility>
#include <vector>

#include "ir.hpp"

namespace presk {

// The byte range [lo, hi) of a buffer a step reads or writes.
struct Span {
    uintptr_t lo, hi;
};

// One step of the sequence, as the batch records it: a launch of a compiled
// kernel over its pointer table (`k` its IR, `handle` the compiled kernel),
// or, with no kernel, an edge conversion (bufs {src, dst, flag}, types
// `from` and `to`) or, with `rate` >= 0, a dropout mask (bufs {key, dst}).
struct BranchStep {
    const Kernel* k = nullptr;
    const void* handle = nullptr;
    std::vector<void*> bufs;
    int from = -1, to = -1;
    int64_t n = 0;
    double rate = -1.0;
};

inline size_t spec_bytes(const BufSpec& s) {
    return s.ty == Ty::Q4 ? (size_t)((s.numel() + 1) / 2) : (size_t)s.numel() * (size_t)ty_bytes(s.ty);
}

// the bytes of one element of a conversion's storage code (0 f64, 1 f32,
// 5 e8m15, else 16-bit)
inline size_t code_bytes(int t) { return t == 0 ? 8 : t == 1 ? 4 : t == 5 ? 3 : 2; }

// The bytes a step reads and writes.  The overflow flag is left out: every
// store into it writes the same nonzero word and only the host reads it,
// after the sequence, so steps that share it commute.  A launch's table
// holds its inputs, its output, then the scales of its integer inputs.
inline void step_spans(const BranchStep& it, std::vector<Span>* rd, std::vector<Span>* wr) {
    auto add = [](std::vector<Span>* v, const void* p, size_t bytes) {
        if (p && bytes) v->push_back({(uintptr_t)p, (uintptr_t)p + bytes});
    };
    if (it.k) {
        const Kernel& k = *it.k;
        for (int b = 0; b < k.out_buf(); ++b) {
            add(rd, it.bufs[b], spec_bytes(k.inputs[b]));
            const int s = k.scale_slot(b);
            if (s >= 0) add(rd, it.bufs[s], (size_t)k.inputs[b].scale_count() * sizeof(float));
        }
        add(wr, it.bufs[k.out_buf()], spec_bytes(k.output));
    } else if (it.rate >= 0.0) {
        add(rd, it.bufs[0], 32);   // the ChaCha20 key
        add(wr, it.bufs[1], (size_t)it.n * code_bytes(it.to));
    } else {
        add(rd, it.bufs[0], (size_t)it.n * code_bytes(it.from));
        add(wr, it.bufs[1], (size_t)it.n * code_bytes(it.to));
    }
}

inline bool spans_meet(const std::vector<Span>& a, const std::vector<Span>& b) {
    for (const Span& x : a)
        for (const Span& y : b)
            if (x.lo < y.hi && y.lo < x.hi) return true;
    return false;
}

// Streams for a branched capture of the sequence.  Step j depends on an
// earlier step i when one writes bytes the other reads or writes, or when
// both launch the same compiled kernel (its workspace is one per handle).
// Each step goes on the stream whose last step it depends on (no wait), else
// on an idle stream, else behind the oldest stream's last step; it then waits
// for the latest step it depends on on each other stream, unless that stream
// is already known to be done up to there.  One stream: program order.
// lane[j]: step j's stream; waits[j]: the (stream, step) pairs it waits for.
inline void plan_branches(const std::vector<BranchStep>& steps, int branches, std::vector<int>* lane,
                          std::vector<std::vector<std::pair<int, int>>>* waits) {
    const int n = (int)steps.size();
    lane->assign(n, 0);
    waits->assign(n, {});
    if (branches <= 1) return;
    std::vector<std::vector<Span>> rd(n), wr(n);
    for (int i = 0; i < n; ++i) step_spans(steps[i], &rd[i], &wr[i]);
    std::vector<int> last(branches, -1);                                             // each stream's last step
    std::vector<std::vector<int>> known(branches, std::vector<int>(branches, -1));   // known[s][t]: t done up to this step before s's end
    for (int j = 0; j < n; ++j) {
        std::vector<int> dep(branches, -1);   // the latest step j depends on, per stream
        for (int i = j - 1; i >= 0; --i) {
            const int t = (*lane)[i];
            if (dep[t] >= i) continue;
            const bool same = steps[i].handle && steps[i].handle == steps[j].handle;
            if (same || spans_meet(wr[i], rd[j]) || spans_meet(wr[i], wr[j]) || spans_meet(rd[i], wr[j])) dep[t] = i;
        }
        int s = -1;
        for (int t = 0; t < branches; ++t)   // continue the chain of the latest dependency
            if (last[t] >= 0 && last[t] == dep[t] && (s < 0 || dep[t] > dep[s])) s = t;
        if (s < 0)
            for (int t = 0; t < branches && s < 0; ++t)
                if (last[t] < 0) s = t;
        if (s < 0) {
            s = 0;
            for (int t = 1; t < branches; ++t)
                if (last[t] < last[s]) s = t;
        }
        (*lane)[j] = s;
        for (int t = 0; t < branches; ++t) {
            if (t == s || dep[t] < 0 || known[s][t] >= dep[t]) continue;
            (*waits)[j].push_back({t, dep[t]});
            known[s][t] = dep[t];
        }
        last[s] = j;
        known[s][s] = j;
    }
}

}  // namespace presk
