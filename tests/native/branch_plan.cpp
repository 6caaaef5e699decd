// A host test of the graph-branch planner (presk_amd/csrc/branches.hpp) on a
// recorded launch sequence, built with AddressSanitizer by
// tests/test_branch_plan.py.  Input (the file named by argv[1]):
//   K <id> <dtype> <lanes> <bytes>\n<kernel text of that many bytes>\n
//   S L <kernel id> <table length> <addresses...>      a launch
//   S C <src> <dst> <flag> <from> <to> <n>              an edge conversion
//   S D <key> <dst> <to> <n> <rate>                     a dropout mask
// For 2, 4 and 8 branches it checks: every step on a stream below the count;
// every wait names an earlier step on another stream; and every pair of
// steps that conflict (bytes written by one and read or written by the
// other, or the same compiled kernel) ordered by the streams' program order
// and the waits.  Exit status 0 when all hold.  With --drop-wait as argv[2]
// the checker is tested instead: each plan loses one wait that orders a
// conflicting pair, and the check must find the pair.
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "branches.hpp"

using namespace presk;

static int fail(const std::string& m) {
    std::cerr << "FAIL: " << m << "\n";
    return 1;
}

int main(int argc, char** argv) {
    if (argc < 2) return fail("usage: branch_plan <sequence file>");
    std::ifstream in(argv[1], std::ios::binary);
    if (!in) return fail("cannot open the sequence file");
    std::map<int, std::unique_ptr<Kernel>> kernels;
    std::vector<BranchStep> steps;
    std::string tag;
    while (in >> tag) {
        if (tag == "K") {
            int id, lanes;
            size_t len;
            std::string dtype;
            in >> id >> dtype >> lanes >> len;
            in.get();
            std::string text(len, '\0');
            in.read(&text[0], (std::streamsize)len);
            std::string err;
            auto k = parse_kernel(text, dtype == "-" ? "" : dtype, lanes, &err);
            if (!k) return fail("kernel " + std::to_string(id) + ": " + err);
            kernels[id] = std::move(k);
        } else if (tag == "S") {
            std::string kind;
            in >> kind;
            BranchStep st;
            if (kind == "L") {
                int id;
                size_t nb;
                in >> id >> nb;
                auto f = kernels.find(id);
                if (f == kernels.end()) return fail("step " + std::to_string(steps.size()) + ": no kernel " + std::to_string(id));
                const Kernel& k = *f->second;
                // the table length presk_hip_batch_add copies
                const size_t want = (size_t)k.flag_slot() + (k.guarded() ? 1 : 0);
                if (nb != want)
                    return fail("step " + std::to_string(steps.size()) + ": a table of " + std::to_string(nb) + " for a kernel that takes " +
                                std::to_string(want));
                st.k = &k;
                st.handle = &k;
                for (size_t i = 0; i < nb; ++i) {
                    unsigned long long a;
                    in >> a;
                    st.bufs.push_back((void*)(uintptr_t)a);
                }
            } else if (kind == "C") {
                unsigned long long src, dst, flag;
                in >> src >> dst >> flag >> st.from >> st.to >> st.n;
                st.bufs = {(void*)(uintptr_t)src, (void*)(uintptr_t)dst, (void*)(uintptr_t)flag};
            } else if (kind == "D") {
                unsigned long long key, dst;
                in >> key >> dst >> st.to >> st.n >> st.rate;
                st.bufs = {(void*)(uintptr_t)key, (void*)(uintptr_t)dst};
            } else {
                return fail("unknown step kind " + kind);
            }
            steps.push_back(std::move(st));
        } else {
            return fail("unknown record " + tag);
        }
    }
    const int n = (int)steps.size();
    if (n == 0) return fail("no steps");
    std::vector<std::vector<Span>> rd(n), wr(n);
    for (int i = 0; i < n; ++i) step_spans(steps[i], &rd[i], &wr[i]);
    const bool drop = argc > 2 && std::string(argv[2]) == "--drop-wait";
    for (int branches : {2, 4, 8}) {
        std::vector<int> lane;
        std::vector<std::vector<std::pair<int, int>>> waits;
        plan_branches(steps, branches, &lane, &waits);
        if ((int)lane.size() != n || (int)waits.size() != n) return fail("plan sizes");
        if (drop) {
            // a wait that alone orders a conflicting pair: the pair (waiter,
            // awaited) itself conflicts when the awaited step is a direct
            // dependency, which every wait of the plan is
            int j = 0;
            while (j < n && waits[j].empty()) ++j;
            if (j == n) return fail("no wait to drop");
            waits[j].erase(waits[j].begin());
        }
        // done[j][t]: the latest step of stream t finished before step j starts
        std::vector<std::vector<int>> done(n, std::vector<int>(branches, -1));
        std::vector<int> prev(branches, -1);
        int nwaits = 0, used = 0;
        for (int j = 0; j < n; ++j) {
            const int s = lane[j];
            if (s < 0 || s >= branches) return fail("step " + std::to_string(j) + " on stream " + std::to_string(s));
            used = std::max(used, s + 1);
            if (prev[s] >= 0) {
                done[j] = done[prev[s]];
                done[j][s] = prev[s];
            }
            for (const auto& w : waits[j]) {
                ++nwaits;
                if (w.first == s || w.first < 0 || w.first >= branches || w.second < 0 || w.second >= j || lane[w.second] != w.first)
                    return fail("step " + std::to_string(j) + ": a bad wait (" + std::to_string(w.first) + ", " + std::to_string(w.second) + ")");
                for (int t = 0; t < branches; ++t) done[j][t] = std::max(done[j][t], done[w.second][t]);
                done[j][w.first] = std::max(done[j][w.first], w.second);
            }
            prev[s] = j;
        }
        long conflicts = 0;
        for (int j = 0; j < n; ++j)
            for (int i = 0; i < j; ++i) {
                const bool same = steps[i].handle && steps[i].handle == steps[j].handle;
                if (!(same || spans_meet(wr[i], rd[j]) || spans_meet(wr[i], wr[j]) || spans_meet(rd[i], wr[j]))) continue;
                ++conflicts;
                if (lane[i] == lane[j]) continue;   // program order on one stream
                if (done[j][lane[i]] < i) {
                    if (drop) {
                        std::printf("branches %d: the dropped wait leaves steps %d and %d unordered: found\n", branches, i, j);
                        goto next;
                    }
                    return fail(std::to_string(branches) + " branches: step " + std::to_string(j) + " may overlap step " +
                                std::to_string(i) + ", which it depends on");
                }
            }
        if (drop) return fail(std::to_string(branches) + " branches: a dropped wait went unnoticed");
        std::printf("branches %d: %d steps on %d streams, %d waits, %ld ordered conflicts\n", branches, n, used, nwaits,
                    conflicts);
    next:;
    }
    std::printf("OK\n");
    return 0;
}
