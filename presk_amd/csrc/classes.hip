// The recognizer: which hand-written kernel runs a nest.  A nest is matched
// by what it computes -- its primitive (the kernel's name, as the lowering
// names it, crates/presk-kernel/src/lower.rs:250-297), its buffers' shapes,
// and, where the primitive leaves the operands' roles open (`ein`), the index
// pattern of its loads -- never by its layout, since every layout point of a
// nest computes the same values (lower.rs:846-905).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <map>
#include <mutex>

#include "devfmt.hpp"
#include "executor.hpp"
#include "gemm.hpp"
#include "reduce.hpp"
#include "rows.hpp"
#include "scatter.hpp"
#include "presk_hip.h"

namespace presk {

namespace {

// `align` (lower.rs:37-55): where each axis of `src` sits in `target`.
bool align(const BufSpec& src, const BufSpec& target, std::vector<int>* out) {
    out->clear();
    if (src.dims.size() > target.dims.size()) return false;
    const size_t off = target.dims.size() - src.dims.size();
    bool positional = true;
    for (size_t i = 0; i < src.dims.size(); ++i) {
        const std::string &a = src.names[i], &t = target.names[off + i];
        if (src.dims[i] != target.dims[off + i] || !(a.empty() || t.empty() || a == t)) positional = false;
    }
    if (positional) {
        for (size_t i = 0; i < src.dims.size(); ++i) out->push_back((int)(off + i));
        return true;
    }
    for (size_t i = 0; i < src.dims.size(); ++i) {
        if (src.names[i].empty()) return false;
        int p = -1;
        for (size_t j = 0; j < target.dims.size(); ++j)
            if (target.names[j] == src.names[i] && target.dims[j] == src.dims[i]) { p = (int)j; break; }
        if (p < 0) return false;
        out->push_back(p);
    }
    return true;
}

int64_t prod(const std::vector<int64_t>& d, size_t from, size_t to) {
    int64_t p = 1;
    for (size_t i = from; i < to && i < d.size(); ++i) p *= d[i];
    return p;
}

// The operands of the product in a contraction nest's innermost statement:
// `acc = acc + x * Load(1, ix1)` with x a Load(0, ix0) or a scalar set from
// one just before.  Fills the loop variables of each load's index.
bool product_pattern(const Kernel& k, std::vector<int>* vars0, std::vector<int>* vars1, std::vector<int>* out_vars) {
    const Expr* load0 = nullptr;
    const Expr* load1 = nullptr;
    const std::vector<const Stmt*>* innermost = nullptr;
    std::function<void(const std::vector<const Stmt*>&)> walk = [&](const std::vector<const Stmt*>& body) {
        for (auto s : body) {
            if (s->kind == Stmt::For) walk(s->body);
            if (s->kind == Stmt::Store && s->buf == k.out_buf()) {
                out_vars->clear();
                for (auto e : s->index) out_vars->push_back(e->kind == Expr::Iv ? e->id : -1);
            }
        }
        for (size_t i = 0; i < body.size(); ++i) {
            const Stmt* s = body[i];
            if (s->kind != Stmt::Set || s->value->kind != Expr::Bin || s->value->op != Op::Add) continue;
            const Expr* a = s->value->kids[0];
            const Expr* m = s->value->kids[1];
            if (a->kind != Expr::Sv || a->id != s->var || m->kind != Expr::Bin || m->op != Op::Mul) continue;
            const Expr* x = m->kids[0];
            const Expr* w = m->kids[1];
            if (w->kind != Expr::Load || w->id != 1) continue;
            if (x->kind == Expr::Sv && i > 0 && body[i - 1]->kind == Stmt::Set && body[i - 1]->var == x->id &&
                body[i - 1]->value->kind == Expr::Load && body[i - 1]->value->id == 0)
                x = body[i - 1]->value;
            // the generic `ein` term (1 * x0) * x1 (lower.rs:625-630): 1*x0 is x0 exactly
            if (x->kind == Expr::Bin && x->op == Op::Mul && x->kids[0]->kind == Expr::Num && x->kids[0]->integral &&
                x->kids[0]->inum == 1)
                x = x->kids[1];
            if (x->kind != Expr::Load || x->id != 0) continue;
            load0 = x;
            load1 = w;
            innermost = &body;
        }
    };
    walk(k.body);
    if (!load0 || !load1 || !innermost) return false;
    auto vars = [](const Expr* l, std::vector<int>* v) {
        v->clear();
        for (auto e : l->kids) {
            if (e->kind != Expr::Iv) return false;
            v->push_back(e->id);
        }
        return true;
    };
    return vars(load0, vars0) && vars(load1, vars1);
}

// ---- the contraction class ---------------------------------------------------------
struct GemmPlan : ClassPlan {
    GemmArgs g{};          // pointers filled at launch
    std::string name;
    int storage = kF32;
    bool epilogue = false;
    int n_in = 2;
    bool guarded = false;
    // what one iteration of the KernelFn split loop covers: a batch entry
    // (the first batch axis), rows_per_iter rows of M, or cols_per_iter
    // columns of N (an `ein` whose first output axis is J)
    bool split_on_batch = false;
    // operands multiplied on the f32 kernel from f32 copies (e8m15 codes,
    // integer weights, and the 16-bit operand beside an integer one): conv[i]
    // the WidenArgs kind of operand i (0: used as it is), wq[i] its integer
    // layout; `narrow` the output's storage when the f32 sums are stored
    // into it afterwards (kBF16, kF16, or 3 for e8m15), else -1
    int conv[2] = {0, 0};
    WidenArgs wq[2] = {};
    int scale_slot[2] = {-1, -1};
    int narrow = -1;
    int flag_slot = 0;
    long long numel_in[2] = {0, 0}, numel_out = 0;
    bool swapped = false;          // operand 1 is A (an `ein` whose operand 1 carries I)
    long long rows_per_iter = 0;
    long long cols_per_iter = 0;

    const char* kind() const override { return "gemm"; }
    std::string order() const override {
        // 16-bit storage: 32x32x16 MFMAs (k in steps of 16) on every tile but
        // the 128 x 96 one (16x16x32, steps of 32)
        std::string o = storage == kF32 ? "mfma-f32-k4" : g.bm == 256 || g.bn != 96 ? "mfma-k16" : "mfma-k32";
        if (g.splits > 1) o += "-split" + std::to_string(g.splits);
        return o;
    }
    // the converted operands' and the output's f32 copies, each 256-byte
    // aligned; then the split-K partials, [splits][M][N] in f32
    static size_t up256(size_t n) { return (n + 255) / 256 * 256; }
    size_t wide_bytes() const {
        return (conv[0] ? up256(4 * (size_t)numel_in[0]) : 0) + (conv[1] ? up256(4 * (size_t)numel_in[1]) : 0) +
               (narrow >= 0 ? up256(4 * (size_t)numel_out) : 0);
    }
    size_t workspace_bytes() const override {
        return wide_bytes() + (g.splits > 1 ? (size_t)g.splits * (size_t)g.M * (size_t)g.N * sizeof(float) : 0);
    }

    hipError_t launch(void* const* bufs, int64_t lo, int64_t hi, void* work, hipStream_t stream) const override {
        int64_t first, count;
        if (!range(lo, hi, &first, &count)) return hipErrorInvalidValue;
        if (count == 0) return hipSuccess;
        GemmArgs a = g;
        a.A = bufs[swapped ? 1 : 0];
        a.B = bufs[swapped ? 0 : 1];
        a.bias = epilogue ? bufs[2] : nullptr;
        a.C = bufs[n_in];
        a.flag = guarded ? (unsigned*)bufs[flag_slot] : nullptr;
        // operands of other types: f32 copies (exact widenings, or the
        // integer weights' loads), the f32 kernel into an f32 copy of the
        // output where its storage is narrower, narrowed afterwards
        unsigned char* n_out = nullptr;
        const unsigned char* n_bias = nullptr;
        if (conv[0] || conv[1] || narrow >= 0) {
            if (!work) return hipErrorInvalidValue;
            char* w = (char*)work;
            const void* op[2] = {bufs[0], bufs[1]};
            for (int i = 0; i < 2; ++i) {
                if (!conv[i]) continue;
                WidenArgs x = wq[i];
                x.src = bufs[i];
                x.dst = (float*)w;
                x.n = numel_in[i];
                x.kind = conv[i];
                x.scales = conv[i] >= 4 ? (const float*)bufs[scale_slot[i]] : nullptr;
                if (hipError_t e = gemm_widen(x, stream); e != hipSuccess) return e;
                op[i] = w;
                w += up256(4 * (size_t)numel_in[i]);
            }
            a.A = op[swapped ? 1 : 0];
            a.B = op[swapped ? 0 : 1];
            if (narrow >= 0) {
                n_out = (unsigned char*)a.C;
                n_bias = (const unsigned char*)a.bias;
                a.C = w;
                a.bias = nullptr;
            }
            work = (char*)work + wide_bytes();
        }
        const int esz = storage == kF32 ? 4 : 2;
        // a partial range: the same tiles, k-blocks and split of K as the
        // whole call, over fewer batch entries, rows or columns -- each
        // element is summed by the same steps, so its bits do not change
        if (count > 0 && count < split) {
            // element offsets of the range's first output and bias elements
            long long c_off = 0, bias_off = 0;
            if (split_on_batch) {
                a.A = (const char*)a.A + first * a.sa_b[0] * esz;
                a.B = (const char*)a.B + first * a.sb_b[0] * esz;
                c_off = first * a.sc_b[0];
                a.batch = a.batch / a.bdim[0] * count;
                a.bdim[0] = count;
            } else if (cols_per_iter > 0) {
                const long long n0 = first * cols_per_iter;
                a.B = (const char*)a.B + n0 * a.sb_n * esz;
                c_off = n0;
                if (a.bias_kind == 1) bias_off = n0;
                a.N = count * cols_per_iter;
                a.tiles_n = (int)((a.N + a.bn - 1) / a.bn);
            } else {
                const long long m0 = first * rows_per_iter;
                a.A = (const char*)a.A + m0 * a.sa_m * esz;
                c_off = m0 * a.sc_m;
                if (a.bias_kind == 2) bias_off = m0 * a.N;
                a.M = count * rows_per_iter;
                a.tiles_m = (int)((a.M + gemm_tile_m_of(a) - 1) / gemm_tile_m_of(a));
            }
            a.C = (char*)a.C + c_off * esz;
            if (a.bias) a.bias = (const char*)a.bias + bias_off * esz;
            const int nsz = narrow == 3 ? 3 : 2;   // the narrowed output's element bytes
            if (n_out) n_out += nsz * c_off;
            if (n_bias) n_bias += nsz * bias_off;
        }
        // the clamped 16-byte loads need whole aligned vectors along the
        // loaded axis: k when it is contiguous, else the rows
        const int vec = storage == kF32 ? 4 : 8;
        auto aligned = [&](const void* p, bool kcontig, long long rows, long long other_stride, const long long* bs) {
            if ((uintptr_t)p % 16) return false;
            if (other_stride % vec) return false;
            if ((kcontig ? a.K : rows) % vec) return false;
            for (int d = 0; d < a.nbatch; ++d)
                if (bs[d] % vec) return false;
            return true;
        };
        a.a_vec = aligned(a.A, a.a_kcontig, a.M, a.a_kcontig ? a.sa_m : a.sa_k, a.sa_b);
        a.b_vec = aligned(a.B, a.b_kcontig, a.N, a.b_kcontig ? a.sb_n : a.sb_k, a.sb_b);
        if (a.splits > 1) {
            if (!work) return hipErrorInvalidValue;
            a.work = (float*)work;
        }
        if (narrow < 0) return gemm_launch(a, stream);
        unsigned* const flag = a.flag;
        a.flag = nullptr;
        hipError_t e = gemm_launch(a, stream);
        if (e != hipSuccess) return e;
        a.flag = flag;
        if (narrow == 3) return gemm_e8_narrow(a, n_out, n_bias, stream);
        return gemm_narrow16(a, narrow, n_out, n_bias, stream);
    }
};

int storage_of(Ty t) {
    switch (t) {
        case Ty::F32: return kF32;
        case Ty::BF16: return kBF16;
        case Ty::F16: return kF16;
        default: return -1;
    }
}

}  // namespace

bool tile_override(TileOverride* t, std::string* err) {
    *t = TileOverride{};
    const char* env = std::getenv("PRESK_HIP_GEMM_TILE");
    if (!env || !*env) return true;
    int bm = 0, bn = 0, splits = 0, used = 0;
    bool ok = std::sscanf(env, "%dx%d%n", &bm, &bn, &used) == 2;
    const char* rest = env + used;
    bool eight = false;
    if (ok && rest[0] == 'w' && rest[1] == '8') {
        eight = true;
        rest += 2;
    }
    if (ok && *rest == '/') {
        ok = std::sscanf(rest, "/%d%n", &splits, &used) == 1 && splits >= 1 && splits <= 64;
        rest += ok ? used : 0;
    }
    const bool shape = (bm == 128 && (bn == 64 || bn == 96 || bn == 128)) || (bm == 256 && (bn == 96 || bn == 128 || bn == 256));
    if (!ok || *rest != '\0' || !shape || (eight && !(bm == 128 && (bn == 128 || bn == 96)))) {
        *err = std::string("PRESK_HIP_GEMM_TILE=") + env +
               ": expected <bm>x<bn>[w8][/<splits>] with bm 128 (bn 64, 96, 128) or 256 (bn 96, 128, 256), w8 only "
               "after 128x128 or 128x96, and splits 1-64";
        return false;
    }
    *t = TileOverride{bm, bn, splits, eight};
    return true;
}

namespace {

// The override's tiles and splits where they apply to `g` (see tile_override).
void apply_override(GemmArgs& g) {
    TileOverride t;
    std::string err;
    if (!tile_override(&t, &err) || t.bm == 0) return;
    // 256-row tiles: 256 x 96 and 256 x 128 in f32, 256 x 128 and 256 x 256
    // in 16-bit storage; another storage's shape leaves the plan as it is
    if (t.bm == 256 && (g.storage == kF32 ? t.bn == 256 : t.bn == 96)) return;
    g.stream = false;     // the named tiles, not the streamed panels
    g.bm = t.bm;
    g.bn = t.bn;
    // (eight-wave 128 x 96 tiles are f32's only)
    g.eight = t.eight && (t.bn == 128 || g.storage == kF32);
    g.tiles_m = (int)((g.M + g.bm - 1) / g.bm);
    g.tiles_n = (int)((g.N + g.bn - 1) / g.bn);
    const int bk = gemm_block_k(g.storage);
    const long long nkb = (g.K + bk - 1) / bk;
    if (g.bm == 256) {
        g.splits = 1;
        g.k_per_split = g.K;
    } else if (t.splits > 0 && g.batch == 1 && t.splits <= nkb) {
        g.splits = t.splits;
        g.k_per_split = t.splits > 1 ? (nkb + t.splits - 1) / t.splits * bk : g.K;
    }
}

void plan_tiles(GemmArgs& g) {
    g.bm = 128;
    g.eight = false;
    g.stream = true;
    g.tiles_m = (int)((g.M + gemm_tile_m() - 1) / gemm_tile_m());
    long long best = -1;
    if (g.storage == kF32) {
        // tile columns: 128, 96 or 64, whichever finishes first when the
        // tiles run in rounds of 512 (two workgroups per CU) and a tile takes
        // time in proportion to its width -- N = 384 fills the CUs in 4
        // columns of 96 rather than 3 of 128, and N = 64 wastes nothing in 64
        // -- the widest on a tie (fewer operand bytes per flop)
        for (int bn : {128, 96, 64}) {
            const long long t = (long long)g.tiles_m * ((g.N + bn - 1) / bn) * g.batch;
            const long long cost = (t + 511) / 512 * bn;
            if (best < 0 || cost < best) {
                best = cost;
                g.bn = bn;
            }
        }
    } else {
        // 16-bit: 128 or 64 columns (32x32x16 MFMAs), in rounds of 512 and
        // 768 workgroups (two and three a CU by their LDS), a 128 x 64 tile
        // taking 3/4 of a 128 x 128 one's time (its A panel is the same) --
        // fitted to the course step's, the MLP block's and the Llama's
        // shapes, where this picks the faster of the two or one within 2 %
        for (int bn : {128, 64}) {
            const long long t = (long long)g.tiles_m * ((g.N + bn - 1) / bn) * g.batch;
            const long long cost = bn == 128 ? (t + 511) / 512 * 4 : (t + 767) / 768 * 3;
            if (best < 0 || cost < best) {
                best = cost;
                g.bn = bn;
            }
        }
    }
    // at most two k-blocks (the attention's K of 64 and 128): a tile is
    // mostly its prologue and epilogue, and narrower tiles, more of them,
    // balance better -- the Llama scores (32 x 2048 x 2048, K 128) 132 ->
    // 125 us, the course's (384 x 256 x 256, K 64) 26.7 -> 22.9 us in bf16
    // and 49.2 -> 46.8 us in f32
    if (g.K <= 128 && g.N > 64) g.bn = 64;
    g.tiles_n = (int)((g.N + g.bn - 1) / g.bn);
    g.splits = 1;
    g.k_per_split = g.K;
    const long long tiles = (long long)g.tiles_m * g.tiles_n * g.batch;
    const int bk = gemm_block_k(g.storage);
    // operands whose strides keep whole 16-byte vectors along the loaded
    // axis (k when contiguous, else the rows), as the tiles loaded straight
    // into LDS need (the pointers' alignment is checked at launch)
    const int vec = g.storage == kF32 ? 4 : 8;
    auto vec_strides = [&](long long other, const long long* bs) {
        if (other % vec) return false;
        for (int d = 0; d < g.nbatch; ++d)
            if (bs[d] % vec) return false;
        return true;
    };
    const bool a_rows_vec = g.a_kcontig || g.M % vec == 0, b_rows_vec = g.b_kcontig || g.N % vec == 0;
    const bool all_vec = a_rows_vec && b_rows_vec && vec_strides(g.a_kcontig ? g.sa_m : g.sa_k, g.sa_b) &&
                         vec_strides(g.b_kcontig ? g.sb_n : g.sb_k, g.sb_b);
    // fewer tiles than compute units and a long K: split K across workgroups
    // (as many splits as fill one round of two workgroups per CU, each split
    // at least 4 k-blocks; split s takes k-blocks [s*nkb/S, (s+1)*nkb/S))
    if (g.batch == 1 && tiles < 256 && g.K >= 8 * bk) {
        const long long nkb = (g.K + bk - 1) / bk;
        // Whole k-blocks and whole vectors: 128 x 128 tiles of eight waves
        // (two a SIMD, four k-blocks in flight, one workgroup a CU), as many
        // splits as fill one round of the CUs -- in f32 the course step's
        // weight gradients [384 x 1536] and [1536 x 384] over K 16384 179 ->
        // 161 us (split 7 against the four-wave tiles' 14), [384 x 384] 60 ->
        // 54 us (split 28 both); in 16-bit storage with each split at least
        // 18 k-blocks long (fewer, longer splits: the partials' round trip
        // halves), [384 x 384] 27.0 -> 23.3 us (split 14 against the
        // four-wave 128 x 64 tiles' 28), [1536 x 384] 47.3 -> 46.0 us (split
        // 7 both).  At fewer than two splits, the four-wave tiles below.
        if (g.K % bk == 0 && all_vec) {
            const long long t8 = (long long)g.tiles_m * ((g.N + 127) / 128);
            long long s8 = 256 / t8;
            const long long min_blocks = g.storage == kF32 ? 4 : 18;
            if (s8 > nkb / min_blocks) s8 = nkb / min_blocks;
            if (s8 > 64) s8 = 64;
            if (s8 > 1) {
                g.bn = 128;
                g.tiles_n = (int)((g.N + 127) / 128);
                g.eight = true;
                g.splits = (int)s8;
                g.k_per_split = (nkb + s8 - 1) / s8 * bk;
                apply_override(g);
                return;
            }
        }
        // f32 of whole k-blocks (its tiles load straight into LDS): the
        // widest tiles whenever each split still runs 16 k-blocks or more --
        // [1536 x 384] and [1152 x 384] over K 16384 measure 10-15 % faster
        // as 128 x 128 tiles split 14 and 18 ways than as 128 x 64 split 7
        // and 9; at [384 x 384] (9 k-blocks a split) the narrower tiles stay
        if (g.storage == kF32 && g.K % bk == 0 && g.bn != 128) {
            const long long t128 = (long long)g.tiles_m * ((g.N + 127) / 128);
            const long long s128 = 512 / t128 < 64 ? 512 / t128 : 64;
            if (s128 > 1 && nkb / s128 >= 16) {
                g.bn = 128;
                g.tiles_n = (int)((g.N + 127) / 128);
            }
        }
        const long long nt = (long long)g.tiles_m * g.tiles_n * g.batch;
        long long s = 512 / nt;
        if (s > nkb / 4) s = nkb / 4;
        if (s > 64) s = 64;
        // many short splits of narrow tiles: the same splits over 128-wide
        // tiles (half the workgroups, each split's panels read half as often)
        // -- [384 x 384] and [384 x 65] over K 16384 measure 2-15 % faster so
        // in f32 and bf16 (split 28 and 64)
        if (s >= 28 && g.bn != 128) {
            g.bn = 128;
            g.tiles_n = (int)((g.N + 127) / 128);
        }
        if (s > 1) {
            g.splits = (int)s;
            g.k_per_split = (nkb + s - 1) / s * bk;  // the longest split
        }
    }
    // 16-bit storage without a k-split, whole k-blocks and strides of whole
    // 16-byte vectors: 256-row tiles of eight waves (two a SIMD, one
    // workgroup a CU).  256 x 256 (a wave 128 x 64, half the operand bytes a
    // flop of a 128 x 128 tile) at K of 3072 or more where they fill three
    // rounds of the CUs -- [2048 x 4096] . [4096 x 32000] 652 -> 524 us
    // against 128 x 128 tiles; else 256 x 128 (a wave 64 x 64) at K of 768
    // or more -- the Llama projections and the MLP block's products 4-18 %
    // faster than on 128 x 128 tiles (e.g. 2048 x 4096 x 4096 80.6 -> 70.7
    // us), the course step's K of 384 not
    //
    // f32 likewise (no k-split, K of 384 or more, whole 32-deep k-blocks, N
    // of 128 or more): 256 x 128, 256 x 96 (three k-blocks deep) or 128 x 128
    // (four deep) tiles of eight waves, one workgroup a CU, whichever does
    // the least work a CU over its rounds of 256 (the larger tile on a tie),
    // where they still fill the CUs once -- the course step's [16384 x 384]
    // products 55 -> 51 us at K 384 (256 x 96) and 188 -> 169 us at K 1536,
    // [16384 x 1536] 197 -> 189 us (256 x 128), the Linear module's [4096 x
    // 1024] 88 -> 74 us (128 x 128), each the fastest of the three measured
    if (g.storage == kF32) {
        if (g.splits == 1 && g.K >= 384 && g.K % gemm_block_k(kF32) == 0 && g.N >= 128 && all_vec) {
            // {rows, columns, workgroups a CU}; on a tie the earlier
            static const int shapes[4][3] = {{256, 128, 1}, {128, 96, 2}, {256, 96, 1}, {128, 128, 1}};
            long long best_cost = -1, best_t = 0;
            int bi = 0;
            for (int i = 0; i < 4; ++i) {
                const int bm = shapes[i][0], bn = shapes[i][1], per = shapes[i][2];
                const long long t = (long long)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn) * g.batch;
                const long long slots = 256LL * per;
                const long long cost = (t + slots - 1) / slots * per * bm * bn;
                if (t >= slots && (best_cost < 0 || cost < best_cost)) {
                    best_cost = cost;
                    best_t = t;
                    bi = i;
                }
            }
            if (best_cost >= 0) {
                g.bm = shapes[bi][0];
                g.bn = shapes[bi][1];
                g.eight = g.bm == 128;
                g.tiles_m = (int)((g.M + g.bm - 1) / g.bm);
                g.tiles_n = (int)((g.N + g.bn - 1) / g.bn);
            }
            (void)best_t;
        }
        apply_override(g);
        return;
    }
    const long long t256 = (long long)((g.M + 255) / 256) * ((g.N + 255) / 256) * g.batch;
    if (g.splits == 1 && g.K >= 3072 && g.K % gemm_block_k(g.storage) == 0 && all_vec && t256 >= 768) {
        g.bm = 256;
        g.bn = 256;
        g.tiles_m = (int)((g.M + 255) / 256);
        g.tiles_n = (int)((g.N + 255) / 256);
    } else if (g.splits == 1 && g.K >= 768 && g.K % gemm_block_k(g.storage) == 0 && all_vec) {
        g.bm = 256;
        g.bn = 128;
        g.tiles_m = (int)((g.M + 255) / 256);
        g.tiles_n = (int)((g.N + 127) / 128);
    }
    apply_override(g);
}

std::unique_ptr<ClassPlan> classify_gemm(const Kernel& k) {
    const std::string& n = k.name;
    const bool is_dot = n == "dot" || n == "dot+add";
    const bool is_l = n == "dot_vjp_l", is_r = n == "dot_vjp_r";
    const bool is_ein = n.compare(0, 4, "ein[") == 0;
    if (!(is_dot || is_l || is_r || is_ein)) return nullptr;
    // e8m15 storage runs as f32 on the exact widenings of its codes; an
    // integer weight (a Quant operand) as f32 on its loads f32(q) * s, the
    // other operand widened exactly
    const bool e8 = k.dtype == Ty::E8M15;
    const bool quant = k.n_quant() > 0;
    const int own = e8 ? kF32 : storage_of(k.dtype);
    if (own < 0 || k.output.ty != k.dtype) return nullptr;
    const bool epi = n == "dot+add";
    if ((int)k.inputs.size() != (epi ? 3 : 2)) return nullptr;
    for (size_t i = 0; i < k.inputs.size(); ++i) {
        const Ty t = k.inputs[i].ty;
        // indices or widened parameters: generic; a Quant bias too
        if (t != k.dtype && !(i < 2 && ty_quant(t))) return nullptr;
        if (k.inputs[i].wide) return nullptr;
    }
    const bool wide = e8 || quant;
    const int st = wide ? kF32 : own;
    const BufSpec &x = k.inputs[0], &w = k.inputs[1], &o = k.output;
    auto p = std::make_unique<GemmPlan>();
    p->flag_slot = k.flag_slot();
    for (int i = 0; i < 2; ++i) {
        const BufSpec& b = k.inputs[i];
        if (ty_quant(b.ty)) {
            p->conv[i] = b.ty == Ty::Q8 ? 4 : 5;
            p->scale_slot[i] = k.scale_slot(i);
            const auto ss = b.scale_strides();
            if (b.dims.empty() || b.dims.size() > 8 || ss.size() != b.dims.size()) return nullptr;
            p->wq[i].ndims = (int)b.dims.size();
            for (size_t d = 0; d < b.dims.size(); ++d) {
                p->wq[i].dims[d] = b.dims[d];
                p->wq[i].sstride[d] = ss[d];
            }
        } else if (wide) {
            p->conv[i] = k.dtype == Ty::BF16 ? 1 : k.dtype == Ty::F16 ? 2 : k.dtype == Ty::E8M15 ? 3 : 0;
        }
    }
    if (wide && k.dtype != Ty::F32) p->narrow = e8 ? 3 : own;
    p->numel_in[0] = x.numel();
    p->numel_in[1] = w.numel();
    p->numel_out = o.numel();
    GemmArgs& g = p->g;
    g.storage = st;
    g.batch = 1;
    g.nbatch = 0;
    p->name = n;
    p->storage = st;
    p->epilogue = epi;
    p->n_in = (int)k.inputs.size();
    p->guarded = k.guarded();
    p->nest = parallel_outer(k);
    if (is_dot) {
        // x[outer..., I, K] . w[K, J] -> [outer..., I, J]   (Contraction::of, lower.rs:700-711)
        if (w.dims.size() != 2 || x.dims.size() < 2 || x.dims.back() != w.dims[0]) return nullptr;
        g.K = w.dims[0];
        g.N = w.dims[1];
        g.M = x.numel() / g.K;
        if (o.numel() != g.M * g.N || o.dims.back() != g.N) return nullptr;
        g.sa_m = g.K; g.sa_k = 1; g.sb_k = g.N; g.sb_n = 1; g.sc_m = g.N;
        p->rows_per_iter = x.dims.size() >= 1 ? g.M / x.dims[0] : 0;
    } else if (is_l) {
        // ct[outer..., I, N] . b[J, N]^T -> [outer..., I, J]   (lower.rs:715-726)
        if (w.dims.size() != 2 || x.dims.size() < 2 || x.dims.back() != w.dims[1]) return nullptr;
        g.K = w.dims[1];
        g.N = w.dims[0];
        g.M = x.numel() / g.K;
        if (o.numel() != g.M * g.N) return nullptr;
        g.sa_m = g.K; g.sa_k = 1; g.sb_k = 1; g.sb_n = g.K; g.sc_m = g.N;
        p->rows_per_iter = g.M / x.dims[0];
    } else if (is_r) {
        // a[lead..., I], ct[lead..., J] -> [I, J], summed over lead   (lower.rs:730-739)
        if (x.dims.size() < 2 || x.dims.size() != w.dims.size()) return nullptr;
        for (size_t i = 0; i + 1 < x.dims.size(); ++i)
            if (x.dims[i] != w.dims[i]) return nullptr;
        g.M = x.dims.back();
        g.N = w.dims.back();
        g.K = prod(x.dims, 0, x.dims.size() - 1);
        if (o.dims.size() != 2 || o.dims[0] != g.M || o.dims[1] != g.N) return nullptr;
        g.sa_m = 1; g.sa_k = g.M; g.sb_k = g.N; g.sb_n = 1; g.sc_m = g.N;
        p->rows_per_iter = 1;
    } else {
        // ein: the roles of the operands' axes from the product's index
        // pattern.  An output axis both operands carry, or one carries and
        // the other broadcasts over (stride 0), is a batch axis; J is the
        // output's last axis (unit stride), carried by one operand only (B);
        // I is the longest output axis A alone carries; the summed axes, in
        // loop order, must read as one K of uniform stride in both operands
        // (`ein[batch, seq, model](o * w)` over groups, per, hd).
        std::vector<int> v0, v1, vo;
        if (!product_pattern(k, &v0, &v1, &vo)) return nullptr;
        if (vo.empty() || v0.size() != x.dims.size() || v1.size() != w.dims.size() || vo.size() != o.dims.size())
            return nullptr;
        auto count = [](const std::vector<int>& v, int var) {
            int c = 0;
            for (int u : v) c += u == var;
            return c;
        };
        auto pos = [](const std::vector<int>& v, int var) {
            for (size_t i = 0; i < v.size(); ++i)
                if (v[i] == var) return (int)i;
            return -1;
        };
        for (const auto* vs : {&v0, &v1, &vo})
            for (int v : *vs)
                if (v < 0 || count(*vs, v) != 1) return nullptr;
        // summed axes: in both operands, not in the output
        std::vector<int> summed;
        for (int v : v0)
            if (pos(vo, v) < 0) {
                if (pos(v1, v) < 0) return nullptr;
                summed.push_back(v);
            }
        for (int v : v1)
            if (pos(vo, v) < 0 && pos(v0, v) < 0) return nullptr;
        if (summed.empty()) return nullptr;
        // the loops' nesting depth: the summed axes outermost first
        std::map<int, int> depth;
        std::function<void(const std::vector<const Stmt*>&, int)> walk = [&](const std::vector<const Stmt*>& body, int d) {
            for (auto st : body)
                if (st->kind == Stmt::For) {
                    depth.emplace(st->var, d);
                    walk(st->body, d + 1);
                }
        };
        walk(k.body, 0);
        for (int v : summed)
            if (!depth.count(v)) return nullptr;
        std::sort(summed.begin(), summed.end(), [&](int a, int b) { return depth[a] < depth[b]; });
        // operand roles: B carries J, the output's last axis
        const int vj = vo.back();
        const BufSpec* xa = &x;
        const BufSpec* wb = &w;
        std::vector<int> va = v0, vb = v1;
        bool swapped = false;
        if (pos(v0, vj) >= 0 && pos(v1, vj) < 0) {
            std::swap(va, vb);
            std::swap(xa, wb);
            swapped = true;
        }
        if (pos(vb, vj) < 0 || pos(va, vj) >= 0) return nullptr;
        p->swapped = swapped;
        const auto sa = xa->strides(), sb = wb->strides(), so = o.strides();
        if (so.back() != 1) return nullptr;
        auto len_of = [&](int v) {
            const int q = pos(vo, v);
            if (q >= 0) return (long long)o.dims[q];
            return (long long)xa->dims[pos(va, v)];
        };
        // K: the summed axes as one, each outer one's stride the next one's
        // times its length, in both operands
        for (int v : summed)
            if (xa->dims[pos(va, v)] != wb->dims[pos(vb, v)]) return nullptr;
        for (size_t i = 0; i + 1 < summed.size(); ++i) {
            const int u = summed[i], v = summed[i + 1];
            if (sa[pos(va, u)] != sa[pos(va, v)] * len_of(v) || sb[pos(vb, u)] != sb[pos(vb, v)] * len_of(v)) return nullptr;
        }
        g.K = 1;
        for (int v : summed) g.K *= len_of(v);
        g.sa_k = sa[pos(va, summed.back())];
        g.sb_k = sb[pos(vb, summed.back())];
        // I: the longest output axis of A alone (the later one on a tie)
        int vi = -1;
        for (int v : vo)
            if (pos(va, v) >= 0 && pos(vb, v) < 0 && (vi < 0 || len_of(v) >= len_of(vi))) vi = v;
        if (vi < 0) return nullptr;
        g.M = len_of(vi);
        g.N = len_of(vj);
        g.sa_m = sa[pos(va, vi)];
        g.sb_n = sb[pos(vb, vj)];
        g.sc_m = so[pos(vo, vi)];
        // batch axes in output order; length-1 axes dropped except the
        // first output axis (the KernelFn split loop), which is never merged
        // into; the others collapsed where all three strides allow it
        std::vector<long long> bd, ba, bb, bc;
        bool first_is_batch = false;
        for (size_t q = 0; q < vo.size(); ++q) {
            const int v = vo[q];
            if (v == vi || v == vj) continue;
            const long long n = o.dims[q];
            const int pa = pos(va, v), pb = pos(vb, v);
            if ((pa >= 0 && xa->dims[pa] != n) || (pb >= 0 && wb->dims[pb] != n)) return nullptr;
            const long long s_a = pa >= 0 ? sa[pa] : 0, s_b = pb >= 0 ? sb[pb] : 0, s_c = so[q];
            if (q == 0) first_is_batch = true;
            else if (n == 1) continue;
            const bool mergeable = !bd.empty() && !(first_is_batch && bd.size() == 1);
            if (mergeable && ba.back() == s_a * n && bb.back() == s_b * n && bc.back() == s_c * n) {
                bd.back() *= n;
                ba.back() = s_a;
                bb.back() = s_b;
                bc.back() = s_c;
            } else {
                bd.push_back(n);
                ba.push_back(s_a);
                bb.push_back(s_b);
                bc.push_back(s_c);
            }
        }
        if (bd.size() > 3) return nullptr;
        g.nbatch = (int)bd.size();
        for (size_t q = 0; q < bd.size(); ++q) {
            g.bdim[q] = bd[q];
            g.sa_b[q] = ba[q];
            g.sb_b[q] = bb[q];
            g.sc_b[q] = bc[q];
            g.batch *= bd[q];
        }
        // a partial range of the split loop (the first output axis): a batch
        // range, a row range, or a column range (J first)
        p->split_on_batch = first_is_batch;
        p->rows_per_iter = vo[0] == vi ? 1 : 0;
        p->cols_per_iter = !first_is_batch && vo[0] == vj ? 1 : 0;
    }
    if (epi) {
        if (g.sc_m != g.N) return nullptr;
        std::vector<int> m;
        const BufSpec& b = k.inputs[2];
        if (!align(b, o, &m)) return nullptr;
        // supported broadcasts: the bias over the last axis (J), over every axis, or a scalar
        const size_t r = o.dims.size();
        if (m.empty()) {
            g.bias_kind = 3;
        } else if (m.size() == 1 && m[0] == (int)r - 1) {
            g.bias_kind = 1;
        } else if (m.size() == r) {
            for (size_t i = 0; i < r; ++i)
                if (m[i] != (int)i) return nullptr;
            g.bias_kind = 2;
        } else {
            return nullptr;
        }
    }
    g.a_kcontig = g.sa_k == 1;
    g.b_kcontig = g.sb_k == 1;
    if (g.M <= 0 || g.N <= 0 || g.K <= 0) return nullptr;
    plan_tiles(g);
    if (g.batch > 65535 || g.splits > 65535) return nullptr;
    // 32-bit element offsets inside one batch entry
    const double lim = 2147483647.0;
    if ((double)g.M * g.N > lim || (double)g.M * g.sc_m > lim || (double)g.M * g.K > lim || (double)g.K * g.N > lim ||
        (double)x.numel() > lim || (double)w.numel() > lim) return nullptr;
    // the split loop the plan honours partial ranges of: the output's first
    // axis, as one batch entry, rows_per_iter whole rows or one column each
    const long long n0 = p->nest;
    if (n0 > 0 && !o.dims.empty() && o.dims[0] == n0) {
        if (p->split_on_batch ? g.nbatch > 0 && g.bdim[0] == n0
                              : p->cols_per_iter > 0 ? g.N == n0 && g.bias_kind != 2
                                                     : p->rows_per_iter > 0 && g.M == n0 * p->rows_per_iter)
            p->split = n0;
    }
    return p;
}

// ---- sum_to onto trailing axes, chunked order (reduce.hip) ---------------------
struct ColSumPlan : ClassPlan {
    ColSumArgs a{};
    bool guarded = false;
    int n_in = 2;
    long long cols_per_iter = 0;   // output columns one iteration of the split loop covers
    const char* kind() const override { return "colsum"; }
    // the executor's own order (a realization's order reaches contractions
    // only, crates/presk-kernel/src/lower.rs:250-303): chunks of 64 rows
    std::string order() const override { return "rows-in-chunks(" + std::to_string(a.chunk) + ")-f32"; }
    // the chunk sums, [nchunks][cols] in f32
    size_t workspace_bytes() const override { return sizeof(float) * (size_t)(a.nchunks * a.cols); }
    hipError_t launch(void* const* bufs, int64_t lo, int64_t hi, void* work, hipStream_t stream) const override {
        int64_t first, count;
        if (!range(lo, hi, &first, &count)) return hipErrorInvalidValue;
        if (count == 0) return hipSuccess;
        if (!work) return hipErrorInvalidValue;
        ColSumArgs x = a;
        const int esz = a.storage == 0 ? 4 : 2;
        x.x = bufs[0];
        x.out = bufs[n_in];
        x.flag = guarded ? (unsigned*)bufs[n_in + 1] : nullptr;
        x.work = (float*)work;
        if (count > 0 && count < split) {
            // columns [c0, c0 + count * cols_per_iter) of every row
            const long long c0 = first * cols_per_iter;
            x.x = (const char*)x.x + c0 * esz;
            x.out = (char*)x.out + c0 * esz;
            x.cols = count * cols_per_iter;
        }
        return colsum_launch(x, stream);
    }
};

std::unique_ptr<ClassPlan> classify_sum_to(const Kernel& k) {
    const int st = k.dtype == Ty::F32 ? 0 : k.dtype == Ty::BF16 ? 1 : k.dtype == Ty::F16 ? 2 : -1;
    if (st < 0 || k.inputs.empty() || k.inputs[0].ty != k.dtype || k.output.ty != k.dtype) return nullptr;
    const bool squares = k.name == "sum_squares";
    // the totals SumAll / MeanAll are the kernels `sum` and `mean` (PrimOp::name)
    if ((k.name == "sum" || k.name == "mean" || squares) && k.inputs.size() == 1 && k.output.dims.empty()) {
        // every element, as one column
        auto p = std::make_unique<ColSumPlan>();
        p->n_in = 1;
        p->a.cols = 1;
        p->a.rows = k.inputs[0].numel();
        if (p->a.rows < 256) return nullptr;
        p->a.chunk = 64;
        p->a.nchunks = (p->a.rows + p->a.chunk - 1) / p->a.chunk;
        if (p->a.nchunks > 65535) return nullptr;
        p->a.div = k.name == "mean" ? (float)(double)p->a.rows : 0.f;
        p->a.square = squares ? 1 : 0;
        p->a.storage = st;
        p->a.ld = 1;
        p->guarded = k.guarded();
        p->nest = parallel_outer(k);
        return p;
    }
    if (k.name != "sum_to" || k.inputs.size() != 2) return nullptr;
    const BufSpec &x = k.inputs[0], &o = k.output;
    std::vector<int> m;
    if (!align(o, x, &m)) return nullptr;
    // the output is x's trailing axes: out[c] = sum_r x[r][c]
    const size_t off = x.dims.size() - o.dims.size();
    for (size_t i = 0; i < m.size(); ++i)
        if (m[i] != (int)(off + i)) return nullptr;
    auto p = std::make_unique<ColSumPlan>();
    p->a.cols = o.numel();
    p->a.rows = o.numel() ? x.numel() / o.numel() : 0;
    if (p->a.rows < 256 || p->a.cols == 0) return nullptr;   // short sums: the interpreter's order is fast enough
    p->a.chunk = 64;
    p->a.nchunks = (p->a.rows + p->a.chunk - 1) / p->a.chunk;
    if (p->a.nchunks > 65535) return nullptr;  // one grid row per chunk
    p->a.storage = st;
    p->a.ld = p->a.cols;
    p->guarded = k.guarded();
    // the split loop runs over the output's first axis, each iteration a
    // run of whole trailing columns
    p->nest = parallel_outer(k);
    if (p->nest > 0 && o.dims[0] == p->nest && p->a.cols % p->nest == 0) {
        p->split = p->nest;
        p->cols_per_iter = p->a.cols / p->nest;
    }
    return p;
}

// ---- row nests in the interpreter's order (rows.hip) ---------------------------
struct RowPlan : ClassPlan {
    RowArgs a{};
    int n_in = 1;
    bool guarded = false;
    long long rows_per_iter = 0;   // rows one iteration of the split loop covers
    bool row_out = false;          // one output element a row (a sum, a mean, a loss)
    // FAST: the sums in the `lanes64-tree` order over blocks of `vec`
    // elements and FAST mode's exponential (wrows.hip)
    bool fast = false;
    int vec = 1;
    const char* kind() const override { return "rows"; }
    std::string order() const override {
        if (!fast) return "sequential";
        const bool exps = a.op != kRowMean && a.op != kRowSum && a.op != kSumToRows;
        return "lanes64x" + std::to_string(vec) + "-tree" + (exps ? "+fast-exp" : "");
    }
    bool masked() const { return a.op == kMaskedSoftmax3 || a.op == kMaskedSoftmax2; }
    // the mask as bits (masked softmax over long rows, and every masked
    // softmax in FAST), [mask_rows][words]
    size_t workspace_bytes() const override {
        return rows_need_mask_bits(a) || (fast && masked() && a.rows > 0)
                   ? (size_t)a.mask_rows * rows_mask_words(a.n) * sizeof(unsigned)
                   : 0;
    }
    hipError_t launch(void* const* bufs, int64_t lo, int64_t hi, void* work, hipStream_t stream) const override {
        int64_t first, count;
        if (!range(lo, hi, &first, &count)) return hipErrorInvalidValue;
        if (count == 0) return hipSuccess;
        RowArgs x = a;
        const int esz = a.storage == 0 ? 4 : 2;
        x.x = bufs[0];
        if (a.op == kMaskedSoftmax3 || a.op == kMaskedSoftmax2) x.mask = bufs[1];
        if (a.op == kCrossEntropy || a.op == kCrossEntropyVjp) x.y = bufs[1];
        if (a.op == kCrossEntropyVjp) x.ct = bufs[2];
        x.out = bufs[n_in];
        x.flag = guarded ? (unsigned*)bufs[n_in + 1] : nullptr;
        if (count > 0 && count < split) {
            // rows [r0, r0 + count * rows_per_iter): the mask row of row r is
            // still r mod mask_rows
            const long long r0 = first * rows_per_iter;
            x.rows = count * rows_per_iter;
            x.x = (const char*)x.x + r0 * a.n * esz;
            x.out = (char*)x.out + (row_out ? r0 : r0 * a.n) * esz;
            if (x.y) x.y = (const long long*)x.y + r0;
            if (x.ct) x.ct = (const char*)x.ct + r0 * esz;
            if (a.mask_rows > 0) x.mask_row0 = r0 % a.mask_rows;
        }
        if (fast && wrows_fits(x)) {
            x.mbits = masked() ? (unsigned*)work : nullptr;
            if (masked() && !work) return hipErrorInvalidValue;
            return wrows_launch(x, stream);
        }
        x.mbits = rows_need_mask_bits(x) ? (unsigned*)work : nullptr;
        if (rows_need_mask_bits(x) && !work) return hipErrorInvalidValue;
        return rows_launch(x, stream);
    }
};

std::unique_ptr<ClassPlan> classify_rows(const Kernel& k, bool fast) {
    const int st = k.dtype == Ty::F32 ? 0 : k.dtype == Ty::BF16 ? 1 : k.dtype == Ty::F16 ? 2 : -1;
    if (st < 0 || k.inputs.empty() || k.inputs[0].ty != k.dtype || k.inputs[0].dims.empty()) return nullptr;
    const BufSpec& x = k.inputs[0];
    const std::string& n = k.name;
    auto p = std::make_unique<RowPlan>();
    p->a.storage = st;
    p->n_in = (int)k.inputs.size();
    p->guarded = k.guarded();
    p->a.n = x.dims.back();
    p->a.rows = p->a.n ? x.numel() / p->a.n : 0;
    p->a.n_real = (float)(double)p->a.n;
    // the reduced or normalized axis must be the last, by name
    auto last_axis = [&](const std::string& prefix, std::string* rest) {
        if (n.compare(0, prefix.size(), prefix) != 0) return false;
        // "<axis>", "<axis> where", "<axis>, two passes", "<axis> where, two passes"
        const std::string ax = n.substr(prefix.size());
        const size_t c = ax.find_first_of(" ,");
        const std::string name = c == std::string::npos ? ax : ax.substr(0, c);
        *rest = ax.substr(name.size());
        return !x.names.back().empty() && x.names.back() == name;
    };
    std::string rest;
    if ((n == "mean" || n == "sum") && k.inputs.size() == 1 && k.output.dims.empty()) {
        // every element as one row, summed in index order (lower.rs:1221-1233)
        p->a.rows = 1;
        p->a.n = x.numel();
        p->a.n_real = (float)(double)p->a.n;
        p->a.op = n == "mean" ? kRowMean : kRowSum;
    } else if (last_axis("mean axis ", &rest) && rest.empty() && k.inputs.size() == 1) {
        p->a.op = kRowMean;
    } else if (last_axis("sum axis ", &rest) && rest.empty() && k.inputs.size() == 1) {
        p->a.op = kRowSum;
    } else if (last_axis("softmax axis ", &rest)) {
        if (rest.empty() && k.inputs.size() == 1) p->a.op = kSoftmax3;
        else if (rest == ", two passes" && k.inputs.size() == 1) p->a.op = kSoftmax2;
        else if ((rest == " where" || rest == " where, two passes") && k.inputs.size() == 2) {
            p->a.op = rest == " where" ? kMaskedSoftmax3 : kMaskedSoftmax2;
            const BufSpec& m = k.inputs[1];
            std::vector<int> map;
            const int r = (int)x.dims.size();
            if (m.ty != Ty::I64 || m.dims.size() != 2 || r < 2 || !align(m, x, &map) || map[0] != r - 2 || map[1] != r - 1) return nullptr;
            p->a.mask_rows = m.dims[0];
        } else {
            return nullptr;
        }
    } else if (n == "sum_to" && k.inputs.size() == 2) {
        // onto x's leading axes: each output element the ordered sum of a row
        std::vector<int> m;
        const BufSpec& o = k.output;
        if (!align(o, x, &m) || o.dims.empty() || o.dims.size() >= x.dims.size()) return nullptr;
        for (size_t i = 0; i < m.size(); ++i)
            if (m[i] != (int)i) return nullptr;
        p->a.rows = o.numel();
        p->a.n = p->a.rows ? x.numel() / p->a.rows : 0;
        p->a.op = kSumToRows;
    } else if ((n == "cross_entropy" && k.inputs.size() == 2) || (n == "cross_entropy_vjp" && k.inputs.size() == 3)) {
        const BufSpec& y = k.inputs[1];
        if (y.ty != Ty::I64 || y.numel() != p->a.rows) return nullptr;
        if (n == "cross_entropy_vjp" && (k.inputs[2].ty != k.dtype || k.inputs[2].numel() != p->a.rows)) return nullptr;
        p->a.op = n == "cross_entropy" ? kCrossEntropy : kCrossEntropyVjp;
    } else {
        return nullptr;
    }
    if (k.output.ty != k.dtype) return nullptr;
    // the split loop runs over x's first axis (and the output's), each
    // iteration a run of whole rows
    p->row_out = p->a.op == kRowMean || p->a.op == kRowSum || p->a.op == kSumToRows || p->a.op == kCrossEntropy;
    // FAST: one wave a row (rows of up to 16 blocks a lane); a single
    // total (`mean`/`sum` of every element) stays ordered
    if (fast && p->a.rows > 1 && wrows_ok(p->a)) {
        p->fast = true;
        p->vec = wrows_vec(p->a);
    }
    p->nest = parallel_outer(k);
    if (p->nest > 0 && x.dims[0] == p->nest && !k.output.dims.empty() && k.output.dims[0] == p->nest &&
        p->a.rows % p->nest == 0) {
        p->split = p->nest;
        p->rows_per_iter = p->a.rows / p->nest;
    }
    return p;
}

}  // namespace

// ---------------------------------------------------------------------------
// embed_vjp: the tokens' cotangent rows added into the table rows they name,
// in token order (exact in every mode)

struct ScatterPlan : ClassPlan {
    ScatterArgs a{};
    bool guarded = false;
    const char* kind() const override { return "scatter"; }
    std::string order() const override { return "sequential"; }
    // the nest zeroes its output before the scatter, so it has no split loop
    // (crates/presk-kernel/src/ir.rs:336-376): only whole calls
    hipError_t launch(void* const* bufs, int64_t lo, int64_t hi, void*, hipStream_t stream) const override {
        int64_t first, count;
        if (!range(lo, hi, &first, &count)) return hipErrorInvalidValue;
        ScatterArgs x = a;
        x.idx = (const long long*)bufs[1];
        x.ct = bufs[2];
        x.out = bufs[3];
        x.flag = guarded ? (unsigned*)bufs[4] : nullptr;
        return embed_vjp_launch(x, stream);
    }
};

std::unique_ptr<ClassPlan> classify_scatter(const Kernel& k) {
    const int st = k.dtype == Ty::F32 ? 0 : k.dtype == Ty::BF16 ? 1 : k.dtype == Ty::F16 ? 2 : -1;
    if (st < 0 || k.name != "embed_vjp" || k.inputs.size() != 3) return nullptr;
    const BufSpec &table = k.inputs[0], &idx = k.inputs[1], &ct = k.inputs[2], &o = k.output;
    if (table.dims.size() != 2 || o.dims != table.dims || idx.ty != Ty::I64 || ct.ty != k.dtype) return nullptr;
    if (ct.dims.size() != idx.dims.size() + 1 || ct.dims.back() != table.dims[1]) return nullptr;
    for (size_t i = 0; i < idx.dims.size(); ++i)
        if (ct.dims[i] != idx.dims[i]) return nullptr;
    auto p = std::make_unique<ScatterPlan>();
    p->a.tokens = idx.numel();
    p->a.vocab = table.dims[0];
    p->a.d = table.dims[1];
    p->a.storage = st;
    p->guarded = k.guarded();
    p->nest = parallel_outer(k);
    if (p->a.tokens > (1ll << 30) || p->a.vocab > 0x7fffffffll) return nullptr;
    return p;
}

std::unique_ptr<ClassPlan> classify(const Kernel& k, int mode) {
    // integer weights (their scales in the slots after the output): in
    // FAST a contraction takes the f32 MFMA kernel on their loads, anything
    // else the generic printer's loads
    if (k.n_quant() > 0) return mode == PRESK_HIP_FAST ? classify_gemm(k) : nullptr;
    // FAST: column sums and totals in the declared chunked order
    if (mode == PRESK_HIP_FAST)
        if (auto p = classify_sum_to(k)) return p;
    // row nests: the interpreter's order (EXACT), FAST's lane tree (FAST)
    if (auto p = classify_rows(k, mode == PRESK_HIP_FAST)) return p;
    if (auto p = classify_scatter(k)) return p;
    if (mode == PRESK_HIP_FAST)
        if (auto p = classify_gemm(k)) return p;
    return nullptr;
}

}  // namespace presk
