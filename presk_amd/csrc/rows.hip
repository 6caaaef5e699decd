// Row nests in the interpreter's own order (EXACT in both modes): the
// softmax over the last axis in three passes, in two, and masked
// (crates/presk-kernel/src/lower.rs:1274-1419), `mean`/`sum` over the last
// axis (lower.rs:1239-1255), `sum_to` onto leading axes (lower.rs:1670-1680),
// `cross_entropy` and `cross_entropy_vjp` (lower.rs:1459-1488).
//
// Only the running reductions of these nests (a sum, a max) have an order;
// everything elementwise (the exponentials, the divisions, the mask tests,
// the stores) does not.  So one wave owns R rows and works in chunks of 64
// columns: lane j loads column c0 + j of every row (R coalesced loads in
// flight), computes the elementwise part in that layout, and for a reduction
// parks the chunk in LDS, where lane i walks row i in index order -- the
// interpreter's sequential sum, bit for bit.  Passes that only write (the
// last pass of a softmax, the vjp) stay in the coalesced layout throughout,
// with the row's max and sum read from the walking lane.  A row of at most
// four chunks is loaded once and kept in registers for all the nest's passes
// (the nest reads the same values each pass); a longer row is read again at
// each pass, as the nest does.
#include <hip/hip_runtime.h>

#include "devfmt.hpp"
#include "rows.hpp"

namespace presk {

namespace {

constexpr int CW = 64;     // columns per chunk, one per lane
constexpr int NRES = 4;    // rows of at most NRES chunks stay in registers for every pass

template <int ST>
__device__ __forceinline__ float ld(const void* p, long long i) {
    if (ST == 0) return ((const float*)p)[i];
    if (ST == 1) return pk_bf16_to_f32(((const unsigned short*)p)[i]);
    return pk_f16_to_f32(((const unsigned short*)p)[i]);
}

// A store of v to element i, rounded to the storage type, under the guard.
template <int ST>
__device__ __forceinline__ void st(void* p, long long i, float v, bool& ovf) {
    if (ST == 0) {
        ((float*)p)[i] = v;
    } else if (ST == 1) {
        ((unsigned short*)p)[i] = pk_f32_to_bf16(v);
    } else {
        ovf |= pk_overflows_f16(v);
        ((unsigned short*)p)[i] = pk_f32_to_f16(v);
    }
}

// The value a store of v leaves in memory, as a load reads it back.
template <int ST>
__device__ __forceinline__ float stored(float v) {
    if (ST == 0) return v;
    if (ST == 1) return pk_bf16_to_f32(pk_f32_to_bf16(v));
    return pk_f16_to_f32(pk_f32_to_f16(v));
}

// lane i's value, in every lane
__device__ __forceinline__ float from_lane(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

// R rows per wave (one wave per workgroup); RES: the row fits in NRES chunks,
// loaded once and kept in registers across the nest's passes
template <int OP, int ST, int R, bool RES>
__global__ void __launch_bounds__(64) rows_kernel(RowArgs a) {
    constexpr bool MASKED = OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2;
    __shared__ float tile[R][CW + 1];
    const int lane = threadIdx.x;
    const long long row0 = (long long)blockIdx.x * R;
    const long long n = a.n;
    const int nr = (int)(a.rows - row0 < R ? a.rows - row0 : R);  // live rows here
    const bool walker = lane < nr;
    const long long r = row0 + lane;  // the walking lane's row
    const float qnan = __int_as_float(0x7fc00000);
    bool ovf = false;

    // the mask row of each of the R rows (the mask repeats over leading axes)
    long long moff[MASKED ? R : 1];
    if (MASKED) {
        long long mr = (row0 + a.mask_row0) % a.mask_rows;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            moff[i] = mr * n;
            mr = mr + 1 == a.mask_rows ? 0 : mr + 1;
        }
    }

    // x[row0 + i][c0 + lane] for every row, and the mask's verdicts as bits
    // (bit i: row i).  Addresses are clamped into the rows and the chunk, so
    // every load is issued unconditionally and all are in flight together;
    // a clamped lane's values are never used.
    auto load = [&](long long c0, int cw, float (&v)[R], unsigned& mb) {
        const long long col = c0 + (lane < cw ? lane : cw - 1);
#pragma unroll
        for (int i = 0; i < R; ++i) v[i] = ld<ST>(a.x, (row0 + (i < nr ? i : nr - 1)) * n + col);
        if (MASKED) {
            const long long* mask = (const long long*)a.mask;
            long long mv[R];
#pragma unroll
            for (int i = 0; i < R; ++i) mv[i] = mask[moff[i] + col];
            unsigned b = 0;
#pragma unroll
            for (int i = 0; i < R; ++i)
                // allowed: real(mask) > 0.5 in the nest's f32
                b |= ((float)(double)mv[i] > 0.5f ? 1u : 0u) << i;
            mb = lane < cw ? b & ((1u << nr) - 1u) : 0u;
        }
    };
    // lane i walks tile row i over columns [0, cw) in order
    auto walk = [&](int cw, auto&& f) {
        __syncthreads();
        if (walker) {
#pragma unroll 8
            for (int j = 0; j < cw; ++j) f(tile[lane][j]);
        }
        __syncthreads();
    };
    // the row's chunks: resident ones loaded once here, others at each pass
    constexpr int NV = RES ? NRES : 1;
    float v[NV][R];
    unsigned mb[NV];
    auto for_chunks = [&](auto&& body) {
        if constexpr (RES) {
#pragma unroll
            for (int ch = 0; ch < NRES; ++ch)
                if (ch * CW < n) body(ch, (long long)ch * CW, (int)(n - ch * CW < CW ? n - ch * CW : CW));
        } else {
            for (long long c0 = 0; c0 < n; c0 += CW) {
                const int cw = (int)(n - c0 < CW ? n - c0 : CW);
                load(c0, cw, v[0], mb[0]);
                body(0, c0, cw);
            }
        }
    };
    if constexpr (RES) {
#pragma unroll
        for (int ch = 0; ch < NRES; ++ch)
            if (ch * CW < n) load(ch * CW, (int)(n - ch * CW < CW ? n - ch * CW : CW), v[ch], mb[ch]);
    }
    auto allowed = [&](int ch, int i) { return MASKED ? ((mb[ch] >> i) & 1u) != 0 : true; };
    // a reduction pass: each element transformed in the coalesced layout
    // (elem may rewrite a resident value), then the chunk walked in order
    auto reduce_pass = [&](auto&& elem, auto&& f) {
        for_chunks([&](int ch, long long, int cw) {
#pragma unroll
            for (int i = 0; i < R; ++i) tile[i][lane] = elem(i, v[ch][i], allowed(ch, i));
            walk(cw, f);
        });
    };
    // a write pass: out[row0 + i][k] = g(i, k, value, allowed), coalesced
    auto write_pass = [&](auto&& g) {
        for_chunks([&](int ch, long long c0, int cw) {
            if (lane < cw) {
#pragma unroll
                for (int i = 0; i < R; ++i)
                    if (i < nr) st<ST>(a.out, (row0 + i) * n + c0 + lane, g(i, c0 + lane, v[ch][i], allowed(ch, i)), ovf);
            }
        });
    };
    auto same = [](int, float& v, bool) { return v; };

    if (OP == kRowMean || OP == kRowSum) {
        float acc = 0.f;
        reduce_pass(same, [&](float x) { acc = acc + x; });
        if (walker) st<ST>(a.out, r, OP == kRowMean ? acc / a.n_real : acc, ovf);
    } else if (OP == kSumToRows) {
        // the running sum lives in the output: every step stored (rounded)
        float acc = 0.f;
        reduce_pass(same, [&](float x) {
            const float s = acc + x;
            if (ST == 2) ovf |= pk_overflows_f16(s);
            acc = stored<ST>(s);
        });
        if (walker) st<ST>(a.out, r, acc, ovf);
    } else {
        if (n == 0) return;
        float m;
        if (!MASKED) {
            // m = x[0]; then m = x[k] wherever x[k] > m
            m = walker ? ld<ST>(a.x, r * n) : 0.f;
            reduce_pass(same, [&](float x) { m = x > m ? x : m; });
        } else {
            // The nest's masked max: the first allowed element, then any
            // later allowed one greater than the running max.  Walked as the
            // plain max from -inf over the allowed elements (a disallowed one
            // walks as NaN, which is never greater), which agrees except when
            // the first allowed element is NaN (the nest's max is then NaN)
            // or none is allowed (the nest's max stays 0): both found here by
            // ballots over the chunks in order.
            unsigned found = 0, nanfirst = 0;  // bit i: row i
            m = -__builtin_inff();
            reduce_pass([&](int i, float& x, bool al) {
                const unsigned long long A = __ballot(al), N = __ballot(al && x != x);
                if (!((found >> i) & 1u) && A) {
                    found |= 1u << i;
                    if (N & (A & (~A + 1ull))) nanfirst |= 1u << i;
                }
                return al ? x : qnan;
            }, [&](float x) { m = x > m ? x : m; });
            m = ((nanfirst >> lane) & 1u) ? qnan : ((found >> lane) & 1u) ? m : 0.f;
        }
        float mi[R];
#pragma unroll
        for (int i = 0; i < R; ++i) mi[i] = from_lane(m, i);
        // the exponentials: a resident row keeps them for the write pass (the
        // nest computes the same exp(x - m) there)
        float z = 0.f;
        reduce_pass([&](int i, float& x, bool al) {
            const float e = al ? pk_expf(x - mi[i]) : 0.f;
            if (RES) x = e;
            return e;
        }, [&](float e) { z = z + e; });
        auto expo = [&](int i, float x, bool al) -> float {
            if (RES) return x;
            return al ? pk_expf(x - mi[i]) : 0.f;
        };
        float zi[R];
#pragma unroll
        for (int i = 0; i < R; ++i) zi[i] = from_lane(z, i);
        if (OP == kSoftmax3 || OP == kMaskedSoftmax3) {
            write_pass([&](int i, long long, float x, bool al) { return al ? expo(i, x, al) / zi[i] : 0.f; });
        } else if (OP == kSoftmax2 || OP == kMaskedSoftmax2) {
            // the stored exponential over z (the first pass's stores of e,
            // guarded, are overwritten)
            write_pass([&](int i, long long, float x, bool al) {
                const float e = expo(i, x, al);
                if (ST == 2) ovf |= pk_overflows_f16(e);
                return al ? stored<ST>(e) / zi[i] : 0.f;
            });
        } else if (OP == kCrossEntropy) {
            if (walker) {
                const long long y = ((const long long*)a.y)[r];
                st<ST>(a.out, r, (pk_logf(z) + m) - ld<ST>(a.x, r * n + y), ovf);
            }
        } else {
            const float ct = walker ? ld<ST>(a.ct, r) : 0.f;
            const float fy = walker ? (float)(double)((const long long*)a.y)[r] : 0.f;
            float cti[R], fyi[R];
#pragma unroll
            for (int i = 0; i < R; ++i) {
                cti[i] = from_lane(ct, i);
                fyi[i] = from_lane(fy, i);
            }
            write_pass([&](int i, long long k, float x, bool al) {
                const float sm = expo(i, x, al) / zi[i];
                const float onehot = (float)(double)k == fyi[i] ? 1.f : 0.f;
                return (sm - onehot) * cti[i];
            });
        }
    }
    if (ovf && a.flag) atomicOr(a.flag, 1u);
}

// A few long rows (a total, `mean_all`, or rows too few to give each lane
// its own): one workgroup per row stages the row through LDS 4096 elements at
// a time, the next stage's loads issued before the current one is walked,
// and one lane adds the stage in index order.
constexpr int LSTAGE = 4096;

template <int OP, int ST>
__global__ void __launch_bounds__(256) rows_long_kernel(RowArgs a) {
    __shared__ __attribute__((aligned(16))) float buf[2][LSTAGE];
    constexpr int PER = LSTAGE / 256;
    const int t = threadIdx.x;
    const long long n = a.n, base = (long long)blockIdx.x * n;
    float acc = 0.f;
    bool ovf = false;
    float nx[PER];
    auto fetch = [&](long long c0) {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const long long c = c0 + j * 256 + t;
            nx[j] = c < n ? ld<ST>(a.x, base + c) : 0.f;
        }
    };
    auto put = [&](int s) {
#pragma unroll
        for (int j = 0; j < PER; ++j) buf[s][j * 256 + t] = nx[j];
    };
    fetch(0);
    put(0);
    __syncthreads();
    int s = 0;
    for (long long c0 = 0; c0 < n; c0 += LSTAGE, s ^= 1) {
        const bool more = c0 + LSTAGE < n;
        if (more) fetch(c0 + LSTAGE);
        if (t == 0) {
            const int cw = (int)(n - c0 < LSTAGE ? n - c0 : LSTAGE);
            int j = 0;
            for (; j + 4 <= cw; j += 4) {
                const float4 q = *(const float4*)&buf[s][j];
                const float e[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (OP == kSumToRows) {
                        const float y = acc + e[u];
                        if (ST == 2) ovf |= pk_overflows_f16(y);
                        acc = stored<ST>(y);
                    } else {
                        acc = acc + e[u];
                    }
                }
            }
            for (; j < cw; ++j) {
                if (OP == kSumToRows) {
                    const float y = acc + buf[s][j];
                    if (ST == 2) ovf |= pk_overflows_f16(y);
                    acc = stored<ST>(y);
                } else {
                    acc = acc + buf[s][j];
                }
            }
        }
        if (more) put(s ^ 1);  // the other buffer was walked last round
        __syncthreads();
    }
    if (t == 0) st<ST>(a.out, blockIdx.x, OP == kRowMean ? acc / a.n_real : acc, ovf);
    if (ovf && a.flag) atomicOr(a.flag, 1u);
}

template <int OP>
hipError_t launch_long(const RowArgs& a, hipStream_t stream) {
    switch (a.storage) {
        case 0: rows_long_kernel<OP, 0><<<(unsigned)a.rows, 256, 0, stream>>>(a); break;
        case 1: rows_long_kernel<OP, 1><<<(unsigned)a.rows, 256, 0, stream>>>(a); break;
        case 2: rows_long_kernel<OP, 2><<<(unsigned)a.rows, 256, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- long rows, many of them: every lane walks a row ---------------------------
//
// A wave owns R rows (a lane each, R <= 64) and streams them in chunks of
// WE = 4096 elements (R rows x CW = WE / R columns).  Each chunk is loaded
// coalesced (16-byte vectors where the rows allow), parked in LDS as f32,
// and walked: lane i runs row i's part of the pass in index order -- the
// nest's own loop, so every running sum is the interpreter's -- while the
// next chunk's loads are already in flight.  (Row means and sums, and `sum_to`
// onto leading axes.)  The mask of a masked softmax over long rows is read as
// bits, packed once per launch (pack_mask_kernel): allowed <=> real(mask) >
// 0.5 <=> mask > 0 for an integer.
constexpr int WE = 4096;

__host__ __device__ constexpr long long mask_words(long long n) { return (n + 63) / 64 * 2; }



__global__ void __launch_bounds__(256) pack_mask_kernel(const long long* mask, unsigned* bits, long long n,
                                                        long long words) {
    const long long r = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const long long c0 = ((long long)blockIdx.x * 4 + (threadIdx.x >> 6)) * 64;
    if (c0 >= n) return;
    const long long c = c0 + lane;
    const unsigned long long b = __ballot(c < n && mask[r * n + c] > 0);
    if (lane < 2) bits[r * words + c0 / 32 + lane] = (unsigned)(lane == 0 ? b : b >> 32);
}

// The same bits a byte a thread: eight columns from four 16-byte loads (a
// wave reads 4 KB of the mask at once, against 512 bytes above), for rows of
// a multiple of 8 columns on a 16-byte-aligned mask.  Byte k of word w holds
// columns 32 w + 8 k .. + 7 (little-endian), as the ballot form lays them;
// columns past the row are zeros.
__global__ void __launch_bounds__(256) pack_mask8_kernel(const long long* mask, unsigned char* bytes, long long n,
                                                         long long row_bytes) {
    typedef long long ll2 __attribute__((ext_vector_type(2)));
    const long long r = blockIdx.y;
    const long long byte = (long long)blockIdx.x * 256 + threadIdx.x;
    if (byte >= row_bytes) return;
    const long long c = 8 * byte;
    unsigned v = 0;
    if (c < n) {   // n % 8 == 0: the eight columns lie in the row
        const ll2* p = (const ll2*)(mask + r * n + c);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const ll2 w = p[q];
            v |= (w.x > 0 ? 1u : 0u) << (2 * q);
            v |= (w.y > 0 ? 1u : 0u) << (2 * q + 1);
        }
    }
    bytes[r * row_bytes + byte] = (unsigned char)v;
}

template <int ST>
struct Raw {
    // storage elements per 16-byte vector
    static constexpr int V = ST == 0 ? 4 : 8;
};

template <int OP, int ST, int R, int VEC>
__global__ void __launch_bounds__(128) rows_walk_kernel(RowArgs a) {
    constexpr int CW = WE / R, TS = CW + 4;     // TS = 4 (mod 32): a b128 walk read is conflict-free
    constexpr int NV = WE / 64 / VEC;            // vectors per lane per chunk
    constexpr int ESZ = ST == 0 ? 4 : 2;
    static_assert(CW % 64 == 0 && CW % VEC == 0, "chunk geometry");
    // two waves: wave 1 loads and converts the chunks into one of two tiles
    // while wave 0's lanes walk the other
    __shared__ __attribute__((aligned(16))) float tiles[2][R * TS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long long row0 = (long long)blockIdx.x * R;
    const long long n = a.n;
    const int nr = (int)(a.rows - row0 < R ? a.rows - row0 : R);
    const bool walker = wave == 0 && lane < nr;
    bool ovf = false;
    const long long nch = (n + CW - 1) / CW;
    using W = unsigned __attribute__((ext_vector_type(VEC * ESZ / 4 > 0 ? VEC * ESZ / 4 : 1)));
    // storage words of this lane's part of a chunk
    typedef unsigned short H;
    W wv[VEC * ESZ >= 4 ? NV : 1];
    H hv[VEC * ESZ >= 4 ? 1 : NV];
    (void)wv;
    (void)hv;
    auto slot = [&](int q, int& row, int& col) {
        const int e = (q * 64 + lane) * VEC;
        row = e / CW;
        col = e % CW;
    };
    auto fetch = [&](long long c0, int cw) {
#pragma unroll
        for (int q = 0; q < NV; ++q) {
            int row, col;
            slot(q, row, col);
            row = row < nr ? row : nr - 1;
            col = col < cw ? col : cw - VEC;
            const long long off = (row0 + row) * n + c0 + col;
            if constexpr (VEC * ESZ >= 4) wv[q] = *(const W*)((const char*)a.x + off * ESZ);
            else hv[q] = ((const H*)a.x)[off];
        }
    };
    auto put = [&](float* tile) {
#pragma unroll
        for (int q = 0; q < NV; ++q) {
            int row, col;
            slot(q, row, col);
            float f[VEC];
            if constexpr (VEC * ESZ >= 4) {
                if constexpr (ST == 0) {
#pragma unroll
                    for (int u = 0; u < VEC; ++u) f[u] = __uint_as_float(wv[q][u]);
                } else {
#pragma unroll
                    for (int u = 0; u < VEC; ++u) {
                        const H h = (H)(wv[q][u / 2] >> (16 * (u & 1)));
                        f[u] = ST == 1 ? pk_bf16_to_f32(h) : pk_f16_to_f32(h);
                    }
                }
            } else {
                f[0] = ST == 1 ? pk_bf16_to_f32(hv[q]) : pk_f16_to_f32(hv[q]);
            }
#pragma unroll
            for (int u = 0; u < VEC; ++u) tile[row * TS + col + u] = f[u];
        }
    };
    // the row in index order: visit(x) in the walking lane.  Wave 1 puts
    // chunk ch + 1 (loaded a step earlier) into the other tile and starts
    // chunk ch + 2's loads while wave 0 walks chunk ch; a barrier a step.
    auto width = [&](long long ch) { return (int)(n - ch * CW < CW ? n - ch * CW : CW); };
    auto pass = [&](auto&& visit) {
        if (wave == 1) {
            fetch(0, width(0));
            put(tiles[0]);
            if (nch > 1) fetch(CW, width(1));
        }
        __syncthreads();
        for (long long ch = 0; ch < nch; ++ch) {
            const int cw = width(ch);
            const float* const tile = tiles[ch & 1];
            if (wave == 1 && ch + 1 < nch) {
                put(tiles[(ch + 1) & 1]);
                if (ch + 2 < nch) fetch((ch + 2) * CW, width(ch + 2));
            }
            if (walker && cw == CW) {
                const float* t = &tile[lane * TS];
                if constexpr (OP == kRowMean || OP == kRowSum || (OP == kSumToRows && ST == 0)) {
                    // one add an element: the chunk straight through, in
                    // groups of 16 elements, each group's four LDS reads
                    // issued three groups (48 dependent adds) ahead of their
                    // use; the scheduler barriers keep them there
                    constexpr int NG = CW / 16, AHEAD = 3;
                    float4 q[NG][4];
                    auto rdg = [&](int g) {
#pragma unroll
                        for (int u = 0; u < 4; ++u) q[g][u] = *(const float4*)&t[16 * g + 4 * u];
                    };
#pragma unroll
                    for (int g = 0; g < AHEAD && g < NG; ++g) rdg(g);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int g = 0; g < NG; ++g) {
                        if (g + AHEAD < NG) rdg(g + AHEAD);
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            visit(q[g][u].x);
                            visit(q[g][u].y);
                            visit(q[g][u].z);
                            visit(q[g][u].w);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                } else {
#pragma unroll 8
                    for (int j = 0; j < CW; j += 4) {
                        const float4 q = *(const float4*)&t[j];
                        visit(q.x);
                        visit(q.y);
                        visit(q.z);
                        visit(q.w);
                    }
                }
            } else if (walker) {
                const float* t = &tile[lane * TS];
                int j = 0;
#pragma unroll 8
                for (; j + 4 <= cw; j += 4) {
                    const float4 q = *(const float4*)&t[j];
                    visit(q.x);
                    visit(q.y);
                    visit(q.z);
                    visit(q.w);
                }
                for (; j < cw; ++j) visit(t[j]);
            }
            __syncthreads();   // this tile walked, the other filled
        }
    };
    const long long r = row0 + lane;
    if (OP == kRowMean || OP == kRowSum) {
        float acc = 0.f;
        pass([&](float x) { acc = acc + x; });
        if (walker) st<ST>(a.out, r, OP == kRowMean ? acc / a.n_real : acc, ovf);
    } else if (OP == kSumToRows) {
        float acc = 0.f;
        pass([&](float x) {
            const float s = acc + x;
            if (ST == 2) ovf |= pk_overflows_f16(s);
            acc = stored<ST>(s);
        });
        if (walker) st<ST>(a.out, r, acc, ovf);
    }
    if (ovf && a.flag) atomicOr(a.flag, 1u);
}

template <int OP, int ST, int R>
hipError_t launch_walk_v(const RowArgs& a, hipStream_t stream) {
    constexpr int V = Raw<ST>::V;
    const unsigned grid = (unsigned)((a.rows + R - 1) / R);
    const int esz = ST == 0 ? 4 : 2;
    const bool vec = (uintptr_t)a.x % 16 == 0 && (uintptr_t)a.out % 16 == 0 && (a.n * esz) % 16 == 0;
    if (vec) rows_walk_kernel<OP, ST, R, V><<<grid, 128, 0, stream>>>(a);
    else rows_walk_kernel<OP, ST, R, 1><<<grid, 128, 0, stream>>>(a);
    return hipGetLastError();
}

template <int OP, int R>
hipError_t launch_walk_r(const RowArgs& a, hipStream_t stream) {
    switch (a.storage) {
        case 0: return launch_walk_v<OP, 0, R>(a, stream);
        case 1: return launch_walk_v<OP, 1, R>(a, stream);
        case 2: return launch_walk_v<OP, 2, R>(a, stream);
    }
    return hipErrorInvalidValue;
}

// ---- softmax over long rows, streamed ------------------------------------------
//
// One wave owns R = 16 rows and streams them in chunks of 64 columns, lane j
// on column c0 + j of every row, the next chunk's loads in flight while the
// current one is worked; the nest's three loops are three passes:
// * the max.  The nest's running max (from element 0, or from the first
//   allowed element; a strict `>` after it) is the max over the non-NaN
//   (allowed) elements unless that first element is NaN (then NaN), or 0
//   when nothing is allowed: order-free apart from the first element, so each
//   lane keeps its own and a wave reduction joins them (a max over +0 and -0
//   may differ in sign, which no exp(x - m) can see);
// * z.  Each exponential is computed in the coalesced layout, parked in LDS,
//   and lane i adds row i's in index order -- the interpreter's running sum,
//   bit for bit.  Sixteen sums a wave and several waves a SIMD keep these
//   dependent chains from waiting on each other;
// * the outputs, e / z (3 passes) or stored(e) / z (2 passes), the
//   exponential computed again as the nest computes it again, stored
//   coalesced.
// The mask arrives as bits (pack_mask_kernel), one uniform 64-bit word per
// row and chunk.
// f[u] <- exp(f[u] - m) where bit u of `al` allows it, else 0: the nest's
// select(allowed, exp(x - m), 0).  A refused element's exponent is taken at
// 0 (its value is never used), so that a group whose allowed exponents all
// lie in (-87.34, 0] -- a softmax's, unless a NaN or an infinity is about --
// takes expf's shorter path (pk_expf_le0, the same bits there).
template <int VEC>
__device__ __forceinline__ void exps(float (&f)[VEC], float m, unsigned al) {
    float arg[VEC];
    bool ok = true;
#pragma unroll
    for (int u = 0; u < VEC; ++u) {
        arg[u] = ((al >> u) & 1u) != 0 ? f[u] - m : 0.f;
        ok = ok && pk_expf_le0_ok(arg[u]);
    }
    if (__all(ok)) {
#pragma unroll
        for (int u = 0; u < VEC; ++u) f[u] = ((al >> u) & 1u) != 0 ? pk_expf_le0(arg[u]) : 0.f;
    } else {
#pragma unroll
        for (int u = 0; u < VEC; ++u) f[u] = ((al >> u) & 1u) != 0 ? pk_expf(arg[u]) : 0.f;
    }
}

// f[u] <- f[u] / z, correctly rounded: Markstein's correction step with
// rz = 1/z (pk_div_by), the division itself for a wave where some element
// falls outside the range the step is exact in -- the same bits.
template <int VEC>
__device__ __forceinline__ void quotients(float (&f)[VEC], float z, float rz) {
    float q[VEC];
    bool need = false;
#pragma unroll
    for (int u = 0; u < VEC; ++u) {
        q[u] = pk_div_by(f[u], z, rz);
        need = need || !pk_div_by_ok(f[u], z);
    }
    if (__any(need)) {
#pragma unroll
        for (int u = 0; u < VEC; ++u) q[u] = pk_div_by_ok(f[u], z) ? q[u] : f[u] / z;
    }
#pragma unroll
    for (int u = 0; u < VEC; ++u) f[u] = q[u];
}

// SR rows a wave (eight waves a SIMD hide the passes' latency better than
// fewer, longer ones), SD chunks of loads in flight (2: the fewer registers
// leave more waves a SIMD, which hide the loads as well -- 443 -> 409 us in
// f32 and 329 -> 323 us in bf16 at config 5's masked shape against 4)
constexpr int SR = 8, SCW = 64, STS = SCW + 4, SD = 2;   // STS = 4 (mod 32): b128 tile reads and writes

// A lane moves 16 bytes a load: VEC elements of one row.  Lane l in slot q of
// a chunk holds row q * RPI + l / LPR, columns (l % LPR) * VEC ..+VEC.
template <int ST>
struct SGeo {
    static constexpr int VEC = ST == 0 ? 4 : 8;
    static constexpr int LPR = SCW / VEC;      // lanes a row
    static constexpr int RPI = 64 / LPR;       // rows an instruction
    static constexpr int NQ = SR / RPI;        // vectors a lane a chunk
};

template <int OP, int ST>
__global__ void __launch_bounds__(64) softmax_stream_kernel(RowArgs a) {
    constexpr bool MASKED = OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2;
    constexpr bool TWO = OP == kSoftmax2 || OP == kMaskedSoftmax2;
    using G = SGeo<ST>;
    constexpr int VEC = G::VEC, LPR = G::LPR, RPI = G::RPI, NQ = G::NQ;
    typedef unsigned U4 __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) float tile[SR * STS];
    const int lane = threadIdx.x;
    const long long row0 = (long long)blockIdx.x * SR;
    const long long n = a.n;
    const int nr = (int)(a.rows - row0 < SR ? a.rows - row0 : SR);
    const long long MW = mask_words(n);
    const int lc = (lane % LPR) * VEC;              // this lane's first column in a chunk
    bool ovf = false;
    int myrow[NQ];
    const unsigned* mrow[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int r = q * RPI + lane / LPR;
        myrow[q] = r < nr ? r : nr - 1;             // clamped: a dead row's values are never used
        mrow[q] = MASKED ? a.mbits + ((row0 + myrow[q] + a.mask_row0) % a.mask_rows) * MW : nullptr;
    }
    // the 16-byte vectors of the chunk at c0 (columns clamped into the row)
    auto load = [&](long long c0, U4 (&w)[NQ]) {
        const long long col = c0 + lc < n ? c0 + lc : n - VEC;
#pragma unroll
        for (int q = 0; q < NQ; ++q) w[q] = *(const U4*)((const char*)a.x + ((row0 + myrow[q]) * n + col) * (ST == 0 ? 4 : 2));
    };
    auto unpack = [&](const U4& w, float (&f)[VEC]) {
#pragma unroll
        for (int u = 0; u < VEC; ++u) {
            if (ST == 0) f[u] = __uint_as_float(w[u]);
            else {
                const unsigned short h = (unsigned short)(w[u / 2] >> (16 * (u & 1)));
                f[u] = ST == 1 ? pk_bf16_to_f32(h) : pk_f16_to_f32(h);
            }
        }
    };
    // this lane's VEC columns at c0 in slot q: allowed and inside the row, as bits
    auto bits = [&](int q, long long c0) -> unsigned {
        const long long c = c0 + lc;
        const unsigned live = c >= n ? 0u : n - c >= VEC ? (1u << VEC) - 1u : (1u << (n - c)) - 1u;
        if (!MASKED) return live;
        return (mrow[q][c >> 5] >> (c & 31)) & live;
    };
    // whether any of the group's rows allows an element of the chunk at c0:
    // a chunk no row allows adds nothing to a max or to a sum (z + 0 is z)
    // and stores zeros, so it is neither read nor computed (the rows above a
    // causal mask's diagonal).  The verdicts of 64 chunks at a time, one
    // chunk a lane (its two mask words in each of the group's rows, all
    // loads in flight together), joined by a ballot.
    unsigned long long lmask = ~0ull;
    long long lbase = -1;
    auto live = [&](long long c0) -> bool {
        if (!MASKED) return true;
        const long long ch = c0 / SCW, grp = ch / 64;
        if (grp != lbase) {
            lbase = grp;
            const long long mine = grp * 64 + lane;
            unsigned any = 0u;
            if (mine * SCW < n) {
#pragma unroll
                for (int r = 0; r < SR; ++r) {
                    const unsigned* w = a.mbits + ((row0 + (r < nr ? r : nr - 1) + a.mask_row0) % a.mask_rows) * MW + 2 * mine;
                    any |= w[0] | w[1];
                }
            }
            lmask = __ballot(any != 0u);
        }
        return (lmask >> (ch - lbase * 64)) & 1ull;
    };
    // a pass over the row group's chunks, SD chunks' loads in flight ahead
    // of the one in use (a ring of registers, its slots fixed by unrolling)
    auto pass = [&](auto&& body, auto&& dead) {
        const long long nch = (n + SCW - 1) / SCW;
        U4 ring[SD][NQ];
        bool lv[SD];
#pragma unroll
        for (int j = 0; j < SD; ++j) {
            lv[j] = j < nch && live((long long)j * SCW);
            if (lv[j]) load((long long)j * SCW, ring[j]);
        }
        for (long long c = 0; c < nch; c += SD) {
#pragma unroll
            for (int j = 0; j < SD; ++j) {
                const long long ch = c + j;
                if (ch < nch) {
                    if (lv[j]) body(ch * SCW, ring[j]);
                    else dead(ch * SCW);
                    const long long nx = ch + SD;
                    lv[j] = nx < nch && live(nx * SCW);
                    if (lv[j]) load(nx * SCW, ring[j]);
                }
            }
        }
    };
    auto nothing = [](long long) {};

    // 1. the max: each lane's allowed non-NaN max and first allowed column,
    //    per row it holds; joined over the row's lanes
    const int BIG = 0x7fffffff;
    float pm[NQ];
    int fa[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        pm[q] = -__builtin_inff();
        fa[q] = BIG;
    }
    pass([&](long long c0, U4 (&w)[NQ]) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            float f[VEC];
            unpack(w[q], f);
            const unsigned al = bits(q, c0);
#pragma unroll
            for (int u = 0; u < VEC; ++u) {
                const bool ok = ((al >> u) & 1u) != 0;
                pm[q] = ok && f[u] > pm[q] ? f[u] : pm[q];
                fa[q] = ok && fa[q] == BIG ? (int)(c0 + lc + u) : fa[q];
            }
        }
    }, nothing);
    float mq[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        float m = pm[q];
        int f = fa[q];
        for (int off = LPR / 2; off > 0; off >>= 1) {
            const float o = __shfl_xor(m, off, 64);
            const int g = __shfl_xor(f, off, 64);
            m = o > m ? o : m;
            f = g < f ? g : f;
        }
        // the first allowed element NaN: the max is NaN; none allowed: 0
        const float first = f == BIG ? 0.f : ld<ST>(a.x, (row0 + myrow[q]) * n + f);
        mq[q] = f == BIG ? 0.f : first != first ? first : m;
    }

    // 2. z: the exponentials into the tile, lane i walking row i in order
    float z = 0.f;
    pass([&](long long c0, U4 (&w)[NQ]) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            float f[VEC];
            unpack(w[q], f);
            const unsigned al = bits(q, c0);
            exps<VEC>(f, mq[q], al);
            float* t = &tile[(q * RPI + lane / LPR) * STS + lc];
#pragma unroll
            for (int u = 0; u < VEC; u += 4) *(float4*)&t[u] = float4{f[u], f[u + 1], f[u + 2], f[u + 3]};
        }
        __syncthreads();
        if (lane < nr) {
            const float* t = &tile[lane * STS];
            const int cw = (int)(n - c0 < SCW ? n - c0 : SCW);
            if (cw == SCW) {
#pragma unroll
                for (int j = 0; j < SCW; j += 4) {
                    const float4 v = *(const float4*)&t[j];
                    z = z + v.x;
                    z = z + v.y;
                    z = z + v.z;
                    z = z + v.w;
                }
            } else {
                for (int j = 0; j < cw; ++j) z = z + t[j];
            }
        }
        __syncthreads();
    }, nothing);
    float zq[NQ], rz[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        // row q * RPI + lane / LPR's z, from its walking lane
        const int src = q * RPI + lane / LPR;
        zq[q] = __shfl(z, src, 64);
        rz[q] = 1.f / zq[q];
    }

    // 3. the outputs, 16 bytes a lane
    pass([&](long long c0, U4 (&w)[NQ]) {
        if (c0 + lc >= n) return;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int row = q * RPI + lane / LPR;
            if (row >= nr) continue;
            float f[VEC];
            unpack(w[q], f);
            const unsigned al = bits(q, c0);
            exps<VEC>(f, mq[q], al);
#pragma unroll
            for (int u = 0; u < VEC; ++u) {
                if (TWO) {
                    if (ST == 2) ovf |= pk_overflows_f16(f[u]);
                    f[u] = stored<ST>(f[u]);
                }
            }
            quotients<VEC>(f, zq[q], rz[q]);
#pragma unroll
            for (int u = 0; u < VEC; ++u) f[u] = ((al >> u) & 1u) != 0 ? f[u] : 0.f;
            U4 o;
            if (ST == 0) {
#pragma unroll
                for (int u = 0; u < VEC; ++u) o[u] = __float_as_uint(f[u]);
            } else {
                o = U4{0u, 0u, 0u, 0u};
#pragma unroll
                for (int u = 0; u < VEC; ++u) {
                    if (ST == 2) ovf |= pk_overflows_f16(f[u]);
                    const unsigned h = ST == 1 ? pk_f32_to_bf16(f[u]) : pk_f32_to_f16(f[u]);
                    o[u / 2] |= h << (16 * (u & 1));
                }
            }
            *(U4*)((char*)a.out + ((row0 + row) * n + c0 + lc) * (ST == 0 ? 4 : 2)) = o;
        }
    }, [&](long long c0) {
        // a chunk no row allows: zeros
        if (c0 + lc >= n) return;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int row = q * RPI + lane / LPR;
            if (row < nr) *(U4*)((char*)a.out + ((row0 + row) * n + c0 + lc) * (ST == 0 ? 4 : 2)) = U4{0u, 0u, 0u, 0u};
        }
    });
    if (ovf && a.flag) atomicOr(a.flag, 1u);
}

// Rows of NC whole 64-column chunks (n = 64 NC, NC <= 4): the streamed
// kernel's three passes over the group's values kept in registers (64 a
// lane at NC = 4), so x is read once and each exponential computed once;
// the same max, the same walk of the tile for z, the same quotient.
template <int OP, int ST, int NC>
__global__ void __launch_bounds__(64) softmax_short_kernel(RowArgs a) {
    constexpr bool MASKED = OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2;
    constexpr bool TWO = OP == kSoftmax2 || OP == kMaskedSoftmax2;
    using G = SGeo<ST>;
    constexpr int VEC = G::VEC, LPR = G::LPR, RPI = G::RPI, NQ = G::NQ;
    constexpr int n = NC * SCW;
    typedef unsigned U4 __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) float tile[SR * STS];
    const int lane = threadIdx.x;
    const long long row0 = (long long)blockIdx.x * SR;
    const int nr = (int)(a.rows - row0 < SR ? a.rows - row0 : SR);
    constexpr long long MW = mask_words(n);
    const int lc = (lane % LPR) * VEC;
    bool ovf = false;
    int myrow[NQ];
    const unsigned* mrow[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int r = q * RPI + lane / LPR;
        myrow[q] = r < nr ? r : nr - 1;
        mrow[q] = MASKED ? a.mbits + ((row0 + myrow[q] + a.mask_row0) % a.mask_rows) * MW : nullptr;
    }
    // the whole group, once
    float v[NC][NQ][VEC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const U4 w = *(const U4*)((const char*)a.x + ((row0 + myrow[q]) * n + c * SCW + lc) * (ST == 0 ? 4 : 2));
#pragma unroll
            for (int u = 0; u < VEC; ++u) {
                if (ST == 0) v[c][q][u] = __uint_as_float(w[u]);
                else {
                    const unsigned short h = (unsigned short)(w[u / 2] >> (16 * (u & 1)));
                    v[c][q][u] = ST == 1 ? pk_bf16_to_f32(h) : pk_f16_to_f32(h);
                }
            }
        }
    auto bits = [&](int q, int c) -> unsigned {
        constexpr unsigned live = (1u << VEC) - 1u;
        if (!MASKED) return live;
        const int col = c * SCW + lc;
        return (mrow[q][col >> 5] >> (col & 31)) & live;
    };

    // 1. the max (as the streamed kernel: lane partials joined over the row),
    //    the first allowed element's value joined beside its column (no
    //    second read of x, whose latency nothing here would hide)
    const int BIG = 0x7fffffff;
    float mq[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        float m = -__builtin_inff(), fv = 0.f;
        int f = BIG;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const unsigned al = bits(q, c);
#pragma unroll
            for (int u = 0; u < VEC; ++u) {
                const bool ok = ((al >> u) & 1u) != 0;
                m = ok && v[c][q][u] > m ? v[c][q][u] : m;
                const bool first = ok && f == BIG;
                fv = first ? v[c][q][u] : fv;
                f = first ? c * SCW + lc + u : f;
            }
        }
        for (int off = LPR / 2; off > 0; off >>= 1) {
            const float o = __shfl_xor(m, off, 64), ov = __shfl_xor(fv, off, 64);
            const int g = __shfl_xor(f, off, 64);
            m = o > m ? o : m;
            fv = g < f ? ov : fv;
            f = g < f ? g : f;
        }
        mq[q] = f == BIG ? 0.f : fv != fv ? fv : m;
    }

    // 2. the exponentials, in place; z by lane i walking row i through the tile
    float z = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            exps<VEC>(v[c][q], mq[q], bits(q, c));
            float* t = &tile[(q * RPI + lane / LPR) * STS + lc];
#pragma unroll
            for (int u = 0; u < VEC; u += 4) *(float4*)&t[u] = float4{v[c][q][u], v[c][q][u + 1], v[c][q][u + 2], v[c][q][u + 3]};
        }
        __syncthreads();
        if (lane < nr) {
            const float* t = &tile[lane * STS];
#pragma unroll
            for (int j = 0; j < SCW; j += 4) {
                const float4 e = *(const float4*)&t[j];
                z = z + e.x;
                z = z + e.y;
                z = z + e.z;
                z = z + e.w;
            }
        }
        __syncthreads();
    }
    float zq[NQ], rz[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        zq[q] = __shfl(z, q * RPI + lane / LPR, 64);
        rz[q] = 1.f / zq[q];
    }

    // 3. the outputs, 16 bytes a lane
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int row = q * RPI + lane / LPR;
            if (row >= nr) continue;
            const unsigned al = bits(q, c);
            float f[VEC];
#pragma unroll
            for (int u = 0; u < VEC; ++u) {
                f[u] = v[c][q][u];
                if (TWO) {
                    if (ST == 2) ovf |= pk_overflows_f16(f[u]);
                    f[u] = stored<ST>(f[u]);
                }
            }
            quotients<VEC>(f, zq[q], rz[q]);
#pragma unroll
            for (int u = 0; u < VEC; ++u) f[u] = ((al >> u) & 1u) != 0 ? f[u] : 0.f;
            U4 o;
            if (ST == 0) {
#pragma unroll
                for (int u = 0; u < VEC; ++u) o[u] = __float_as_uint(f[u]);
            } else {
                o = U4{0u, 0u, 0u, 0u};
#pragma unroll
                for (int u = 0; u < VEC; ++u) {
                    if (ST == 2) ovf |= pk_overflows_f16(f[u]);
                    const unsigned h = ST == 1 ? pk_f32_to_bf16(f[u]) : pk_f32_to_f16(f[u]);
                    o[u / 2] |= h << (16 * (u & 1));
                }
            }
            *(U4*)((char*)a.out + ((row0 + row) * n + c * SCW + lc) * (ST == 0 ? 4 : 2)) = o;
        }
    if (ovf && a.flag) atomicOr(a.flag, 1u);
}

template <int OP, int NC>
hipError_t launch_short(const RowArgs& a, hipStream_t stream) {
    const unsigned grid = (unsigned)((a.rows + SR - 1) / SR);
    switch (a.storage) {
        case 0: softmax_short_kernel<OP, 0, NC><<<grid, 64, 0, stream>>>(a); break;
        case 1: softmax_short_kernel<OP, 1, NC><<<grid, 64, 0, stream>>>(a); break;
        case 2: softmax_short_kernel<OP, 2, NC><<<grid, 64, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int OP, int R, bool RES>
hipError_t launch_r(const RowArgs& a, hipStream_t stream);

template <int OP>
hipError_t launch_stream(const RowArgs& a, hipStream_t stream) {
    // whole 16-byte vectors: rows of a multiple of 64 columns on aligned
    // buffers (the last chunk of a row is then whole too); others take the
    // general row kernel
    const int esz = a.storage == 0 ? 4 : 2;
    if (a.n % SCW != 0 || (uintptr_t)a.x % 16 != 0 || (uintptr_t)a.out % 16 != 0 || (a.n * esz) % 16 != 0)
        return launch_r<OP, 16, false>(a, stream);
    // rows of at most four chunks: kept in registers
    switch (a.n / SCW) {
        case 1: return launch_short<OP, 1>(a, stream);
        case 2: return launch_short<OP, 2>(a, stream);
        case 3: return launch_short<OP, 3>(a, stream);
        case 4: return launch_short<OP, 4>(a, stream);
        default: break;
    }
    const unsigned grid = (unsigned)((a.rows + SR - 1) / SR);
    switch (a.storage) {
        case 0: softmax_stream_kernel<OP, 0><<<grid, 64, 0, stream>>>(a); break;
        case 1: softmax_stream_kernel<OP, 1><<<grid, 64, 0, stream>>>(a); break;
        case 2: softmax_stream_kernel<OP, 2><<<grid, 64, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Rows per wave for the walk: 64 (every lane walks) where that still leaves
// 1024 waves, else fewer, down to 4, to keep some 512 waves in flight.
template <int OP>
hipError_t launch_walk(const RowArgs& a, hipStream_t stream) {
    constexpr bool SOFTMAX = OP == kSoftmax3 || OP == kSoftmax2 || OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2;
    if (OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2) {
        hipError_t e = rows_pack_mask(a, stream);
        if (e != hipSuccess) return e;
    }
    if constexpr (SOFTMAX) {
        return launch_stream<OP>(a, stream);
    } else {
        const long long r = a.rows;
        if (r >= 64 * 1024) return launch_walk_r<OP, 64>(a, stream);
        if (r >= 32 * 512) return launch_walk_r<OP, 32>(a, stream);
        if (r >= 16 * 512) return launch_walk_r<OP, 16>(a, stream);
        if (r >= 8 * 512) return launch_walk_r<OP, 8>(a, stream);
        return launch_walk_r<OP, 4>(a, stream);
    }
}

// softmax rows that fit in registers but are many and of whole 64-column
// chunks take the streamed kernel as well (aligned buffers permitting)
bool streams_short(const RowArgs& a) { return a.n % SCW == 0 && a.rows >= 8192; }

// the long-row walk serves these nests when their rows do not fit in registers
constexpr bool walks(int op) {
    return op == kRowMean || op == kRowSum || op == kSumToRows || op == kSoftmax3 || op == kSoftmax2 ||
           op == kMaskedSoftmax3 || op == kMaskedSoftmax2;
}

template <int OP, int R, bool RES>
hipError_t launch_r(const RowArgs& a, hipStream_t stream) {
    const unsigned grid = (unsigned)((a.rows + R - 1) / R);
    switch (a.storage) {
        case 0: rows_kernel<OP, 0, R, RES><<<grid, 64, 0, stream>>>(a); break;
        case 1: rows_kernel<OP, 1, R, RES><<<grid, 64, 0, stream>>>(a); break;
        case 2: rows_kernel<OP, 2, R, RES><<<grid, 64, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Rows per wave: a walk costs the same issue slots however many of its
// lanes are live, so 16 rows a wave -- unless that leaves fewer waves than
// SIMDs (under 8192 rows), when 4 rows a wave spreads the walks wider.
template <int OP>
hipError_t launch_op(const RowArgs& a, hipStream_t stream) {
    if (a.rows == 0) return hipSuccess;
    if constexpr (OP == kRowMean || OP == kRowSum || OP == kSumToRows) {
        // rows too few for a lane each and long enough to stage
        if (a.rows < 1024 && a.n >= 1024) return launch_long<OP>(a, stream);
    }
    if ((OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2) && a.mask_rows <= 0) return hipErrorInvalidValue;
    if ((a.rows + 3) / 4 > 0x7fffffffll) return hipErrorInvalidValue;
    const bool res = a.n <= NRES * CW;
    if constexpr (walks(OP)) {
        if (!res) return launch_walk<OP>(a, stream);
    }
    if constexpr (OP == kSoftmax3 || OP == kSoftmax2 || OP == kMaskedSoftmax3 || OP == kMaskedSoftmax2) {
        // short rows of whole 64-column chunks on aligned buffers stream too:
        // 16-byte loads and the mask as bits beat the register-resident rows
        if (streams_short(a) && (uintptr_t)a.x % 16 == 0 && (uintptr_t)a.out % 16 == 0)
            return launch_walk<OP>(a, stream);
    }
    if (a.rows >= 8192)
        return res ? launch_r<OP, 16, true>(a, stream) : launch_r<OP, 16, false>(a, stream);
    return res ? launch_r<OP, 4, true>(a, stream) : launch_r<OP, 4, false>(a, stream);
}

}  // namespace

long long rows_mask_words(long long n) { return mask_words(n); }

hipError_t rows_pack_mask(const RowArgs& a, hipStream_t stream) {
    if (!a.mbits || a.mask_rows <= 0) return hipErrorInvalidValue;
    const long long words = mask_words(a.n);
    if (a.n % 8 == 0 && (uintptr_t)a.mask % 16 == 0) {
        const dim3 grid((unsigned)((words * 4 + 255) / 256), (unsigned)a.mask_rows);
        pack_mask8_kernel<<<grid, 256, 0, stream>>>((const long long*)a.mask, (unsigned char*)a.mbits, a.n, words * 4);
    } else {
        const dim3 grid((unsigned)((a.n + 255) / 256), (unsigned)a.mask_rows);
        pack_mask_kernel<<<grid, 256, 0, stream>>>((const long long*)a.mask, a.mbits, a.n, words);
    }
    return hipGetLastError();
}

bool rows_need_mask_bits(const RowArgs& a) {
    return (a.op == kMaskedSoftmax3 || a.op == kMaskedSoftmax2) && a.rows > 0 &&
           (a.n > NRES * CW || streams_short(a));
}

hipError_t rows_launch(const RowArgs& a, hipStream_t stream) {
    switch (a.op) {
        case kRowMean: return launch_op<kRowMean>(a, stream);
        case kRowSum: return launch_op<kRowSum>(a, stream);
        case kSumToRows: return launch_op<kSumToRows>(a, stream);
        case kSoftmax3: return launch_op<kSoftmax3>(a, stream);
        case kSoftmax2: return launch_op<kSoftmax2>(a, stream);
        case kMaskedSoftmax3: return launch_op<kMaskedSoftmax3>(a, stream);
        case kMaskedSoftmax2: return launch_op<kMaskedSoftmax2>(a, stream);
        case kCrossEntropy: return launch_op<kCrossEntropy>(a, stream);
        case kCrossEntropyVjp: return launch_op<kCrossEntropyVjp>(a, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace presk
