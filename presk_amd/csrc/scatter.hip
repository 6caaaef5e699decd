// `embed_vjp` (crates/presk-kernel/src/lower.rs:1444-1457): the gradient of a
// table lookup.  The nest zeroes the [vocab][d] output, then walks the tokens
// in order and adds each token's cotangent row into the table row its index
// names: out[idx[t]][j] = out[idx[t]][j] + ct[t][j], every step a store
// (rounded to the storage type, checked by the f16 guard).  Each output
// element therefore receives the cotangents of the tokens that name its row,
// in token order.  The printer's nest can only spread over j (the rows
// collide), leaving 16K dependent steps per thread.
//
// Here one workgroup owns one table row v and 256 of its columns.  Its four
// waves scan the indices together, 4096 tokens a round (sixteen coalesced
// loads per lane in flight), and compact the positions of the tokens naming v
// into an LDS list in token order (a ballot per 64 tokens, counts shared
// through LDS).  Then each lane adds its column of those tokens' rows in list
// order -- the nest's order, bit for bit -- the next 64 rows' loads in flight
// while 64 are added (the rows lie anywhere in the cotangent, so each load
// waits on HBM: 128 in flight a lane).  An
// index outside [0, vocab) names no row here and is never added.
#include <hip/hip_runtime.h>

#include "devfmt.hpp"
#include "scatter.hpp"

namespace presk {

namespace {

constexpr int WAVES = 4;
constexpr int PER = 16;                       // indices per lane per round
constexpr int ROUND = PER * WAVES * 64;       // tokens scanned per round
constexpr int BATCH = 64;                     // row loads a batch, one list entry a lane (two batches in flight)

template <int ST>
__device__ __forceinline__ float ld(const void* p, long long i) {
    if (ST == 0) return ((const float*)p)[i];
    if (ST == 1) return pk_bf16_to_f32(((const unsigned short*)p)[i]);
    return pk_f16_to_f32(((const unsigned short*)p)[i]);
}

template <int ST>
__device__ __forceinline__ float stored(float v) {
    if (ST == 0) return v;
    if (ST == 1) return pk_bf16_to_f32(pk_f32_to_bf16(v));
    return pk_f16_to_f32(pk_f32_to_f16(v));
}

template <int ST>
__global__ void __launch_bounds__(WAVES * 64) embed_vjp_kernel(ScatterArgs a) {
    __shared__ int list[ROUND];
    __shared__ int cnt[PER][WAVES];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const long long v = blockIdx.x;
    const long long col = (long long)blockIdx.y * (WAVES * 64) + tid;
    const bool live = col < a.d;
    const unsigned long long below = lane ? ~0ull >> (64 - lane) : 0ull;
    float acc = 0.f;  // the zeroed output element
    bool ovf = false;

    for (long long base = 0; base < a.tokens; base += ROUND) {
        // token base + k*256 + tid: lane order within a wave, waves in order,
        // then k -- so (k, w, lane) is token order
        bool hit[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const long long t = base + k * (WAVES * 64) + tid;
            hit[k] = t < a.tokens && a.idx[t] == v;
        }
        unsigned long long bal[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) bal[k] = __ballot(hit[k]);
        if (lane == 0) {
#pragma unroll
            for (int k = 0; k < PER; ++k) cnt[k][w] = __popcll(bal[k]);
        }
        __syncthreads();
        int before = 0, total = 0;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            int mine = before;
            for (int q = 0; q < WAVES; ++q) {
                if (q < w) mine += cnt[k][q];
                before += cnt[k][q];
            }
            if (hit[k]) list[mine + __popcll(bal[k] & below)] = k * (WAVES * 64) + tid;
        }
        total = before;
        __syncthreads();
        // BATCH list entries at a time, one a lane (read once per wave, then
        // handed out uniform by readlane: no LDS wait per row); the next
        // batch's row loads in flight while this one is added.  Entries past
        // the list repeat its last and are not added; a column past the row
        // loads a live one and is never stored -- no lane diverges.
        {
            const long long colc = live ? col : a.d - 1;
            float xa[BATCH], xb[BATCH];
            auto fetch = [&](float (&x)[BATCH], int i0) {
                const int n = total - i0 < BATCH ? total - i0 : BATCH;
                const int mine = list[i0 + (lane < n ? lane : n - 1)];
#pragma unroll
                for (int q = 0; q < BATCH; ++q) {
                    const long long t = base + __builtin_amdgcn_readlane(mine, q);
                    x[q] = ld<ST>(a.ct, t * a.d + colc);
                }
            };
            auto add = [&](const float (&x)[BATCH], int i0) {
                const int n = total - i0 < BATCH ? total - i0 : BATCH;
#pragma unroll
                for (int q = 0; q < BATCH; ++q) {
                    const float s = acc + x[q];
                    if (ST == 2) ovf |= q < n && pk_overflows_f16(s);
                    acc = q < n ? stored<ST>(s) : acc;
                }
            };
            if (total > 0) fetch(xa, 0);
            for (int i0 = 0; i0 < total; i0 += 2 * BATCH) {
                if (i0 + BATCH < total) fetch(xb, i0 + BATCH);
                add(xa, i0);
                if (i0 + BATCH >= total) break;
                if (i0 + 2 * BATCH < total) fetch(xa, i0 + 2 * BATCH);
                add(xb, i0 + BATCH);
            }
        }
        __syncthreads();  // the list is rewritten next round
    }
    if (live) {
        const long long o = v * a.d + col;
        if (ST == 0) ((float*)a.out)[o] = acc;
        else ((unsigned short*)a.out)[o] = ST == 1 ? pk_f32_to_bf16(acc) : pk_f32_to_f16(acc);
    }
    if (ovf && a.flag) atomicOr(a.flag, 1u);
}

}  // namespace

hipError_t embed_vjp_launch(const ScatterArgs& a, hipStream_t stream) {
    if (a.vocab == 0 || a.d == 0) return hipSuccess;
    if (a.tokens < 0 || a.tokens > (1ll << 31) - ROUND || a.vocab > 0x7fffffffll) return hipErrorInvalidValue;
    const dim3 grid((unsigned)a.vocab, (unsigned)((a.d + WAVES * 64 - 1) / (WAVES * 64)));
    switch (a.storage) {
        case 0: embed_vjp_kernel<0><<<grid, WAVES * 64, 0, stream>>>(a); break;
        case 1: embed_vjp_kernel<1><<<grid, WAVES * 64, 0, stream>>>(a); break;
        case 2: embed_vjp_kernel<2><<<grid, WAVES * 64, 0, stream>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace presk
