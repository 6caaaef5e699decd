// The host's conversion of a buffer at a kernel's edge, on the device:
// Buf::of(to, b.to_f64()) (crates/presk-rt/src/lib.rs:868-876), called where a
// mixed realization hands a kernel a buffer another site wrote in another
// type (crates/presk-kernel/src/host.rs:793-829).  A buffer of the kernel's
// own type is lent as it is; otherwise each element is widened to f64
// exactly, then stored as `to` stores an f64: f32 rounds once to nearest
// even, bf16 rounds to f32 and then to bf16 (two roundings, as the reference
// does), binary16 and e8m15 round once from the f64.  NaNs follow the
// reference host's x86 casts: widening quiets and keeps the payload,
// narrowing to f32 quiets and keeps the payload's top bits.  The guard:
// storing a finite value at or past binary16's or e8m15's overflow threshold
// (presk_rt::codes::overflows).
#include <hip/hip_runtime.h>

#include "convert.hpp"
#include "devfmt.hpp"

namespace presk {

namespace {

__device__ __forceinline__ unsigned long long bits64(double x) { return (unsigned long long)__double_as_longlong(x); }
__device__ __forceinline__ double from_bits64(unsigned long long b) { return __longlong_as_double((long long)b); }

// f32 -> f64, exact; a NaN made quiet with its payload moved up
__device__ __forceinline__ double widen(float x) {
    const unsigned b = pk_bits(x);
    if ((b & 0x7fffffffu) > 0x7f800000u)
        return from_bits64(((unsigned long long)(b >> 31) << 63) | 0x7ff0000000000000ull |
                           ((unsigned long long)((b & 0x7fffffu) | 0x400000u) << 29));
    return (double)x;
}

// f64 -> f32, to nearest even; a NaN made quiet with its payload's top bits
__device__ __forceinline__ float narrow32(double x) {
    const unsigned long long b = bits64(x);
    if ((b & 0x7fffffffffffffffull) > 0x7ff0000000000000ull)
        return pk_float((unsigned)(b >> 63) << 31 | 0x7f800000u | (((unsigned)(b >> 29) & 0x7fffffu) | 0x400000u));
    return (float)x;
}

// f64 -> a binary format of `t` fraction bits and `w` exponent bits, one
// rounding to nearest even: past the largest finite number, the infinity; a
// NaN quiet with the top t-1 bits of its payload; below the format's
// subnormals, a signed zero.
template <int t, int w>
__device__ __forceinline__ unsigned narrow_bits(double x) {
    const unsigned long long b = bits64(x);
    const unsigned sign = (unsigned)(b >> 63) << (t + w);
    const unsigned inf = ((1u << w) - 1u) << t;
    const unsigned long long mag = b & 0x7fffffffffffffffull;
    if (mag > 0x7ff0000000000000ull) return sign | inf | (1u << (t - 1)) | (unsigned)((mag >> (52 - t)) & ((1ull << (t - 1)) - 1));
    if (mag == 0x7ff0000000000000ull) return sign | inf;
    const int field = (int)(mag >> 52);
    if (field == 0) return sign;  // an f64 subnormal: far below every format here
    constexpr int bias = (1 << (w - 1)) - 1;
    const int e = field - 1023;
    const unsigned long long sig = (mag & 0xfffffffffffffull) | 0x10000000000000ull;  // 53 bits
    // drop 52 - t bits, and below the normal range as many more as the
    // exponent falls short (the leading one then lands in the fraction)
    const int drop = 52 - t + (e < 1 - bias ? (1 - bias) - e : 0);
    unsigned long long q;
    if (drop >= 64) {
        q = 0;
    } else {
        q = sig >> drop;
        const unsigned long long rest = sig & ((1ull << drop) - 1), half = 1ull << (drop - 1);
        if (rest > half || (rest == half && (q & 1))) ++q;
    }
    // a normal number's field is e + bias, its leading one carried in q
    const unsigned long long code = e >= 1 - bias ? ((unsigned long long)(e + bias - 1) << t) + q : q;
    return sign | (unsigned)(code < inf ? code : inf);
}

template <int T>
__device__ __forceinline__ double load_f64(const void* p, long long i) {
    if (T == 0) return ((const double*)p)[i];
    if (T == 1) return widen(((const float*)p)[i]);
    if (T == 2) return widen(pk_bf16_to_f32(((const unsigned short*)p)[i]));
    if (T == 4) return widen(pk_f16_to_f32(((const unsigned short*)p)[i]));
    return widen(pk_e8m15_to_f32(pk_ld24((const unsigned char*)p, i)));
}

template <int T>
__device__ __forceinline__ void store_f64(void* p, long long i, double x) {
    if (T == 0) ((double*)p)[i] = x;
    else if (T == 1) ((float*)p)[i] = narrow32(x);
    else if (T == 2) ((unsigned short*)p)[i] = pk_f32_to_bf16(narrow32(x));
    else if (T == 4) ((unsigned short*)p)[i] = (unsigned short)narrow_bits<10, 5>(x);
    else pk_st24((unsigned char*)p, i, narrow_bits<15, 8>(x));
}

template <int F, int T>
__global__ void __launch_bounds__(256) convert_kernel(const void* src, void* dst, long long n, unsigned* flag) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const double x = load_f64<F>(src, i);
    bool ovf = false;
    if (T == 4 || T == 5) {
        // the midpoints above the largest finite numbers: binary16 65520,
        // e8m15 (2 - 2^-16) * 2^127
        const double a = x < 0 ? -x : x;
        const double threshold = T == 4 ? 65520.0 : 0x1.ffffp127;
        ovf = a == a && a != __builtin_inf() && a >= threshold;
    }
    store_f64<T>(dst, i, x);
    if (ovf && flag) atomicOr(flag, 1u);
}

template <int F>
hipError_t launch_from(int to, const void* src, void* dst, long long n, unsigned* flag, hipStream_t s) {
    const unsigned grid = (unsigned)((n + 255) / 256);
    switch (to) {
        case 0: convert_kernel<F, 0><<<grid, 256, 0, s>>>(src, dst, n, flag); break;
        case 1: convert_kernel<F, 1><<<grid, 256, 0, s>>>(src, dst, n, flag); break;
        case 2: convert_kernel<F, 2><<<grid, 256, 0, s>>>(src, dst, n, flag); break;
        case 4: convert_kernel<F, 4><<<grid, 256, 0, s>>>(src, dst, n, flag); break;
        case 5: convert_kernel<F, 5><<<grid, 256, 0, s>>>(src, dst, n, flag); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

size_t width(int t) { return t == 0 ? 8 : t == 1 ? 4 : (t == 2 || t == 4) ? 2 : t == 5 ? 3 : 0; }


// ---- .psk.d leaves (crates/presk-data/src/lib.rs:205-219, Enc::decode) ------
// A real leaf's elements are codes of its encoding: f64, f32 and bf16 are the
// conversions above; a format given by its parameters (encoding 3) is decoded
// to the f64 it denotes (crates/presk-format/src/lib.rs:460-476,
// Float::decode), exactly, then stored as Buf::of stores an f64.  Codes are
// `width` bytes, little-endian; bits above the format's are ignored.
__device__ __forceinline__ double exp2i(int k) {
    return k >= -1022 ? from_bits64((unsigned long long)(k + 1023) << 52) : from_bits64(1ull << (k + 1074));
}

__device__ __forceinline__ double format_decode(unsigned long long code, const PskFormat& f) {
    const int t = f.p - 1;
    const bool negative = (code >> (f.bits - 1)) & 1ull;
    const unsigned long long top = (1ull << f.ebits) - 1, tmask = (1ull << t) - 1;
    const unsigned long long field = (code >> t) & top, trailing = code & tmask;
    double v;
    if (f.specials == 0 && field == top) v = trailing == 0 ? __builtin_inf() : from_bits64(0x7ff8000000000000ull);
    else if (f.specials == 1 && field == top && trailing == tmask) v = from_bits64(0x7ff8000000000000ull);
    else if (field == 0) v = f.subnormals ? (double)trailing * exp2i(f.emin - t) : 0.0;
    else v = (double)((1ull << t) | trailing) * exp2i((int)field - (1 - f.emin) - t);
    // negation flips the sign bit, a NaN's included
    return negative ? from_bits64(bits64(v) ^ 0x8000000000000000ull) : v;
}

template <int T>
__global__ void __launch_bounds__(256) format_decode_kernel(const unsigned char* src, PskFormat f, long long n, void* dst,
                                                            unsigned* flag) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    unsigned long long code = 0;
    for (int b = 0; b < f.width; ++b) code |= (unsigned long long)src[i * f.width + b] << (8 * b);
    const double x = format_decode(code, f);
    if (T == 4 || T == 5) {
        const double a = x < 0 ? -x : x;
        const double threshold = T == 4 ? 65520.0 : 0x1.ffffp127;
        if (a == a && a != __builtin_inf() && a >= threshold && flag) atomicOr(flag, 1u);
    }
    store_f64<T>(dst, i, x);
}

// an idx[N] leaf: the smallest unsigned integer holding N-1, widened to i64
__global__ void __launch_bounds__(256) idx_widen_kernel(const unsigned char* src, int width, long long n, long long* dst) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    unsigned long long v = 0;
    for (int b = 0; b < width; ++b) v |= (unsigned long long)src[i * width + b] << (8 * b);
    dst[i] = (long long)v;
}

// ---- dropout masks (crates/presk-kernel/src/host.rs:1893-1926) ----------------
// Element e is 1/(1-rate) where the key's e-th uniform draw is below 1-rate,
// else 0, stored as Buf::of stores it (store_f64).  The draw is rand_chacha's
// ChaCha20Rng read from word 2e: u64 e = words 2e, 2e+1 (the low one first)
// of the stream -- block e / 8, the counter in state words 12-13, stream 0 in
// 14-15 -- and uniform01 = (u64 >> 11) / 2^53.  A thread computes one block,
// eight elements: the mask is counter-based, each piece independent.
__device__ __forceinline__ unsigned rotl32(unsigned x, int r) { return (x << r) | (x >> (32 - r)); }

__device__ __forceinline__ void chacha20_block(const unsigned (&k)[8], unsigned long long ctr, unsigned (&o)[16]) {
    unsigned x[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u, k[0], k[1], k[2], k[3],
                      k[4], k[5], k[6], k[7], (unsigned)ctr, (unsigned)(ctr >> 32), 0u, 0u};
    unsigned s[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = x[i];
    auto qr = [&](int a, int b, int c, int d) {
        x[a] += x[b]; x[d] = rotl32(x[d] ^ x[a], 16);
        x[c] += x[d]; x[b] = rotl32(x[b] ^ x[c], 12);
        x[a] += x[b]; x[d] = rotl32(x[d] ^ x[a], 8);
        x[c] += x[d]; x[b] = rotl32(x[b] ^ x[c], 7);
    };
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        qr(0, 4, 8, 12); qr(1, 5, 9, 13); qr(2, 6, 10, 14); qr(3, 7, 11, 15);
        qr(0, 5, 10, 15); qr(1, 6, 11, 12); qr(2, 7, 8, 13); qr(3, 4, 9, 14);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = x[i] + s[i];
}

template <int T>
__global__ void __launch_bounds__(256) dropout_kernel(const unsigned* key, double keep, double scale, long long n,
                                                      void* out) {
    const long long b = (long long)blockIdx.x * 256 + threadIdx.x;
    if (8 * b >= n) return;
    unsigned k[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) k[i] = key[i];   // the key's 32 bytes as little-endian words
    unsigned w[16];
    chacha20_block(k, (unsigned long long)b, w);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const long long e = 8 * b + j;
        if (e >= n) break;
        const unsigned long long u64 = (unsigned long long)w[2 * j] | ((unsigned long long)w[2 * j + 1] << 32);
        const double u = (double)(u64 >> 11) / 9007199254740992.0;
        store_f64<T>(out, e, u < keep ? scale : 0.0);
    }
}
}  // namespace

int convert_type(const char* name) {
    const std::string s = name ? name : "";
    if (s == "f64") return 0;
    if (s == "f32") return 1;
    if (s == "bf16") return 2;
    if (s == "f16") return 4;
    if (s == "e8m15") return 5;
    return -1;
}

hipError_t convert_launch(const void* src, int from, void* dst, int to, long long n, unsigned* flag, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (from == to) return hipMemcpyAsync(dst, src, (size_t)n * width(to), hipMemcpyDeviceToDevice, s);
    if ((n + 255) / 256 > 0x7fffffffLL) return hipErrorInvalidValue;
    switch (from) {
        case 0: return launch_from<0>(to, src, dst, n, flag, s);
        case 1: return launch_from<1>(to, src, dst, n, flag, s);
        case 2: return launch_from<2>(to, src, dst, n, flag, s);
        case 4: return launch_from<4>(to, src, dst, n, flag, s);
        case 5: return launch_from<5>(to, src, dst, n, flag, s);
    }
    return hipErrorInvalidValue;
}

hipError_t pskd_decode_launch(const void* src, int enc, const PskFormat& f, long long n, void* dst, int to, unsigned* flag,
                              hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (enc == 0 || enc == 1 || enc == 2) return convert_launch(src, enc, dst, to, n, flag, s);
    if (enc != 3 || (n + 255) / 256 > 0x7fffffffLL) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)((n + 255) / 256);
    const unsigned char* b = (const unsigned char*)src;
    switch (to) {
        case 0: format_decode_kernel<0><<<grid, 256, 0, s>>>(b, f, n, dst, flag); break;
        case 1: format_decode_kernel<1><<<grid, 256, 0, s>>>(b, f, n, dst, flag); break;
        case 2: format_decode_kernel<2><<<grid, 256, 0, s>>>(b, f, n, dst, flag); break;
        case 4: format_decode_kernel<4><<<grid, 256, 0, s>>>(b, f, n, dst, flag); break;
        case 5: format_decode_kernel<5><<<grid, 256, 0, s>>>(b, f, n, dst, flag); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t pskd_idx_launch(const void* src, int width, long long n, long long* dst, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if ((n + 255) / 256 > 0x7fffffffLL || !(width == 1 || width == 2 || width == 4 || width == 8)) return hipErrorInvalidValue;
    idx_widen_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>((const unsigned char*)src, width, n, dst);
    return hipGetLastError();
}

hipError_t dropout_launch(const void* key, double rate, int type, long long n, void* dst, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const double keep = 1.0 - rate, scale = 1.0 / (1.0 - rate);
    const long long blocks = (n + 7) / 8;
    const dim3 grid((unsigned)((blocks + 255) / 256)), block(256);
    const unsigned* k = (const unsigned*)key;
    switch (type) {
        case 0: dropout_kernel<0><<<grid, block, 0, s>>>(k, keep, scale, n, dst); break;
        case 1: dropout_kernel<1><<<grid, block, 0, s>>>(k, keep, scale, n, dst); break;
        case 2: dropout_kernel<2><<<grid, block, 0, s>>>(k, keep, scale, n, dst); break;
        case 4: dropout_kernel<4><<<grid, block, 0, s>>>(k, keep, scale, n, dst); break;
        case 5: dropout_kernel<5><<<grid, block, 0, s>>>(k, keep, scale, n, dst); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace presk
