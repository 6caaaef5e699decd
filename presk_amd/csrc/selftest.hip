// Device self-test of the scalar functions (presk_hip_scalar_digest): the
// digest oracle/digest.c defines, computed with the executor's own device
// conversions and transcendentals over a block of their domain.
#include <hip/hip_runtime.h>

#include "devfmt.hpp"
#include "executor.hpp"

namespace presk {

namespace {

__device__ __forceinline__ unsigned long long mix64(unsigned long long z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// the f64 sample of the narrowings from f64 (oracle/digest.c pd_sample_f64_bits)
__device__ __forceinline__ unsigned long long sample_f64_bits(unsigned long long i) {
    unsigned long long r = mix64(i * 0x9e3779b97f4a7c15ull + 0x632be59bd9b4e019ull);
    if ((i & 3) == 3) return r;
    unsigned long long e = 1023 - 40 + (r >> 52) % 65, frac = r & ((1ull << 52) - 1);
    if ((i & 3) == 2) frac &= ~((1ull << 28) - 1) | (r >> 40 & 1);
    return (r & (1ull << 63)) | (e << 52) | frac;
}

// the argument sample of f64 function fn (oracle/digest.c pd_sample_f64_arg)
__device__ __forceinline__ unsigned long long sample_f64_arg(int fn, unsigned long long i) {
    const unsigned long long r = mix64(i * 0x9e3779b97f4a7c15ull + 0x2545f4914f6cdd1dull * (unsigned long long)(fn + 1));
    const unsigned long long cls = i & 7;
    if (cls == 0) return r;
    const unsigned long long m = mix64(r);
    const unsigned long long e = cls == 1 ? m % 2047 : 1023 - 30 + m % 43;
    return (r & (1ull << 63)) | (e << 52) | (r & ((1ull << 52) - 1));
}

__device__ double eval_f64(int fn, double x) {
    switch (fn) {
        case 40: return pk_exp(x);
        case 41: return pk_log(x);
        case 42: return pk_tanh(x);
        case 43: return pk_erf(x);
        case 44: return pk_sin(x);
        default: return pk_cos(x);
    }
}

// A double's narrowing as a native kernel performs it: the value is an f32
// when a kernel stores it, so these go through the f32 of the double only
// when it is exact; otherwise the f64 path of codes.rs:29-56, written here
// for the self-test alone.
__device__ unsigned long long narrow64(unsigned long long b, unsigned t, unsigned w) {
    const unsigned long long sign = (b >> 63) << (t + w), inf = ((1ull << w) - 1) << t, mag = b & ~(1ull << 63);
    if (mag > (0x7ffull << 52)) return sign | inf | (1ull << (t - 1)) | ((mag >> (52 - t)) & ((1ull << (t - 1)) - 1));
    const int field = (int)(mag >> 52);
    if (field == 0) return sign;
    const unsigned long long sig = (mag & ((1ull << 52) - 1)) | (1ull << 52);
    const int e = field - 1023, bias = (1 << (w - 1)) - 1, emin = 1 - bias;
    const int shift = 52 - (int)t + (emin - e > 0 ? emin - e : 0);
    unsigned long long q = 0;
    if (shift <= 63) {
        const unsigned long long low = sig & ((1ull << shift) - 1), half = 1ull << (shift - 1);
        q = sig >> shift;
        if (low > half || (low == half && (q & 1))) q += 1;
    }
    unsigned long long code = e >= emin ? ((unsigned long long)(e + bias - 1) << t) + q : q;
    return sign | (code > inf ? inf : code);
}

__device__ const float kDivisors[16] = {1.f, 1.0000001f, 1.5f, 1.9999999f, 2.f, 3.1415927f, 7.f, 10.f, 100.25f, 1000.3f,
                                         12345.678f, 65535.9f, 1048577.f, 8388607.5f, 16777215.f, 16777216.f};

__device__ unsigned eval1(int fn, unsigned long long i) {
    const float x = pk_float((unsigned)i);
    switch (fn) {
        case 0: return pk_bits(pk_expf(x));
        case 1: return pk_bits(pk_logf(x));
        case 2: return pk_bits(pk_tanhf(x));
        case 3: return pk_bits(pk_erff(x));
        case 4: return pk_bits(pk_sinf(x));
        case 5: return pk_bits(pk_cosf(x));
        // expf through the softmax's fast path where it applies: expf's bits
        case 6: return pk_bits(pk_expf_le0_ok(x) ? pk_expf_le0(x) : pk_expf(x));
        // x / z for a table of divisors z >= 1: the softmax's quotient
        // (Markstein's step where it applies, else the division) and the
        // correctly rounded division itself
        case 7: case 8: {
            const float z = kDivisors[(i >> 3) % 16];
            return pk_bits(fn == 8 || !pk_div_by_ok(x, z) ? x / z : pk_div_by(x, z, 1.f / z));
        }
        case 10: return pk_f32_to_bf16(x);
        case 11: return pk_f32_to_f16(x);
        case 12: return pk_f32_to_e8m15(x);
        case 20: return pk_bits(pk_bf16_to_f32((unsigned short)i));
        case 21: return pk_bits(pk_f16_to_f32((unsigned short)i));
        case 22: return pk_bits(pk_e8m15_to_f32((unsigned)i));
        case 30: return (unsigned)narrow64(sample_f64_bits(i), 10, 5);
        case 31: return (unsigned)narrow64(sample_f64_bits(i), 15, 8);
        case 32: return pk_overflows_f16(x) ? 1u : 0u;
        case 33: return pk_overflows_e8m15(x) ? 1u : 0u;
        // f64 functions over their argument sample, the result folded to 32 bits
        case 40: case 41: case 42: case 43: case 44: case 45:
            return (unsigned)(mix64(pk_bits64(eval_f64(fn, pk_double(sample_f64_arg(fn, i))))) >> 32);
        default: return 0;
    }
}

// FAST mode's functions against the interpreter's (fn 50: expf, 51: erff):
// the distance in units in the last place between the two results, the f32
// bit patterns ordered as integers (-0 and +0 one point), two NaNs 0 apart
// and a NaN from a number 2^32
__device__ __forceinline__ long long ordered(unsigned b) {
    const long long m = b & 0x7fffffffu;
    return (b >> 31) ? -m : m;
}
// the divisors of the division scans (fn 70-77): sqrt 2 and sqrt(2 pi) as
// GELU and its derivative divide by them, small odd parts, a significand of
// all ones, a subnormal, a large and a small magnitude
__device__ float scan_divisor(int k) {
    switch (k) {
        case 0: return 0x1.6a09e6p+0f;
        case 1: return 0x1.40d932p+1f;
        case 2: return 3.0f;
        case 3: return 0x1.99999ap-4f;
        case 4: return 0x1.fffffep+0f;
        case 5: return 0x1.16c2p-133f;
        case 6: return 0x1.2eec2ep+101f;
        default: return -6.0f;
    }
}
__device__ unsigned long long ulp_distance(int fn, unsigned long long i) {
    const float x = pk_float((unsigned)i);
    if (fn >= 70) {
        // pk_div_rc against the correctly rounded division: 1 where the bits
        // differ (two NaNs agree)
        const float c = scan_divisor(fn - 70);
        const float a = pk_div_rc(x, 1.0 / (double)c), b = x / c;
        if (a != a || b != b) return (a != a) == (b != b) ? 0ull : 1ull;
        return pk_bits(a) != pk_bits(b) ? 1ull : 0ull;
    }
    float a, b;
    if (fn == 50) {
        a = pk_expf_fast(x);
        b = pk_expf(x);
    } else {
        a = pk_erff_fast(x);
        b = pk_erff(x);
    }
    if (a != a || b != b) return (a != a) == (b != b) ? 0ull : 1ull << 32;
    const long long d = ordered(pk_bits(a)) - ordered(pk_bits(b));
    return (unsigned long long)(d < 0 ? -d : d);
}

// the largest distance over [lo, lo + n) (fn 50, 51) or the count of inputs
// at a nonzero distance (fn 60, 61; fn 70-77 the count of dividends whose
// quotients differ)
__global__ void __launch_bounds__(256) ulp_kernel(int fn, unsigned long long lo, unsigned long long n,
                                                  unsigned long long per_thread, unsigned long long* out) {
    const unsigned long long t = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x;
    const bool count = fn >= 60;
    const int f = fn >= 70 ? fn : count ? fn - 10 : fn;
    unsigned long long acc = 0;
    const unsigned long long first = t * per_thread;
    for (unsigned long long j = 0; j < per_thread; ++j) {
        const unsigned long long k = first + j;
        if (k >= n) break;
        const unsigned long long d = ulp_distance(f, lo + k);
        acc = count ? acc + (d != 0) : (d > acc ? d : acc);
    }
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_down(acc, off, 64);
        acc = count ? acc + o : (o > acc ? o : acc);
    }
    __shared__ unsigned long long part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        if (count) {
            atomicAdd(out, part[0] + part[1] + part[2] + part[3]);
        } else {
            unsigned long long m = part[0];
            for (int q = 1; q < 4; ++q) m = part[q] > m ? part[q] : m;
            atomicMax(out, m);
        }
    }
}

__global__ void __launch_bounds__(256) digest_kernel(int fn, unsigned long long lo, unsigned long long n,
                                                     unsigned long long per_thread, unsigned long long* out) {
    const unsigned long long t = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x;
    unsigned long long acc = 0;
    const unsigned long long first = t * per_thread;
    for (unsigned long long j = 0; j < per_thread; ++j) {
        const unsigned long long k = first + j;
        if (k >= n) break;
        const unsigned long long i = lo + k;
        acc += mix64((i << 32) | eval1(fn, i));
    }
    // wave then block sum (order-free: the digest is a sum mod 2^64)
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_down(acc, off, 64);
    __shared__ unsigned long long part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd(out, part[0] + part[1] + part[2] + part[3]);
}

}  // namespace

hipError_t scalar_digest(int fn, uint64_t lo, uint64_t hi, uint64_t* digest) {
    const int known[] = {0, 1, 2, 3, 4, 5, 6, 7, 8, 10, 11, 12, 20, 21, 22, 30, 31, 32, 33, 40, 41, 42, 43, 44, 45,
                         50, 51, 60, 61, 70, 71, 72, 73, 74, 75, 76, 77};
    bool ok = false;
    for (int f : known) ok |= f == fn;
    if (!ok || hi < lo) return hipErrorInvalidValue;
    const unsigned long long n = hi - lo;
    unsigned long long* d = nullptr;
    hipError_t e = hipMalloc(&d, sizeof *d);
    if (e != hipSuccess) return e;
    e = hipMemset(d, 0, sizeof *d);
    const unsigned long long per_thread = 64, threads = (n + per_thread - 1) / per_thread;
    const unsigned long long blocks = (threads + 255) / 256;
    if (e == hipSuccess && n) {
        if (fn >= 50)
            ulp_kernel<<<dim3((unsigned)blocks), dim3(256)>>>(fn, lo, n, per_thread, d);
        else
            digest_kernel<<<dim3((unsigned)blocks), dim3(256)>>>(fn, lo, n, per_thread, d);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    unsigned long long h = 0;
    if (e == hipSuccess) e = hipMemcpy(&h, d, sizeof h, hipMemcpyDeviceToHost);
    hipFree(d);
    *digest = h;
    return e;
}

}  // namespace presk
