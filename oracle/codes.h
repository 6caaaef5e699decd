/* oracle/codes.h -- TEST INFRASTRUCTURE ONLY (the parity oracle).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * include, link or run anything under oracle/.  The product (presk_amd/) never
 * does.
 *
 * The storage formats' conversions, restated from the reference's bit recipes:
 *   bf16   : presk_rt::f32_to_bf16 / bf16_to_f32   crates/presk-rt/src/lib.rs:228-241
 *   f16    : codes::{narrow, wide_bits, f32_to_f16, f64_to_f16, f16_to_f32}
 *                                                   crates/presk-rt/src/codes.rs:29-87
 *   e8m15  : codes::{f32_to_e8m15, f64_to_e8m15, e8m15_to_f32}
 *                                                   crates/presk-rt/src/codes.rs:89-110
 *   guard  : codes::{overflow_threshold, overflows} crates/presk-rt/src/codes.rs:112-136
 *
 * Pinned by tests/test_oracle_codes.py against the reference's own C runtime
 * (crates/presk-export-c/c/presk_rt.h, compiled into oracle/_ref by
 * oracle/Makefile) over every f32 and every code, and against numpy's IEEE
 * float16 rounding for every non-NaN f32.
 */
#ifndef PRESK_ORACLE_CODES_H
#define PRESK_ORACLE_CODES_H

#include <stdint.h>
#include <string.h>

static inline uint32_t oc_bits32(float x) { uint32_t b; memcpy(&b, &x, 4); return b; }
static inline float oc_float(uint32_t b) { float x; memcpy(&x, &b, 4); return x; }
static inline uint64_t oc_bits64(double x) { uint64_t b; memcpy(&b, &x, 8); return b; }
static inline double oc_double(uint64_t b) { double x; memcpy(&x, &b, 8); return x; }

/* ---- bf16: the top half of an f32, rounded to nearest even ------------- */
static inline uint16_t oc_f32_to_bf16(float x)
{
    uint32_t b = oc_bits32(x);
    if ((b & 0x7fffffffu) > 0x7f800000u)          /* NaN: quiet, sign kept */
        return (uint16_t)((b >> 16) | 0x0040u);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
static inline float oc_bf16_to_f32(uint16_t h) { return oc_float((uint32_t)h << 16); }

/* ---- the generic IEEE narrowing from the f64 of bits `b` --------------
 * to a format of `t` trailing bits and `w` exponent bits: round to nearest,
 * ties to even, once; overflow to the infinity; a NaN quiet with the top
 * t-1 payload bits; an f64 subnormal to a signed zero. */
static inline uint64_t oc_narrow(uint64_t b, unsigned t, unsigned w)
{
    const uint64_t sign = (b >> 63) << (t + w);
    const uint64_t inf = (((uint64_t)1 << w) - 1) << t;
    const uint64_t mag = b & ~((uint64_t)1 << 63);
    if (mag > (uint64_t)0x7ff << 52) {
        uint64_t keep = (mag >> (52 - t)) & (((uint64_t)1 << (t - 1)) - 1);
        return sign | inf | ((uint64_t)1 << (t - 1)) | keep;
    }
    const int field = (int)(mag >> 52);
    if (field == 0)
        return sign;
    const uint64_t sig = (mag & (((uint64_t)1 << 52) - 1)) | ((uint64_t)1 << 52);
    const int e = field - 1023;                       /* unbiased exponent */
    const int bias = (1 << (w - 1)) - 1;
    const int emin = 1 - bias;
    const int denorm = emin - e > 0 ? emin - e : 0;   /* extra shift below normal */
    const int shift = 52 - (int)t + denorm;
    uint64_t q = 0;
    if (shift <= 63) {
        const uint64_t low = sig & (((uint64_t)1 << shift) - 1);
        const uint64_t half = (uint64_t)1 << (shift - 1);
        q = sig >> shift;
        if (low > half || (low == half && (q & 1)))
            q += 1;
    }
    uint64_t code = e >= emin ? ((uint64_t)(e + bias - 1) << t) + q : q;
    if (code > inf)
        code = inf;
    return sign | code;
}

/* An f32's bits moved into an f64's without a conversion (a NaN's payload and
 * quiet bit kept as they are). */
static inline uint64_t oc_wide_bits(float x)
{
    uint32_t b = oc_bits32(x);
    if ((b & 0x7fffffffu) > 0x7f800000u)
        return ((uint64_t)(b >> 31) << 63) | ((uint64_t)0x7ff << 52) | ((uint64_t)(b & 0x7fffffu) << 29);
    return oc_bits64((double)x);
}

/* ---- binary16 ----------------------------------------------------------- */
static inline uint16_t oc_f32_to_f16(float x) { return (uint16_t)oc_narrow(oc_wide_bits(x), 10, 5); }
static inline uint16_t oc_f64_to_f16(double x) { return (uint16_t)oc_narrow(oc_bits64(x), 10, 5); }
static inline float oc_f16_to_f32(uint16_t c)
{
    const uint32_t sign = (uint32_t)(c & 0x8000u) << 16;
    const uint32_t field = (c >> 10) & 0x1fu, frac = c & 0x3ffu;
    uint32_t mag;
    if (field == 0x1f)
        mag = frac == 0 ? 0x7f800000u : (0x7fc00000u | (frac << 13));
    else if (field == 0)
        mag = oc_bits32((float)frac * oc_float(0x33800000u));   /* frac * 2^-24, exact */
    else
        mag = ((field + 112u) << 23) | (frac << 13);
    return oc_float(sign | mag);
}

/* ---- e8m15: the top 24 bits of an f32, 3 bytes little-endian ------------ */
static inline uint32_t oc_f32_to_e8m15(float x)
{
    uint32_t b = oc_bits32(x);
    if ((b & 0x7fffffffu) > 0x7f800000u)
        return (b >> 8) | 0x4000u;
    return (b + 0x7fu + ((b >> 8) & 1u)) >> 8;
}
static inline uint32_t oc_f64_to_e8m15(double x) { return (uint32_t)oc_narrow(oc_bits64(x), 15, 8); }
static inline float oc_e8m15_to_f32(uint32_t c) { return oc_float(c << 8); }

/* ---- the overflow guard: a finite value whose narrowing is an infinity -- */
static inline int oc_overflows_f16(double x)
{
    double a = x < 0 ? -x : x;
    return a == a && a != 1.0 / 0.0 && a >= 65520.0;
}
static inline int oc_overflows_e8m15(double x)
{
    double a = x < 0 ? -x : x;
    return a == a && a != 1.0 / 0.0 && a >= (double)oc_float(0x7f7fff80u);
}

#endif
