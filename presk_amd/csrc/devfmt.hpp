// Device-side storage conversions and f32/f64 transcendentals (gfx950).
//
// Included by the hand-written kernels and, as text, by every kernel the
// generic printer builds with hiprtc, so it uses compiler builtins only.
// Compile with -ffp-contract=off and correctly rounded f32 division/sqrt:
// every function below must round each f32 operation where its reference
// does, for equal bits.
//
// Conversions, from the reference's bit recipes:
//   bf16   crates/presk-rt/src/lib.rs:228-241
//   f16    crates/presk-rt/src/codes.rs:29-87 (IEEE round to nearest even,
//          overflow to infinity, a NaN quiet with its top 9 payload bits)
//   e8m15  crates/presk-rt/src/codes.rs:89-110 (the top 24 bits of the f32)
//   guard  crates/presk-rt/src/codes.rs:112-136 (a finite value whose
//          narrowing is an infinity)
// Transcendentals: the kernel interpreter's (exec.rs:158-170), the `libm`
// crate 0.2.16 = musl 1.1.22 = fdlibm's f32 method; same reductions,
// coefficients and operation order as crates/presk-export-c/c/presk_libm.c
// (expf :1605, logf :1811, expm1f :436, tanhf :1915, erff :2542, sinf :2054,
// cosf :2213).
//
// The f64 functions of the interpreter's f64 arm (exec.rs:115-130): the same
// crate's double functions, musl's exp/log/expm1/tanh/erf/sin/cos (presk_libm.c
// lines at each below).
//
// Each f32 function is checked over every f32 input on the GPU against the
// reference's compiled C, each f64 function over a sample of 2^24 arguments
// (tests/test_gpu_scalar.py, digests in tests/golden/digests.json).
//
// Notices.  The method, constants and operation order restated here are
// those of the following sources, whose terms ask that these notices be
// kept with any work derived from them:
//
//   musl libc 1.1.22 -- Copyright (c) 2005-2014 Rich Felker, et al.
//   Permission is hereby granted, free of charge, to any person obtaining
//   a copy of this software and associated documentation files (the
//   "Software"), to deal in the Software without restriction, including
//   without limitation the rights to use, copy, modify, merge, publish,
//   distribute, sublicense, and/or sell copies of the Software, and to
//   permit persons to whom the Software is furnished to do so, subject to
//   the following conditions: The above copyright notice and this
//   permission notice shall be included in all copies or substantial
//   portions of the Software.  THE SOFTWARE IS PROVIDED "AS IS", WITHOUT
//   WARRANTY OF ANY KIND, EXPRESS OR IMPLIED.
//
//   fdlibm (via FreeBSD msun) -- Copyright (C) 1993 by Sun Microsystems,
//   Inc. All rights reserved.  Developed at SunPro, a Sun Microsystems,
//   Inc. business.  Permission to use, copy, modify, and distribute this
//   software is freely granted, provided that this notice is preserved.
//   (The f32 conversions of these functions are by Ian Lance Taylor,
//   Cygnus Support, and Bruce D. Evans, under the same terms.)
#pragma once

#define PK_DEV __device__ __forceinline__

PK_DEV unsigned pk_bits(float x) { return __builtin_bit_cast(unsigned, x); }
PK_DEV float pk_float(unsigned b) { return __builtin_bit_cast(float, b); }

// ---- bf16 ---------------------------------------------------------------------
PK_DEV float pk_bf16_to_f32(unsigned short h) { return pk_float((unsigned)h << 16); }
// Round to nearest even; a NaN keeps its sign and top payload bits and is
// quieted (bit 6 set).  gfx950's v_cvt_pk_bf16_f32 computes exactly this,
// denormals included (pinned by the all-f32 digest of the conversion): one
// instruction against six for the integer form (b + 0x7fff + ((b >> 16) &
// 1)) >> 16 with a select for a NaN.  Written as assembly so that the
// compiler cannot fold the rounding into the operation that produced x (a
// product and its rounding to 16 bits as one mixed-precision FMA rounds
// once where the interpreter rounds twice).
PK_DEV unsigned short pk_f32_to_bf16(float x) {
    unsigned r;
    asm("v_cvt_pk_bf16_f32 %0, %1, 0" : "=v"(r) : "v"(x));
    return (unsigned short)r;
}

// ---- binary16 -----------------------------------------------------------------
// Exact; a NaN is quieted with its payload kept (v_cvt_f32_f16: pinned by the
// digest over every code)
PK_DEV float pk_f16_to_f32(unsigned short c) { return (float)__builtin_bit_cast(_Float16, c); }
// Round to nearest even, overflow to infinity, subnormals kept; a NaN keeps
// its sign and top payload bits and is quieted.  v_cvt_f16_f32 computes
// exactly this (pinned by the all-f32 digest of the conversion); assembly,
// as for bf16, so that no product is rounded to binary16 in one step by a
// mixed-precision FMA (v_fma_mixlo_f16), which the interpreter rounds twice.
PK_DEV unsigned short pk_f32_to_f16(float x) {
    unsigned r;
    asm("v_cvt_f16_f32 %0, %1" : "=v"(r) : "v"(x));
    return (unsigned short)r;
}
PK_DEV bool pk_overflows_f16(float x) {
    unsigned a = pk_bits(x) & 0x7fffffffu;
    return a >= 0x477ff000u && a < 0x7f800000u;
}

// ---- e8m15: 3 bytes, little-endian, the f32's top 24 bits ---------------------
PK_DEV float pk_e8m15_to_f32(unsigned c) { return pk_float(c << 8); }
PK_DEV unsigned pk_f32_to_e8m15(float x) {
    const unsigned b = pk_bits(x);
    const unsigned nan = (b >> 8) | 0x4000u, rne = (b + 0x7fu + ((b >> 8) & 1u)) >> 8;
    return (b & 0x7fffffffu) > 0x7f800000u ? nan : rne;
}
PK_DEV bool pk_overflows_e8m15(float x) {
    unsigned a = pk_bits(x) & 0x7fffffffu;
    return a >= 0x7f7fff80u && a < 0x7f800000u;
}
PK_DEV unsigned pk_ld24(const unsigned char* p, long long e) {
    return (unsigned)p[3 * e] | ((unsigned)p[3 * e + 1] << 8) | ((unsigned)p[3 * e + 2] << 16);
}
// int4 weights (crates/presk-rt/src/quant.rs:333-337): element e is the
// nibble of byte e/2, the low one when e is even, two's complement
PK_DEV int pk_nibble(const unsigned char* p, long long e) {
    const unsigned b = p[e >> 1];
    const unsigned n = (e & 1) ? b >> 4 : b & 15u;
    return (int)(n << 28) >> 28;
}
PK_DEV void pk_st24(unsigned char* p, long long e, unsigned c) {
    p[3 * e] = (unsigned char)c;
    p[3 * e + 1] = (unsigned char)(c >> 8);
    p[3 * e + 2] = (unsigned char)(c >> 16);
}

// x / z correctly rounded, by Markstein's method for a divisor used many
// times (P. Markstein, "Computation of elementary functions on the IBM RISC
// System/6000 processor", IBM J. Res. Dev. 34(1), 1990; J.-M. Muller et al.,
// Handbook of Floating-Point Arithmetic, the theorem on the correction
// step): with rz = RN(1/z), q0 = RN(x * rz) lies within one ulp of x / z,
// the residual x - z * q0 is exact in an fma, and RN(q0 + r * rz) is
// RN(x / z) -- when neither the quotient nor the residual leaves the normal
// range.  pk_div_by_ok says when that holds (x zero, or |x| in [2^-100,
// 2^100] with z in [1, 2^24]: the quotient then lies in [2^-124, 2^100]);
// elsewhere the caller divides.
PK_DEV float pk_div_by(float x, float z, float rz) {
    const float q0 = x * rz;
    const float r = __builtin_fmaf(-q0, z, x);
    // a zero quotient keeps x's sign (the correction step would give +0)
    return x == 0.f ? q0 : __builtin_fmaf(r, rz, q0);
}
PK_DEV bool pk_div_by_ok(float x, float z) {
    const float ax = __builtin_fabsf(x);
    return z >= 1.f && z <= 16777216.f && (x == 0.f || (ax >= 0x1p-100f && ax <= 0x1p100f));
}

// Rust's `f as i64`: saturating, NaN to zero.
PK_DEV long long pk_i64(double x) {
    if (x != x) return 0;
    if (x >= 9223372036854775807.0) return 9223372036854775807LL;
    if (x <= -9223372036854775808.0) return (-9223372036854775807LL - 1);
    return (long long)x;
}

// ---- f32 transcendentals ---------------------------------------------------------
PK_DEV float pk_ldexpf(float y, int n) {
    if (n > 127) {
        y *= 0x1p127f;
        n -= 127;
        if (n > 127) {
            y *= 0x1p127f;
            n -= 127;
            if (n > 127) n = 127;
        }
    } else if (n < -126) {
        y *= 0x1p-102f;
        n += 102;
        if (n < -126) {
            y *= 0x1p-102f;
            n += 102;
            if (n < -126) n = -126;
        }
    }
    return y * pk_float((unsigned)(0x7f + n) << 23);
}

// expf's quotient r c / (2 - c): |r| <= 0.35, so 2 - c lies in [1.6, 2.4]
// and |r c| < 0.13.  Markstein's step on a reciprocal refined once from the
// hardware estimate (y0 = rcp(b), y = y0 + y0 (1 - b y0); q0 = a y,
// q = q0 + y (a - b q0), each in one fma) in place of the correctly rounded
// division's scale/fixup sequence.  Not correctly rounded in general: it
// gives the division's bits on every argument expf sees (pinned by the
// all-f32 digests of pk_expf and its softmax fast path).
PK_DEV float pk_expf_quot(float a, float b) {
    const float y0 = __builtin_amdgcn_rcpf(b);
    const float y = __builtin_fmaf(__builtin_fmaf(-b, y0, 1.0f), y0, y0);
    const float q0 = a * y;
    return __builtin_fmaf(__builtin_fmaf(-q0, b, a), y, q0);
}

// The same quotient for erff's rational approximations, whose denominators
// lie in [1, 50] there and whose numerators are bounded: the division's bits
// on every f32 (pinned by the all-f32 digest of erff).
PK_DEV float pk_erf_quot(float a, float b) { return pk_expf_quot(a, b); }

// fdlibm's expf, its branches written as selects (the same operations on
// every path, so the same bits): k = 0 is the general reduction with k = 0
// (x - 0 * ln2_hi is x, 0 * ln2_lo is 0), scalbnf is one ldexp, and the
// special inputs are chosen last.
PK_DEV float pk_expf(float x) {
    const float ln2_hi = 6.9314575195e-1f, ln2_lo = 1.4286067653e-6f, inv_ln2 = 1.4426950216e+0f;
    const float p1 = 1.6666625440e-1f, p2 = -2.7667332906e-3f;
    const unsigned bx = pk_bits(x);
    const bool neg = (bx >> 31) != 0;
    const unsigned ax = bx & 0x7fffffffu;
    // the reduction's multiple of ln2 (|x| below 104 here, so in range of int)
    const float xk = ax < 0x42d00000u ? x : 0.0f;
    const int kbig = (int)(inv_ln2 * xk + (neg ? -0.5f : 0.5f));
    const int k = ax > 0x3f851592u ? kbig : ax > 0x3eb17218u ? 1 - 2 * (int)neg : 0;
    const float fk = (float)k;
    const float hi = xk - fk * ln2_hi;
    const float lo = fk * ln2_lo;
    const float r = hi - lo;
    const float rr = r * r;
    const float c = r - rr * (p1 + rr * p2);
    const float y = 1.0f + (pk_expf_quot(r * c, 2.0f - c) - lo + hi);
    // y * 2^k as scalbnf computes it (k lies in [-150, 150]): its
    // pre-scaling by 2^127 or 2^-102 is exact, so the one rounding is that of
    // y * 2^k, which v_ldexp_f32 gives directly (denormals and overflow
    // included; k = 0 leaves y)
    float res = __builtin_amdgcn_ldexpf(y, k);
    res = ax <= 0x39000000u ? 1.0f + x : res;
    res = neg && ax >= 0x42cff1b5u ? 0.0f : res;
    res = !neg && ax >= 0x42b17218u ? x * 0x1p127f : res;
    return ax > 0x7f800000u ? x : res;
}

// pk_expf on (-87.34, 0] (a softmax's exp(x - m)): there no special input
// occurs and k lies in [-126, 0], so the same operations without the special
// cases' selects and scalbnf's pre-scaling give the same bits.
PK_DEV bool pk_expf_le0_ok(float x) {
    const unsigned b = pk_bits(x);
    return b == 0u || (b >= 0x80000000u && b < 0xc2aeac50u);
}
PK_DEV float pk_expf_le0(float x) {
    const float ln2_hi = 6.9314575195e-1f, ln2_lo = 1.4286067653e-6f, inv_ln2 = 1.4426950216e+0f;
    const float p1 = 1.6666625440e-1f, p2 = -2.7667332906e-3f;
    const unsigned ax = pk_bits(x) & 0x7fffffffu;
    const int k = ax > 0x3f851592u ? (int)(inv_ln2 * x + -0.5f) : ax > 0x3eb17218u ? -1 : 0;
    const float fk = (float)k;
    const float hi = x - fk * ln2_hi;
    const float lo = fk * ln2_lo;
    const float r = hi - lo;
    const float rr = r * r;
    const float c = r - rr * (p1 + rr * p2);
    const float y = 1.0f + (pk_expf_quot(r * c, 2.0f - c) - lo + hi);
    const float res = __builtin_amdgcn_ldexpf(y, k);   // y * 2^k, k in [-126, 0]
    return ax <= 0x39000000u ? 1.0f + x : res;
}

PK_DEV float pk_logf(float x) {
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
    const float lg1 = 0xaaaaaa.0p-24f, lg2 = 0xccce13.0p-25f, lg3 = 0x91e9ee.0p-25f, lg4 = 0xf89e26.0p-26f;
    unsigned ix = pk_bits(x);
    int k = 0;
    if (ix < 0x00800000u || (ix >> 31)) {
        if ((ix << 1) == 0) return -1.0f / (x * x);
        if (ix >> 31) return (x - x) / 0.0f;
        k -= 25;
        x *= 0x1p25f;
        ix = pk_bits(x);
    } else if (ix >= 0x7f800000u) {
        return x;
    } else if (ix == 0x3f800000u) {
        return 0.0f;
    }
    ix += 0x3f800000u - 0x3f3504f3u;
    k += (int)(ix >> 23) - 0x7f;
    ix = (ix & 0x007fffffu) + 0x3f3504f3u;
    x = pk_float(ix);
    const float f = x - 1.0f;
    const float s = f / (2.0f + f);
    const float z = s * s;
    const float w = z * z;
    const float t1 = w * (lg2 + w * lg4);
    const float t2 = z * (lg1 + w * lg3);
    const float r = t2 + t1;
    const float hfsq = 0.5f * f * f;
    const float dk = (float)k;
    return s * (hfsq + r) + dk * ln2_lo - hfsq + f + dk * ln2_hi;
}

PK_DEV float pk_expm1f(float x) {
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, inv_ln2 = 1.4426950216e+00f;
    const float q1 = -3.3333212137e-2f, q2 = 1.5807170421e-3f;
    const unsigned ux = pk_bits(x), ax = ux & 0x7fffffffu;
    const int neg = (int)(ux >> 31);
    float hi, lo, c = 0.0f, t;
    int k;
    if (ax >= 0x4195b844u) {
        if (ax > 0x7f800000u) return x;
        if (neg) return -1.0f;
        if (ax > 0x42b17217u) return x * 0x1p127f;
    }
    if (ax > 0x3eb17218u) {
        if (ax < 0x3f851592u) {
            if (!neg) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
            else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
        } else {
            k = (int)(inv_ln2 * x + (neg ? -0.5f : 0.5f));
            t = (float)k;
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (ax < 0x33000000u) {
        return x;
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x;
    const float hxs = x * hfx;
    const float r1 = 1.0f + hxs * (q1 + hxs * q2);
    t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = x * (e - c) - c;
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return 1.0f + 2.0f * (x - e);
    }
    const float twopk = pk_float((unsigned)(0x7f + k) << 23);
    float y;
    if (k < 0 || k > 56) {
        y = x - e + 1.0f;
        if (k == 128) y = y * 2.0f * 0x1p127f;
        else y = y * twopk;
        return y - 1.0f;
    }
    const float twomk = pk_float((unsigned)(0x7f - k) << 23);
    if (k < 23) y = (x - e + (1.0f - twomk)) * twopk;
    else y = (x - (e + twomk) + 1.0f) * twopk;
    return y;
}

PK_DEV float pk_tanhf(float x) {
    const unsigned ux = pk_bits(x);
    const int neg = (int)(ux >> 31);
    const unsigned w = ux & 0x7fffffffu;
    x = pk_float(w);
    float t;
    if (w > 0x3f0c9f54u) {
        if (w > 0x41200000u) t = 1.0f + 0.0f / x;
        else { t = pk_expm1f(2.0f * x); t = 1.0f - 2.0f / (t + 2.0f); }
    } else if (w > 0x3e82c578u) {
        t = pk_expm1f(2.0f * x);
        t = t / (t + 2.0f);
    } else if (w >= 0x00800000u) {
        t = pk_expm1f(-2.0f * x);
        t = -t / (t + 2.0f);
    } else {
        t = x;
    }
    return neg ? -t : t;
}

PK_DEV float pk_erf_mid(float x) {
    const float erx = 8.4506291151e-01f;
    const float a0 = -2.3621185683e-03f, a1 = 4.1485610604e-01f, a2 = -3.7220788002e-01f, a3 = 3.1834661961e-01f,
                a4 = -1.1089469492e-01f, a5 = 3.5478305072e-02f, a6 = -2.1663755178e-03f;
    const float b1 = 1.0642088205e-01f, b2 = 5.4039794207e-01f, b3 = 7.1828655899e-02f, b4 = 1.2617121637e-01f,
                b5 = 1.3637083583e-02f, b6 = 1.1984500103e-02f;
    const float s = __builtin_fabsf(x) - 1.0f;
    const float p = a0 + s * (a1 + s * (a2 + s * (a3 + s * (a4 + s * (a5 + s * a6)))));
    const float q = 1.0f + s * (b1 + s * (b2 + s * (b3 + s * (b4 + s * (b5 + s * b6)))));
    return 1.0f - erx - pk_erf_quot(p, q);
}

PK_DEV float pk_erfc_tail(unsigned ax, float x) {
    if (ax < 0x3fa00000u) return pk_erf_mid(x);
    x = __builtin_fabsf(x);
    // the quotients by the refined-reciprocal step (their operands lie in
    // the normal range here: x^2 in [1.56, 36], q >= 1, the product of the
    // exponentials above 2^-60), the first exponential's argument in
    // (-37, -2] (expf's fast path): erff's bits on every f32, pinned by its
    // all-f32 digest
    const float s = pk_erf_quot(1.0f, x * x);
    float r, q;
    if (ax < 0x4036db6du) {
        r = -9.8649440333e-03f + s * (-6.9385856390e-01f + s * (-1.0558626175e+01f + s * (-6.2375331879e+01f +
            s * (-1.6239666748e+02f + s * (-1.8460508728e+02f + s * (-8.1287437439e+01f + s * -9.8143291473e+00f))))));
        q = 1.0f + s * (1.9651271820e+01f + s * (1.3765776062e+02f + s * (4.3456588745e+02f + s * (6.4538726807e+02f +
            s * (4.2900814819e+02f + s * (1.0863500214e+02f + s * (6.5702495575e+00f + s * -6.0424413532e-02f)))))));
    } else {
        r = -9.8649431020e-03f + s * (-7.9928326607e-01f + s * (-1.7757955551e+01f + s * (-1.6063638306e+02f +
            s * (-6.3756646729e+02f + s * (-1.0250950928e+03f + s * -4.8351919556e+02f)))));
        q = 1.0f + s * (3.0338060379e+01f + s * (3.2579251099e+02f + s * (1.5367296143e+03f + s * (3.1998581543e+03f +
            s * (2.5530502930e+03f + s * (4.7452853394e+02f + s * -2.2440952301e+01f))))));
    }
    const float z = pk_float(pk_bits(x) & 0xffffe000u);
    return pk_erf_quot(pk_expf_le0(-z * z - 0.5625f) * pk_expf((z - x) * (z + x) + pk_erf_quot(r, q)), x);
}

PK_DEV float pk_erff(float x) {
    const float efx8 = 1.0270333290e+00f;
    unsigned ax = pk_bits(x);
    const int neg = (int)(ax >> 31);
    ax &= 0x7fffffffu;
    if (ax >= 0x7f800000u) return (float)(1 - 2 * neg) + 1.0f / x;
    if (ax < 0x3f580000u) {
        if (ax < 0x31800000u) return 0.125f * (8.0f * x + efx8 * x);
        const float z = x * x;
        const float r = 1.2837916613e-01f + z * (-3.2504209876e-01f + z * (-2.8481749818e-02f + z * (-5.7702702470e-03f + z * -2.3763017452e-05f)));
        const float s = 1.0f + z * (3.9791721106e-01f + z * (6.5022252500e-02f + z * (5.0813062117e-03f + z * (1.3249473704e-04f + z * -3.9602282413e-06f))));
        const float y = pk_erf_quot(r, s);
        return x + x * y;
    }
    float y;
    if (ax < 0x40c00000u) y = 1.0f - pk_erfc_tail(ax, x);
    else y = 1.0f - 0x1p-120f;
    return neg ? -y : y;
}

// ---- division by a constant ------------------------------------------------------
// a / c for f32 a and a finite nonzero f32 constant c, given rc = RN64(1/c):
// the f64 product a * rc rounded to f32.  It is the correctly rounded f32
// quotient for every a: the product is within 2^-52 of a/c relative (two
// f64 roundings); a quotient that is not a midpoint of the f32 grid
// (subnormal grid included) lies more than 2^-49 relative from every
// midpoint (a - m c is a nonzero multiple of the grid of a or of m c), so
// the product rounds to the same f32; a quotient that is a midpoint has at
// most 25 significant bits, so the product, within half an f64 ulp of it,
// is it exactly and rounds as it does.  Pinned on the device against the
// division over every f32 dividend for a set of divisors
// (presk_hip_scalar_digest fn 70-77).
PK_DEV float pk_div_rc(float a, double rc) { return (float)((double)a * rc); }

// ---- FAST mode's functions ------------------------------------------------------
// Not the interpreter's bits: FAST mode's exponential and error function, each
// within a bound stated against musl's (the functions above) and measured on
// the device over every f32 input (presk_hip_scalar_digest's ulp scans).

// e^x: x = k ln2 + r by Cody-Waite in two fmas (ln2's high part has 16
// significant bits, so k ln2_hi is exact for |k| < 2^8), |r| <= ln2 / 2;
// e^r = 2^(r log2 e) by the hardware's v_exp_f32 (an argument within 1/2,
// a normal result); then v_ldexp_f32 by k (one rounding where the result
// is subnormal, overflow to infinity and underflow to zero as it
// rounds).  The argument is clamped to [-104, 89] first (e^x rounds to 0
// below and overflows above), a NaN passed through.
PK_DEV float pk_expf_fast(float x) {
    const float xc = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 89.0f);
    const float k = __builtin_rintf(xc * 1.44269502e+0f);
    float r = __builtin_fmaf(-k, 6.93145751953125e-1f, xc);
    r = __builtin_fmaf(-k, 1.42860677e-6f, r);
    const float y = __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f(r * 1.44269502e+0f), (int)k);
    return x != x ? x + x : y;
}

// erf(x): x P(x^2) below |x| = 1 (P of degree 5, a relative minimax fit of
// erf(sqrt z)/sqrt z on [0, 1]), else 1 - 2^t, t = -u^2 log2 e + G2(u), with
// G2 of degree 8 in u - 2.5 (log2 e times a fit of log(erfc(u)) + u^2 on
// [1, 4]) and u = |x| clamped to 4, where 1 - erfc already rounds to 1; the
// sign restored.  Both polynomials by fma Horner steps; 2^t by v_exp_f32
// alone (t in [-24, -2.6], a normal result below 0.16, so its error moves
// 1 - 2^t by well under an ulp).  Both branches are evaluated and one
// chosen, so a wave runs no divergent paths; a NaN takes the first
// branch, which returns it quieted.
PK_DEV float pk_erff_fast(float x) {
    const float u = __builtin_fabsf(x);
    const float z = x * x;
    float p = __builtin_fmaf(z, -5.63141890e-4f, 4.91755083e-3f);
    p = __builtin_fmaf(z, p, -2.67113112e-2f);
    p = __builtin_fmaf(z, p, 1.12801798e-1f);
    p = __builtin_fmaf(z, p, -3.76123250e-1f);
    p = __builtin_fmaf(z, p, 1.12837911e+0f);
    const float small = x * p;
    const float uc = __builtin_fminf(u, 4.0f);
    const float s = uc - 2.5f;
    float g = __builtin_fmaf(s, 2.308051080e-06f, -1.919030910e-05f);
    g = __builtin_fmaf(s, g, 1.117438296e-04f);
    g = __builtin_fmaf(s, g, -6.061816821e-04f);
    g = __builtin_fmaf(s, g, 3.123552306e-03f);
    g = __builtin_fmaf(s, g, -1.566548645e-02f);
    g = __builtin_fmaf(s, g, 8.094441146e-02f);
    g = __builtin_fmaf(s, g, -5.088106990e-01f);
    g = __builtin_fmaf(s, g, -2.246009588e+00f);
    const float t = __builtin_fmaf(-(uc * 1.44269502e+0f), uc, g);
    const float large = __builtin_copysignf(1.0f - __builtin_amdgcn_exp2f(t), x);
    return u >= 1.0f ? large : small;
}

// ---- sinf / cosf: fdlibm's method in f64 (presk_libm.c:672-746 the
// kernels, 1372-1447 the reduction, 749-1189 its large-argument form,
// 2054-2111 sinf, 2213-2272 cosf) ---------------------------------------------
PK_DEV float pk_ksin(double x) {
    const double S1 = -0x15555554cbac77.0p-55, S2 = 0x111110896efbb2.0p-59, S3 = -0x1a00f9e2cae774.0p-65,
                 S4 = 0x16cd878c3b46a7.0p-71;
    const double z = x * x, w = z * z, r = S3 + z * S4, s = z * x;
    return (float)((x + s * (S1 + z * S2)) + s * w * r);
}
PK_DEV float pk_kcos(double x) {
    const double C0 = -0x1ffffffd0c5e81.0p-54, C1 = 0x155553e1053a42.0p-57, C2 = -0x16c087e80f1e27.0p-62,
                 C3 = 0x199342e0ee5069.0p-68;
    const double z = x * x, w = z * z, r = C2 + z * C3;
    return (float)(((1.0 + z * C0) + w * C1) + (w * z) * r);
}

// |x| past 2^28 pi/2: Payne-Hanek with the 24-bit digits of 2/pi, one piece
// of x (an integer of 24 bits times 2^e0), single precision (3 + 1 digits
// of the product kept, more taken when the fraction cancels)
static __device__ __noinline__ int pk_rem_pio2_big(double x0, int e0, double* y) {
    const int ipio2[] = {0xA2F983, 0x6E4E44, 0x1529FC, 0x2757D1, 0xF534DD, 0xC0DB62, 0x95993C, 0x439041,
                         0xFE5163, 0xABDEBB, 0xC561B7, 0x246E3A, 0x424DD2, 0xE00649, 0x2EEA09, 0xD1921C,
                         0xFE1DEB, 0x1CB129, 0xA73EE8, 0x8235F5, 0x2EBB44, 0x84E99C, 0x7026B4, 0x5F7E41,
                         0x3991D6, 0x398353, 0x39F49C, 0x845F8B, 0xBDF928, 0x3B1FF8};
    const double pio2_24[] = {1.57079625129699707031e+00, 7.54978941586159635335e-08, 5.39030252995776476554e-15,
                              3.28200341580791294123e-22};
    constexpr int JK = 3;
    int iq[20];
    double f[20], q[20], fq[20];
    for (int i = 0; i < 20; ++i) fq[i] = 0.0;
    int jv = (e0 - 3) / 24;
    if (jv < 0) jv = 0;
    int q0 = e0 - 24 * (jv + 1);
    for (int i = 0; i <= JK; ++i) {
        f[i] = (double)ipio2[jv + i];
        q[i] = 0.0 + x0 * f[i];
    }
    int jz = JK, n, ih;
    double z;
    for (;;) {
        z = q[jz];
        for (int i = 0, j = jz; j > 0; ++i, --j) {
            const double hi = (double)(int)(0x1p-24 * z);
            iq[i] = (int)(z - 0x1p24 * hi);
            z = q[j - 1] + hi;
        }
        z = __builtin_ldexp(z, q0);
        z -= 8.0 * __builtin_floor(z * 0.125);
        n = (int)z;
        z -= (double)n;
        ih = 0;
        if (q0 > 0) {
            const int top = iq[jz - 1] >> (24 - q0);
            n += top;
            iq[jz - 1] -= top << (24 - q0);
            ih = iq[jz - 1] >> (23 - q0);
        } else if (q0 == 0) {
            ih = iq[jz - 1] >> 23;
        } else if (z >= 0.5) {
            ih = 2;
        }
        if (ih > 0) {
            n += 1;
            int carry = 0;
            for (int i = 0; i < jz; ++i) {
                const int d = iq[i];
                if (carry == 0) {
                    if (d != 0) {
                        carry = 1;
                        iq[i] = 0x1000000 - d;
                    }
                } else {
                    iq[i] = 0xffffff - d;
                }
            }
            if (q0 == 1) iq[jz - 1] &= 0x7fffff;
            else if (q0 == 2) iq[jz - 1] &= 0x3fffff;
            if (ih == 2) {
                z = 1.0 - z;
                if (carry != 0) z -= __builtin_ldexp(1.0, q0);
            }
        }
        if (z == 0.0) {
            int any = 0;
            for (int i = jz - 1; i >= JK; --i) any |= iq[i];
            if (any == 0) {
                int k = 1;
                while (iq[JK - k] == 0) ++k;
                for (int i = jz + 1; i <= jz + k; ++i) {
                    f[i] = (double)ipio2[jv + i];
                    q[i] = 0.0 + x0 * f[i];
                }
                jz += k;
                continue;
            }
        }
        break;
    }
    if (z == 0.0) {
        jz -= 1;
        q0 -= 24;
        while (iq[jz] == 0) {
            --jz;
            q0 -= 24;
        }
    } else {
        z = __builtin_ldexp(z, -q0);
        if (z >= 0x1p24) {
            const double hi = (double)(int)(0x1p-24 * z);
            iq[jz] = (int)(z - 0x1p24 * hi);
            jz += 1;
            q0 += 24;
            iq[jz] = (int)hi;
        } else {
            iq[jz] = (int)z;
        }
    }
    double fw = __builtin_ldexp(1.0, q0);
    for (int i = jz; i >= 0; --i) {
        q[i] = fw * (double)iq[i];
        fw *= 0x1p-24;
    }
    for (int i = jz; i >= 0; --i) {
        fw = 0.0;
        for (int k = 0; k <= JK && k <= jz - i; ++k) fw += pio2_24[k] * q[i + k];
        fq[jz - i] = fw;
    }
    fw = 0.0;
    for (int i = jz; i >= 0; --i) fw += fq[i];
    *y = ih == 0 ? fw : -fw;
    return n;
}

// x mod pi/2 in *y, the quotient's low bits returned
PK_DEV int pk_rem_pio2f(float x, double* y) {
    const double toint = 1.5 / 0x1p-52, invpio2 = 6.36619772367581382433e-01, pio2_1 = 1.57079631090164184570e+00,
                 pio2_1t = 1.58932547735281966916e-08;
    const unsigned b = pk_bits(x), ix = b & 0x7fffffffu;
    if (ix < 0x4dc90fdbu) {
        const double fn = (double)x * invpio2 + toint - toint;
        *y = x - fn * pio2_1 - fn * pio2_1t;
        return (int)fn;
    }
    if (ix >= 0x7f800000u) {
        *y = x - x;
        return 0;
    }
    const int e0 = (int)(ix >> 23) - (0x7f + 23);
    double r;
    const int n = pk_rem_pio2_big((double)pk_float(ix - ((unsigned)e0 << 23)), e0, &r);
    *y = (b >> 31) ? -r : r;
    return (b >> 31) ? -n : n;
}

PK_DEV float pk_sinf(float x) {
    const double p1 = 1 * 1.57079632679489661923, p2 = 2 * 1.57079632679489661923, p3 = 3 * 1.57079632679489661923,
                 p4 = 4 * 1.57079632679489661923;
    const unsigned b = pk_bits(x), ix = b & 0x7fffffffu;
    const bool neg = (b >> 31) != 0;
    if (ix <= 0x3f490fdau) return ix < 0x39800000u ? x : pk_ksin(x);
    if (ix <= 0x407b53d1u) {
        if (ix <= 0x4016cbe3u) return neg ? -pk_kcos(x + p1) : pk_kcos(x - p1);
        return pk_ksin(neg ? -(x + p2) : -(x - p2));
    }
    if (ix <= 0x40e231d5u) {
        if (ix <= 0x40afeddfu) return neg ? pk_kcos(x + p3) : -pk_kcos(x - p3);
        return pk_ksin(neg ? x + p4 : x - p4);
    }
    if (ix >= 0x7f800000u) return x - x;
    double y;
    switch (pk_rem_pio2f(x, &y) & 3) {
        case 0: return pk_ksin(y);
        case 1: return pk_kcos(y);
        case 2: return pk_ksin(-y);
        default: return -pk_kcos(y);
    }
}

PK_DEV float pk_cosf(float x) {
    const double p1 = 1 * 1.57079632679489661923, p2 = 2 * 1.57079632679489661923, p3 = 3 * 1.57079632679489661923,
                 p4 = 4 * 1.57079632679489661923;
    const unsigned b = pk_bits(x), ix = b & 0x7fffffffu;
    const bool neg = (b >> 31) != 0;
    if (ix <= 0x3f490fdau) return ix < 0x39800000u ? 1.0f : pk_kcos(x);
    if (ix <= 0x407b53d1u) {
        if (ix > 0x4016cbe3u) return -pk_kcos(neg ? x + p2 : x - p2);
        return neg ? pk_ksin(x + p1) : pk_ksin(p1 - x);
    }
    if (ix <= 0x40e231d5u) {
        if (ix > 0x40afeddfu) return pk_kcos(neg ? x + p4 : x - p4);
        return neg ? pk_ksin(-x - p3) : pk_ksin(x - p3);
    }
    if (ix >= 0x7f800000u) return x - x;
    double y;
    switch ((unsigned)pk_rem_pio2f(x, &y) & 3) {
        case 0: return pk_kcos(y);
        case 1: return pk_ksin(-y);
        case 2: return -pk_kcos(y);
        default: return pk_ksin(y);
    }
}

// ---- f64: the interpreter's f64 arm (exec.rs:115-130), musl 1.1.22's double
// functions (presk_libm.c: exp :1520, log :1738, expm1 :323, tanh :1871, erf
// :2383-2541, sin :1999, cos :2159, k_sin/k_cos :575-690, rem_pio2 :1221,
// rem_pio2_large :876 at double precision) -----------------------------------
PK_DEV unsigned long long pk_bits64(double x) { return __builtin_bit_cast(unsigned long long, x); }
PK_DEV double pk_double(unsigned long long b) { return __builtin_bit_cast(double, b); }

// y * 2^n in at most two scalings before the final power of two (scalbn)
PK_DEV double pk_scalbn(double y, int n) {
    if (n > 1023) {
        y *= 0x1p1023;
        n -= 1023;
        if (n > 1023) {
            y *= 0x1p1023;
            n -= 1023;
            if (n > 1023) n = 1023;
        }
    } else if (n < -1022) {
        // the final scaling stays below -53: a subnormal result rounds once
        y *= 0x1p-1022 * 0x1p53;
        n += 1022 - 53;
        if (n < -1022) {
            y *= 0x1p-1022 * 0x1p53;
            n += 1022 - 53;
            if (n < -1022) n = -1022;
        }
    }
    return y * pk_double((unsigned long long)(0x3ff + n) << 52);
}

// x = k ln2 + r, exp(r) = 1 + r + r c(r) / (2 - c(r)), c the degree-5 remez
PK_DEV double pk_exp(double x) {
    const double LN2_HI = 6.93147180369123816490e-01, LN2_LO = 1.90821492927058770002e-10,
                 INV_LN2 = 1.44269504088896338700e+00;
    const double P1 = 1.66666666666666019037e-01, P2 = -2.77777777770155933842e-03, P3 = 6.61375632143793436117e-05,
                 P4 = -1.65339022054652515390e-06, P5 = 4.13813679705723846039e-08;
    const unsigned top = (unsigned)(pk_bits64(x) >> 32);
    const int neg = (int)(top >> 31);
    const unsigned ax = top & 0x7fffffffu;
    if (ax >= 0x4086232bu) {  // |x| >= 708.39 or NaN
        if (x != x) return x;
        if (x > 709.782712893383973096) return x * 0x1p1023;
        if (x < -708.39641853226410622 && x < -745.13321910194110842) return 0;
    }
    double hi, lo;
    int k;
    if (ax > 0x3fd62e42u) {
        if (ax >= 0x3ff0a2b2u)
            k = (int)(INV_LN2 * x + (neg ? -0.5 : 0.5));
        else
            k = 1 - neg - neg;
        hi = x - k * LN2_HI;
        lo = k * LN2_LO;
        x = hi - lo;
    } else if (ax > 0x3e300000u) {
        k = 0;
        hi = x;
        lo = 0;
    } else {
        return 1 + x;
    }
    const double xx = x * x;
    const double c = x - xx * (P1 + xx * (P2 + xx * (P3 + xx * (P4 + xx * P5))));
    const double y = 1 + (x * c / (2 - c) - lo + hi);
    return k == 0 ? y : pk_scalbn(y, k);
}

// x = 2^k (1 + f), log(1+f) = f - hfsq + s (hfsq + R(s^2)), s = f / (2 + f)
PK_DEV double pk_log(double x) {
    const double LN2_HI = 6.93147180369123816490e-01, LN2_LO = 1.90821492927058770002e-10;
    const double LG1 = 6.666666666666735130e-01, LG2 = 3.999999999940941908e-01, LG3 = 2.857142874366239149e-01,
                 LG4 = 2.222219843214978396e-01, LG5 = 1.818357216161805012e-01, LG6 = 1.531383769920937332e-01,
                 LG7 = 1.479819860511658591e-01;
    unsigned long long b = pk_bits64(x);
    unsigned top = (unsigned)(b >> 32);
    int k = 0;
    if (top < 0x00100000u || (top >> 31)) {
        if ((b << 1) == 0) return -1 / (x * x);
        if (top >> 31) return (x - x) / 0.0;
        k -= 54;
        x *= 0x1p54;
        b = pk_bits64(x);
        top = (unsigned)(b >> 32);
    } else if (top >= 0x7ff00000u) {
        return x;
    } else if (top == 0x3ff00000u && (b << 32) == 0) {
        return 0;
    }
    top += 0x3ff00000u - 0x3fe6a09eu;
    k += (int)(top >> 20) - 0x3ff;
    top = (top & 0x000fffffu) + 0x3fe6a09eu;
    x = pk_double((unsigned long long)top << 32 | (b & 0xffffffffull));
    const double f = x - 1.0, hfsq = 0.5 * f * f, s = f / (2.0 + f), z = s * s, w = z * z;
    const double t1 = w * (LG2 + w * (LG4 + w * LG6));
    const double t2 = z * (LG1 + w * (LG3 + w * (LG5 + w * LG7)));
    const double R = t2 + t1, dk = k;
    return s * (hfsq + R) + dk * LN2_LO - hfsq + f + dk * LN2_HI;
}

// e^x - 1: x = k ln2 + r with the reduction's rounding error carried
PK_DEV double pk_expm1(double x) {
    const double O_THRESHOLD = 7.09782712893383973096e+02, LN2_HI = 6.93147180369123816490e-01,
                 LN2_LO = 1.90821492927058770002e-10, INV_LN2 = 1.44269504088896338700e+00;
    const double Q1 = -3.33333333333331316428e-02, Q2 = 1.58730158725481460165e-03, Q3 = -7.93650757867487942473e-05,
                 Q4 = 4.00821782732936239552e-06, Q5 = -2.01099218183624371326e-07;
    const unsigned long long b = pk_bits64(x);
    const unsigned ax = (unsigned)(b >> 32) & 0x7fffffffu;
    const int neg = (int)(b >> 63);
    if (ax >= 0x4043687au) {
        if (x != x) return x;
        if (neg) return -1;
        if (x > O_THRESHOLD) return x * 0x1p1023;
    }
    double hi, lo, c = 0;
    int k;
    if (ax > 0x3fd62e42u) {
        if (ax < 0x3ff0a2b2u) {
            if (!neg) {
                hi = x - LN2_HI;
                lo = LN2_LO;
                k = 1;
            } else {
                hi = x + LN2_HI;
                lo = -LN2_LO;
                k = -1;
            }
        } else {
            k = (int)(INV_LN2 * x + (neg ? -0.5 : 0.5));
            const double t = k;
            hi = x - t * LN2_HI;
            lo = t * LN2_LO;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (ax < 0x3c900000u) {
        return x;
    } else {
        k = 0;
    }
    const double hfx = 0.5 * x, hxs = x * hfx;
    const double r1 = 1.0 + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    const double t = 3.0 - r1 * hfx;
    double e = hxs * ((r1 - t) / (6.0 - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = x * (e - c) - c;
    e -= hxs;
    if (k == -1) return 0.5 * (x - e) - 0.5;
    if (k == 1) {
        if (x < -0.25) return -2.0 * (e - (x + 0.5));
        return 1.0 + 2.0 * (x - e);
    }
    const double twopk = pk_double((unsigned long long)(0x3ff + k) << 52);
    if (k < 0 || k > 56) {
        double y = x - e + 1.0;
        y = k == 1024 ? y * 2.0 * 0x1p1023 : y * twopk;
        return y - 1.0;
    }
    const double twomk = pk_double((unsigned long long)(0x3ff - k) << 52);
    if (k < 20) return (x - e + (1 - twomk)) * twopk;
    return (x - (e + twomk) + 1) * twopk;
}

PK_DEV double pk_tanh(double x) {
    const unsigned long long b = pk_bits64(x);
    const int neg = (int)(b >> 63);
    x = pk_double(b & 0x7fffffffffffffffull);
    const unsigned w = (unsigned)(b >> 32) & 0x7fffffffu;
    double t;
    if (w > 0x3fe193eau) {
        if (w > 0x40340000u) {
            t = 1 - 0 / x;
        } else {
            t = pk_expm1(2 * x);
            t = 1 - 2 / (t + 2);
        }
    } else if (w > 0x3fd058aeu) {
        t = pk_expm1(2 * x);
        t = t / (t + 2);
    } else if (w >= 0x00100000u) {
        t = pk_expm1(-2 * x);
        t = -t / (t + 2);
    } else {
        t = x;
    }
    return neg ? -t : t;
}

// erfc on [0.84375, 1.25)
PK_DEV double pk_erfc_mid(double x) {
    const double ERX = 8.45062911510467529297e-01;
    const double PA0 = -2.36211856075265944077e-03, PA1 = 4.14856118683748331666e-01, PA2 = -3.72207876035701323847e-01,
                 PA3 = 3.18346619901161753674e-01, PA4 = -1.10894694282396677476e-01, PA5 = 3.54783043256182359371e-02,
                 PA6 = -2.16637559486879084300e-03;
    const double QA1 = 1.06420880400844228286e-01, QA2 = 5.40397917702171048937e-01, QA3 = 7.18286544141962662868e-02,
                 QA4 = 1.26171219808761642112e-01, QA5 = 1.36370839120290507362e-02, QA6 = 1.19844998467991074170e-02;
    const double s = __builtin_fabs(x) - 1;
    const double P = PA0 + s * (PA1 + s * (PA2 + s * (PA3 + s * (PA4 + s * (PA5 + s * PA6)))));
    const double Q = 1 + s * (QA1 + s * (QA2 + s * (QA3 + s * (QA4 + s * (QA5 + s * QA6)))));
    return 1 - ERX - P / Q;
}

// erfc on [0.84375, 6)
PK_DEV double pk_erfc_far(unsigned ix, double x) {
    const double RA0 = -9.86494403484714822705e-03, RA1 = -6.93858572707181764372e-01, RA2 = -1.05586262253232909814e+01,
                 RA3 = -6.23753324503260060396e+01, RA4 = -1.62396669462573470355e+02, RA5 = -1.84605092906711035994e+02,
                 RA6 = -8.12874355063065934246e+01, RA7 = -9.81432934416914548592e+00;
    const double SA1 = 1.96512716674392571292e+01, SA2 = 1.37657754143519042600e+02, SA3 = 4.34565877475229228821e+02,
                 SA4 = 6.45387271733267880336e+02, SA5 = 4.29008140027567833386e+02, SA6 = 1.08635005541779435134e+02,
                 SA7 = 6.57024977031928170135e+00, SA8 = -6.04244152148580987438e-02;
    const double RB0 = -9.86494292470009928597e-03, RB1 = -7.99283237680523006574e-01, RB2 = -1.77579549177547519889e+01,
                 RB3 = -1.60636384855821916062e+02, RB4 = -6.37566443368389627722e+02, RB5 = -1.02509513161107724954e+03,
                 RB6 = -4.83519191608651397019e+02;
    const double SB1 = 3.03380607434824582924e+01, SB2 = 3.25792512996573918826e+02, SB3 = 1.53672958608443695994e+03,
                 SB4 = 3.19985821950859553908e+03, SB5 = 2.55305040643316442583e+03, SB6 = 4.74528541206955367215e+02,
                 SB7 = -2.24409524465858183362e+01;
    if (ix < 0x3ff40000u) return pk_erfc_mid(x);
    x = __builtin_fabs(x);
    const double s = 1 / (x * x);
    double R, S;
    if (ix < 0x4006db6du) {
        R = RA0 + s * (RA1 + s * (RA2 + s * (RA3 + s * (RA4 + s * (RA5 + s * (RA6 + s * RA7))))));
        S = 1.0 + s * (SA1 + s * (SA2 + s * (SA3 + s * (SA4 + s * (SA5 + s * (SA6 + s * (SA7 + s * SA8)))))));
    } else {
        R = RB0 + s * (RB1 + s * (RB2 + s * (RB3 + s * (RB4 + s * (RB5 + s * RB6)))));
        S = 1.0 + s * (SB1 + s * (SB2 + s * (SB3 + s * (SB4 + s * (SB5 + s * (SB6 + s * SB7))))));
    }
    const double z = pk_double(pk_bits64(x) & 0xffffffff00000000ull);
    return pk_exp(-z * z - 0.5625) * pk_exp((z - x) * (z + x) + R / S) / x;
}

PK_DEV double pk_erf(double x) {
    const double EFX8 = 1.02703333676410069053e+00;
    const double PP0 = 1.28379167095512558561e-01, PP1 = -3.25042107247001499370e-01, PP2 = -2.84817495755985104766e-02,
                 PP3 = -5.77027029648944159157e-03, PP4 = -2.37630166566501626084e-05;
    const double QQ1 = 3.97917223959155352819e-01, QQ2 = 6.50222499887672944485e-02, QQ3 = 5.08130628187576562776e-03,
                 QQ4 = 1.32494738004321644526e-04, QQ5 = -3.96022827877536812320e-06;
    const unsigned top = (unsigned)(pk_bits64(x) >> 32);
    const int neg = (int)(top >> 31);
    const unsigned ix = top & 0x7fffffffu;
    if (ix >= 0x7ff00000u) return 1 - 2 * neg + 1 / x;
    if (ix < 0x3feb0000u) {
        if (ix < 0x3e300000u) return 0.125 * (8 * x + EFX8 * x);
        const double z = x * x;
        const double r = PP0 + z * (PP1 + z * (PP2 + z * (PP3 + z * PP4)));
        const double s = 1.0 + z * (QQ1 + z * (QQ2 + z * (QQ3 + z * (QQ4 + z * QQ5))));
        return x + x * (r / s);
    }
    const double y = ix < 0x40180000u ? 1 - pk_erfc_far(ix, x) : 1 - 0x1p-1022;
    return neg ? -y : y;
}

// sin and cos of x + y on [-pi/4, pi/4] (iy = 0: y is zero)
PK_DEV double pk_ksin64(double x, double y, int iy) {
    const double S1 = -1.66666666666666324348e-01, S2 = 8.33333333332248946124e-03, S3 = -1.98412698298579493134e-04,
                 S4 = 2.75573137070700676789e-06, S5 = -2.50507602534068634195e-08, S6 = 1.58969099521155010221e-10;
    const double z = x * x, w = z * z;
    const double r = S2 + z * (S3 + z * S4) + z * w * (S5 + z * S6);
    const double v = z * x;
    if (iy == 0) return x + v * (S1 + z * r);
    return x - ((z * (0.5 * y - v * r) - y) - v * S1);
}
PK_DEV double pk_kcos64(double x, double y) {
    const double C1 = 4.16666666666666019037e-02, C2 = -1.38888888888741095749e-03, C3 = 2.48015872894767294178e-05,
                 C4 = -2.75573143513906633035e-07, C5 = 2.08757232129817482790e-09, C6 = -1.13596475577881948265e-11;
    const double z = x * x;
    double w = z * z;
    const double r = z * (C1 + z * (C2 + z * C3)) + w * w * (C4 + z * (C5 + z * C6));
    const double hz = 0.5 * z;
    w = 1.0 - hz;
    return w + (((1.0 - w) - hz) + (z * r - x * y));
}

// x (nx pieces of 24 bits, x[0] times 2^e0 the leading one) mod pi/2 as
// y[0] + y[1]: Payne-Hanek with the 24-bit digits of 2/pi at double
// precision (jk = 4 digits of the product kept, more when the fraction
// cancels); returns the quotient's low 3 bits
static __device__ __noinline__ int pk_rem_pio2_large(const double* x, double* y, int e0, int nx) {
    const int ipio2[] = {0xA2F983, 0x6E4E44, 0x1529FC, 0x2757D1, 0xF534DD, 0xC0DB62, 0x95993C, 0x439041, 0xFE5163,
                         0xABDEBB, 0xC561B7, 0x246E3A, 0x424DD2, 0xE00649, 0x2EEA09, 0xD1921C, 0xFE1DEB, 0x1CB129,
                         0xA73EE8, 0x8235F5, 0x2EBB44, 0x84E99C, 0x7026B4, 0x5F7E41, 0x3991D6, 0x398353, 0x39F49C,
                         0x845F8B, 0xBDF928, 0x3B1FF8, 0x97FFDE, 0x05980F, 0xEF2F11, 0x8B5A0A, 0x6D1F6D, 0x367ECF,
                         0x27CB09, 0xB74F46, 0x3F669E, 0x5FEA2D, 0x7527BA, 0xC7EBE5, 0xF17B3D, 0x0739F7, 0x8A5292,
                         0xEA6BFB, 0x5FB11F, 0x8D5D08, 0x560330, 0x46FC7B, 0x6BABF0, 0xCFBC20, 0x9AF436, 0x1DA9E3,
                         0x91615E, 0xE61B08, 0x659985, 0x5F14A0, 0x68408D, 0xFFD880, 0x4D7327, 0x310606, 0x1556CA,
                         0x73A8C9, 0x60E27B, 0xC08C6B};
    const double pio2_24[] = {1.57079625129699707031e+00, 7.54978941586159635335e-08, 5.39030252995776476554e-15,
                              3.28200341580791294123e-22, 1.27065575308067607349e-29};
    constexpr int JK = 4;
    int iq[20];
    double f[20], q[20], fq[20];
    for (int i = 0; i < 20; ++i) fq[i] = 0.0;
    const int jx = nx - 1;
    int jv = (e0 - 3) / 24;
    if (jv < 0) jv = 0;
    int q0 = e0 - 24 * (jv + 1);
    for (int i = 0, j = jv - jx; i <= jx + JK; ++i, ++j) f[i] = j < 0 ? 0.0 : (double)ipio2[j];
    for (int i = 0; i <= JK; ++i) {
        double fw = 0.0;
        for (int j = 0; j <= jx; ++j) fw += x[j] * f[jx + i - j];
        q[i] = fw;
    }
    int jz = JK, n, ih;
    double z;
    for (;;) {
        z = q[jz];
        for (int i = 0, j = jz; j > 0; ++i, --j) {
            const double hi = (double)(int)(0x1p-24 * z);
            iq[i] = (int)(z - 0x1p24 * hi);
            z = q[j - 1] + hi;
        }
        z = pk_scalbn(z, q0);
        z -= 8.0 * __builtin_floor(z * 0.125);
        n = (int)z;
        z -= (double)n;
        ih = 0;
        if (q0 > 0) {
            const int top = iq[jz - 1] >> (24 - q0);
            n += top;
            iq[jz - 1] -= top << (24 - q0);
            ih = iq[jz - 1] >> (23 - q0);
        } else if (q0 == 0) {
            ih = iq[jz - 1] >> 23;
        } else if (z >= 0.5) {
            ih = 2;
        }
        if (ih > 0) {
            n += 1;
            int carry = 0;
            for (int i = 0; i < jz; ++i) {
                const int d = iq[i];
                if (carry == 0) {
                    if (d != 0) {
                        carry = 1;
                        iq[i] = 0x1000000 - d;
                    }
                } else {
                    iq[i] = 0xffffff - d;
                }
            }
            if (q0 == 1)
                iq[jz - 1] &= 0x7fffff;
            else if (q0 == 2)
                iq[jz - 1] &= 0x3fffff;
            if (ih == 2) {
                z = 1.0 - z;
                if (carry != 0) z -= pk_scalbn(1.0, q0);
            }
        }
        if (z == 0.0) {
            int any = 0;
            for (int i = jz - 1; i >= JK; --i) any |= iq[i];
            if (any == 0) {
                int k = 1;
                while (iq[JK - k] == 0) ++k;
                for (int i = jz + 1; i <= jz + k; ++i) {
                    f[jx + i] = (double)ipio2[jv + i];
                    double fw = 0.0;
                    for (int j = 0; j <= jx; ++j) fw += x[j] * f[jx + i - j];
                    q[i] = fw;
                }
                jz += k;
                continue;
            }
        }
        break;
    }
    if (z == 0.0) {
        jz -= 1;
        q0 -= 24;
        while (iq[jz] == 0) {
            --jz;
            q0 -= 24;
        }
    } else {
        z = pk_scalbn(z, -q0);
        if (z >= 0x1p24) {
            const double hi = (double)(int)(0x1p-24 * z);
            iq[jz] = (int)(z - 0x1p24 * hi);
            jz += 1;
            q0 += 24;
            iq[jz] = (int)hi;
        } else {
            iq[jz] = (int)z;
        }
    }
    double fw = pk_scalbn(1.0, q0);
    for (int i = jz; i >= 0; --i) {
        q[i] = fw * (double)iq[i];
        fw *= 0x1p-24;
    }
    for (int i = jz; i >= 0; --i) {
        fw = 0.0;
        for (int k = 0; k <= JK && k <= jz - i; ++k) fw += pio2_24[k] * q[i + k];
        fq[jz - i] = fw;
    }
    fw = 0.0;
    for (int i = jz; i >= 0; --i) fw += fq[i];
    y[0] = ih == 0 ? fw : -fw;
    fw = fq[0] - fw;
    for (int i = 1; i <= jz; ++i) fw += fq[i];
    y[1] = ih == 0 ? fw : -fw;
    return n & 7;
}

// x mod pi/2 as y[0] + y[1] (the caller handles |x| <= pi/4)
PK_DEV int pk_rem_pio2(double x, double* y) {
    const double TOINT = 1.5 / 0x1p-52, INVPIO2 = 6.36619772367581382433e-01, PIO2_1 = 1.57079632673412561417e+00,
                 PIO2_1T = 6.07710050650619224932e-11, PIO2_2 = 6.07710050630396597660e-11,
                 PIO2_2T = 2.02226624879595063154e-21, PIO2_3 = 2.02226624871116645580e-21,
                 PIO2_3T = 8.47842766036889956997e-32;
    const unsigned long long b = pk_bits64(x);
    const int neg = (int)(b >> 63);
    const unsigned ix = (unsigned)(b >> 32) & 0x7fffffffu;
    int near = 0;
    if (ix <= 0x400f6a7au) {
        if ((ix & 0xfffffu) != 0x921fbu) near = ix <= 0x4002d97cu ? 1 : 2;
    } else if (ix <= 0x401c463bu) {
        if (ix <= 0x4015fdbcu) {
            if (ix != 0x4012d97cu) near = 3;
        } else if (ix != 0x401921fbu) {
            near = 4;
        }
    }
    if (near) {
        const double m = near;
        if (!neg) {
            const double z = x - m * PIO2_1;
            y[0] = z - m * PIO2_1T;
            y[1] = (z - y[0]) - m * PIO2_1T;
            return near;
        }
        const double z = x + m * PIO2_1;
        y[0] = z + m * PIO2_1T;
        y[1] = (z - y[0]) + m * PIO2_1T;
        return -near;
    }
    if (ix < 0x413921fbu) {
        const double fn = x * INVPIO2 + TOINT - TOINT;
        const int n = (int)fn;
        double r = x - fn * PIO2_1;
        double w = fn * PIO2_1T;
        y[0] = r - w;
        const int ex = (int)(ix >> 20);
        int ey = (int)(pk_bits64(y[0]) >> 52 & 0x7ff);
        if (ex - ey > 16) {
            double t = r;
            w = fn * PIO2_2;
            r = t - w;
            w = fn * PIO2_2T - ((t - r) - w);
            y[0] = r - w;
            ey = (int)(pk_bits64(y[0]) >> 52 & 0x7ff);
            if (ex - ey > 49) {
                t = r;
                w = fn * PIO2_3;
                r = t - w;
                w = fn * PIO2_3T - ((t - r) - w);
                y[0] = r - w;
            }
        }
        y[1] = (r - y[0]) - w;
        return n;
    }
    if (ix >= 0x7ff00000u) {
        y[0] = y[1] = x - x;
        return 0;
    }
    double z = pk_double((b & (~0ull >> 12)) | ((unsigned long long)(0x3ff + 23) << 52));
    double tx[3], ty[2];
    int i;
    for (i = 0; i < 2; ++i) {
        tx[i] = (double)(int)z;
        z = (z - tx[i]) * 0x1p24;
    }
    tx[i] = z;
    while (tx[i] == 0.0) --i;
    const int n = pk_rem_pio2_large(tx, ty, (int)(ix >> 20) - (0x3ff + 23), i + 1);
    if (neg) {
        y[0] = -ty[0];
        y[1] = -ty[1];
        return -n;
    }
    y[0] = ty[0];
    y[1] = ty[1];
    return n;
}

PK_DEV double pk_sin(double x) {
    const unsigned ix = (unsigned)(pk_bits64(x) >> 32) & 0x7fffffffu;
    if (ix <= 0x3fe921fbu) return ix < 0x3e500000u ? x : pk_ksin64(x, 0.0, 0);
    if (ix >= 0x7ff00000u) return x - x;
    double y[2];
    switch ((unsigned)pk_rem_pio2(x, y) & 3) {
        case 0: return pk_ksin64(y[0], y[1], 1);
        case 1: return pk_kcos64(y[0], y[1]);
        case 2: return -pk_ksin64(y[0], y[1], 1);
        default: return -pk_kcos64(y[0], y[1]);
    }
}

PK_DEV double pk_cos(double x) {
    const unsigned ix = (unsigned)(pk_bits64(x) >> 32) & 0x7fffffffu;
    if (ix <= 0x3fe921fbu) return ix < 0x3e46a09eu ? 1.0 : pk_kcos64(x, 0);
    if (ix >= 0x7ff00000u) return x - x;
    double y[2];
    switch ((unsigned)pk_rem_pio2(x, y) & 3) {
        case 0: return pk_kcos64(y[0], y[1]);
        case 1: return -pk_ksin64(y[0], y[1], 1);
        case 2: return -pk_kcos64(y[0], y[1]);
        default: return pk_ksin64(y[0], y[1], 1);
    }
}
