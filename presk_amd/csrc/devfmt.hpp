// Device-side storage conversions and f32 transcendentals (gfx950).
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
// Each is checked over every f32 input on the GPU against the reference's
// compiled C (tests/test_gpu_scalar.py, digests in tests/golden/digests.json).
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
// (written as a select, not a branch: in a running sum it is one step of a
// dependent chain, where a branch costs an exec-mask round trip)
PK_DEV unsigned short pk_f32_to_bf16(float x) {
    const unsigned b = pk_bits(x);
    const unsigned nan = (b >> 16) | 0x0040u, rne = (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
    return (unsigned short)((b & 0x7fffffffu) > 0x7f800000u ? nan : rne);
}

// ---- binary16 -----------------------------------------------------------------
PK_DEV float pk_f16_to_f32(unsigned short c) {
    const unsigned sign = (unsigned)(c & 0x8000u) << 16, field = (c >> 10) & 0x1fu, frac = c & 0x3ffu;
    const unsigned special = frac == 0 ? 0x7f800000u : (0x7fc00000u | (frac << 13));
    const unsigned sub = pk_bits((float)frac * 5.9604644775390625e-8f);   // frac * 2^-24, exact
    const unsigned normal = ((field + 112u) << 23) | (frac << 13);
    return pk_float(sign | (field == 0x1fu ? special : field == 0 ? sub : normal));
}
PK_DEV unsigned short pk_f32_to_f16(float x) {
    const unsigned b = pk_bits(x), sign = (b >> 16) & 0x8000u, a = b & 0x7fffffffu;
    const unsigned nan = 0x7e00u | ((a >> 13) & 0x1ffu);                  // NaN, quiet
    const unsigned r = a - 0x38000000u;                                   // normal binary16: rebias 127 -> 15
    const unsigned normal = (r + 0xfffu + ((r >> 13) & 1u)) >> 13;
    // subnormal or zero: |x| / 2^-24 rounded to even (computed on 0 otherwise)
    const unsigned sub = (unsigned)__builtin_rintf(pk_float(a < 0x38800000u ? a : 0u) * 16777216.0f);
    const unsigned code = a > 0x7f800000u ? nan : a >= 0x477ff000u ? 0x7c00u : a >= 0x38800000u ? normal : sub;
    return (unsigned short)(sign | code);
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

// fdlibm's expf, its branches written as selects (the same operations on
// every path, so the same bits): k = 0 is the general reduction with k = 0
// (x - 0 * ln2_hi is x, 0 * ln2_lo is 0), scalbnf's one pre-scaling step is
// a select of the factor, and the special inputs are chosen last.
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
    const float y = 1.0f + (r * c / (2.0f - c) - lo + hi);
    // y * 2^k as scalbnf computes it (k lies in [-150, 150])
    const bool up = k > 127, down = k < -126;
    const float s = up ? 0x1p127f : down ? 0x1p-102f : 1.0f;
    const int kk = up ? k - 127 : down ? k + 102 : k;
    const float scaled = (y * s) * pk_float((unsigned)(0x7f + kk) << 23);
    float res = k == 0 ? y : scaled;
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
    const float y = 1.0f + (r * c / (2.0f - c) - lo + hi);
    const float res = k == 0 ? y : y * pk_float((unsigned)(0x7f + k) << 23);
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
    return 1.0f - erx - p / q;
}

PK_DEV float pk_erfc_tail(unsigned ax, float x) {
    if (ax < 0x3fa00000u) return pk_erf_mid(x);
    x = __builtin_fabsf(x);
    const float s = 1.0f / (x * x);
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
    return pk_expf(-z * z - 0.5625f) * pk_expf((z - x) * (z + x) + r / q) / x;
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
        const float y = r / s;
        return x + x * y;
    }
    float y;
    if (ax < 0x40c00000u) y = 1.0f - pk_erfc_tail(ax, x);
    else y = 1.0f - 0x1p-120f;
    return neg ? -y : y;
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
