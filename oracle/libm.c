/* oracle/libm.c -- TEST INFRASTRUCTURE ONLY (the parity oracle).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * link or run this file.  The product carries its own device restatement.
 *
 * The f32 transcendentals the kernel interpreter calls (exec.rs:158-170: the
 * `libm` crate 0.2.16, which is musl 1.1.22's fdlibm-derived code, the C form
 * of which the reference ships as crates/presk-export-c/c/presk_libm.c).
 * Restated here from the published fdlibm/FreeBSD-msun method: the same
 * reductions, the same minimax coefficients (these are the algorithm's
 * constants and must be equal for equal bits) and the same order of f32
 * operations.  Build with -ffp-contract=off and without -ffast-math.
 *
 *   ok_expf   follows presk_libm.c:1605-1737 (e_expf)
 *   ok_logf   follows presk_libm.c:1811-1870 (e_logf)
 *   ok_expm1f follows presk_libm.c:436-574   (s_expm1f)
 *   ok_tanhf  follows presk_libm.c:1915-1998 (s_tanhf)
 *   ok_erff   follows presk_libm.c:2542-2680 (s_erff)
 *
 * Pinned by tests/test_oracle_scalar.py: every f32 input, digest against the
 * reference's C compiled into oracle/_ref.
 *
 * Notices.  The method, constants and operation order restated here are
 * those of the following sources, whose terms ask that these notices be
 * kept with any work derived from them:
 *
 *   musl libc 1.1.22 -- Copyright (c) 2005-2014 Rich Felker, et al.
 *   Permission is hereby granted, free of charge, to any person obtaining
 *   a copy of this software and associated documentation files (the
 *   "Software"), to deal in the Software without restriction, including
 *   without limitation the rights to use, copy, modify, merge, publish,
 *   distribute, sublicense, and/or sell copies of the Software, and to
 *   permit persons to whom the Software is furnished to do so, subject to
 *   the following conditions: The above copyright notice and this
 *   permission notice shall be included in all copies or substantial
 *   portions of the Software.  THE SOFTWARE IS PROVIDED "AS IS", WITHOUT
 *   WARRANTY OF ANY KIND, EXPRESS OR IMPLIED.
 *
 *   fdlibm (via FreeBSD msun) -- Copyright (C) 1993 by Sun Microsystems,
 *   Inc. All rights reserved.  Developed at SunPro, a Sun Microsystems,
 *   Inc. business.  Permission to use, copy, modify, and distribute this
 *   software is freely granted, provided that this notice is preserved.
 *   (The f32 conversions of these functions are by Ian Lance Taylor,
 *   Cygnus Support, and Bruce D. Evans, under the same terms.)
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

static inline uint32_t lm_bits(float x) { uint32_t b; memcpy(&b, &x, 4); return b; }
static inline float lm_from(uint32_t b) { float x; memcpy(&x, &b, 4); return x; }

/* y * 2^n for the range of n the callers need, in at most two scalings
 * before the final power of two, as fdlibm's scalbnf does. */
static float lm_ldexpf(float y, int n)
{
    if (n > 127) {
        y *= 0x1p127f;
        n -= 127;
        if (n > 127) {
            y *= 0x1p127f;
            n -= 127;
            if (n > 127)
                n = 127;
        }
    } else if (n < -126) {
        y *= 0x1p-126f * 0x1p24f;
        n += 126 - 24;
        if (n < -126) {
            y *= 0x1p-126f * 0x1p24f;
            n += 126 - 24;
            if (n < -126)
                n = -126;
        }
    }
    return y * lm_from((uint32_t)(0x7f + n) << 23);
}

float ok_expf(float x)
{
    /* ln2 split so that k*LN2_HI is exact; degree-2 rational remez of
     * x*(e^x+1)/(e^x-1) on [-0.34568, 0.34568]. */
    const float LN2_HI = 6.9314575195e-1f, LN2_LO = 1.4286067653e-6f, INV_LN2 = 1.4426950216e+0f;
    const float P1 = 1.6666625440e-1f, P2 = -2.7667332906e-3f;
    uint32_t ax = lm_bits(x);
    const int neg = (int)(ax >> 31);
    ax &= 0x7fffffffu;

    if (ax >= 0x42aeac50u) {                 /* |x| >= 87.33655 or NaN */
        if (ax > 0x7f800000u)
            return x;                         /* NaN */
        if (ax >= 0x42b17218u && !neg)
            return x * 0x1p127f;              /* overflow to +inf */
        if (neg && ax >= 0x42cff1b5u)
            return 0;                         /* underflow to +0 */
    }
    float hi, lo;
    int k;
    if (ax > 0x3eb17218u) {                  /* |x| > ln2/2 */
        if (ax > 0x3f851592u)                /* |x| > 1.5 ln2 */
            k = (int)(INV_LN2 * x + (neg ? -0.5f : 0.5f));
        else
            k = 1 - neg - neg;
        hi = x - (float)k * LN2_HI;
        lo = (float)k * LN2_LO;
        x = hi - lo;
    } else if (ax > 0x39000000u) {           /* |x| > 2^-14 */
        k = 0;
        hi = x;
        lo = 0;
    } else {
        return 1 + x;
    }
    const float xx = x * x;
    const float c = x - xx * (P1 + xx * P2);
    const float y = 1 + (x * c / (2 - c) - lo + hi);
    return k == 0 ? y : lm_ldexpf(y, k);
}

float ok_logf(float x)
{
    const float LN2_HI = 6.9313812256e-01f, LN2_LO = 9.0580006145e-06f;
    const float LG1 = 0xaaaaaa.0p-24f, LG2 = 0xccce13.0p-25f, LG3 = 0x91e9ee.0p-25f, LG4 = 0xf89e26.0p-26f;
    uint32_t ix = lm_bits(x);
    int k = 0;
    if (ix < 0x00800000u || (ix >> 31)) {    /* subnormal, zero or negative */
        if ((ix << 1) == 0)
            return -1 / (x * x);              /* log(+-0) = -inf */
        if (ix >> 31)
            return (x - x) / 0.0f;            /* log(<0) = NaN */
        k -= 25;                              /* scale a subnormal up */
        x *= 0x1p25f;
        ix = lm_bits(x);
    } else if (ix >= 0x7f800000u) {
        return x;                             /* +inf or NaN */
    } else if (ix == 0x3f800000u) {
        return 0;
    }
    /* x = 2^k * m with m in [sqrt(2)/2, sqrt(2)) */
    ix += 0x3f800000u - 0x3f3504f3u;
    k += (int)(ix >> 23) - 0x7f;
    ix = (ix & 0x007fffffu) + 0x3f3504f3u;
    x = lm_from(ix);

    const float f = x - 1.0f;
    const float s = f / (2.0f + f);
    const float z = s * s;
    const float w = z * z;
    const float t1 = w * (LG2 + w * LG4);
    const float t2 = z * (LG1 + w * LG3);
    const float r = t2 + t1;
    const float hfsq = 0.5f * f * f;
    const float dk = (float)k;
    return s * (hfsq + r) + dk * LN2_LO - hfsq + f + dk * LN2_HI;
}

float ok_expm1f(float x)
{
    const float LN2_HI = 6.9313812256e-01f, LN2_LO = 9.0580006145e-06f, INV_LN2 = 1.4426950216e+00f;
    const float Q1 = -3.3333212137e-2f, Q2 = 1.5807170421e-3f;
    const uint32_t ux = lm_bits(x);
    const uint32_t ax = ux & 0x7fffffffu;
    const int neg = (int)(ux >> 31);
    float hi, lo, c = 0, t;
    int k;

    if (ax >= 0x4195b844u) {                 /* |x| >= 27 ln2 */
        if (ax > 0x7f800000u)
            return x;
        if (neg)
            return -1;
        if (ax > 0x42b17217u)
            return x * 0x1p127f;
    }
    if (ax > 0x3eb17218u) {                  /* |x| > ln2/2 */
        if (ax < 0x3F851592u) {              /* and < 1.5 ln2 */
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
            k = (int)(INV_LN2 * x + (neg ? -0.5f : 0.5f));
            t = (float)k;
            hi = x - t * LN2_HI;
            lo = t * LN2_LO;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (ax < 0x33000000u) {           /* |x| < 2^-25 */
        return x;
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x;
    const float hxs = x * hfx;
    const float r1 = 1.0f + hxs * (Q1 + hxs * Q2);
    t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0)
        return x - (x * e - hxs);
    e = x * (e - c) - c;
    e -= hxs;
    if (k == -1)
        return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f)
            return -2.0f * (e - (x + 0.5f));
        return 1.0f + 2.0f * (x - e);
    }
    const float twopk = lm_from((uint32_t)(0x7f + k) << 23);
    float y;
    if (k < 0 || k > 56) {
        y = x - e + 1.0f;
        if (k == 128)
            y = y * 2.0f * 0x1p127f;
        else
            y = y * twopk;
        return y - 1.0f;
    }
    const float twomk = lm_from((uint32_t)(0x7f - k) << 23);
    if (k < 23)
        y = (x - e + (1 - twomk)) * twopk;
    else
        y = (x - (e + twomk) + 1) * twopk;
    return y;
}

float ok_tanhf(float x)
{
    const uint32_t ux = lm_bits(x);
    const int neg = (int)(ux >> 31);
    const uint32_t w = ux & 0x7fffffffu;
    x = lm_from(w);
    float t;
    if (w > 0x3f0c9f54u) {                   /* |x| > log(3)/2 or NaN */
        if (w > 0x41200000u) {               /* |x| > 10 */
            t = 1 + 0 / x;
        } else {
            t = ok_expm1f(2 * x);
            t = 1 - 2 / (t + 2);
        }
    } else if (w > 0x3e82c578u) {            /* |x| > log(5/3)/2 */
        t = ok_expm1f(2 * x);
        t = t / (t + 2);
    } else if (w >= 0x00800000u) {
        t = ok_expm1f(-2 * x);
        t = -t / (t + 2);
    } else {
        t = x;                                /* subnormal */
    }
    return neg ? -t : t;
}

/* erf on [0.84375, 1.25): 1 - erx - P(s)/Q(s), s = |x| - 1 */
static float lm_erf_mid(float x)
{
    const float ERX = 8.4506291151e-01f;
    const float A0 = -2.3621185683e-03f, A1 = 4.1485610604e-01f, A2 = -3.7220788002e-01f,
                A3 = 3.1834661961e-01f, A4 = -1.1089469492e-01f, A5 = 3.5478305072e-02f,
                A6 = -2.1663755178e-03f;
    const float B1 = 1.0642088205e-01f, B2 = 5.4039794207e-01f, B3 = 7.1828655899e-02f,
                B4 = 1.2617121637e-01f, B5 = 1.3637083583e-02f, B6 = 1.1984500103e-02f;
    const float s = fabsf(x) - 1;
    const float p = A0 + s * (A1 + s * (A2 + s * (A3 + s * (A4 + s * (A5 + s * A6)))));
    const float q = 1 + s * (B1 + s * (B2 + s * (B3 + s * (B4 + s * (B5 + s * B6)))));
    return 1 - ERX - p / q;
}

/* erfc for |x| in [0.84375, 6) */
static float lm_erfc_tail(uint32_t ax, float x)
{
    const float RA0 = -9.8649440333e-03f, RA1 = -6.9385856390e-01f, RA2 = -1.0558626175e+01f,
                RA3 = -6.2375331879e+01f, RA4 = -1.6239666748e+02f, RA5 = -1.8460508728e+02f,
                RA6 = -8.1287437439e+01f, RA7 = -9.8143291473e+00f;
    const float SA1 = 1.9651271820e+01f, SA2 = 1.3765776062e+02f, SA3 = 4.3456588745e+02f,
                SA4 = 6.4538726807e+02f, SA5 = 4.2900814819e+02f, SA6 = 1.0863500214e+02f,
                SA7 = 6.5702495575e+00f, SA8 = -6.0424413532e-02f;
    const float RB0 = -9.8649431020e-03f, RB1 = -7.9928326607e-01f, RB2 = -1.7757955551e+01f,
                RB3 = -1.6063638306e+02f, RB4 = -6.3756646729e+02f, RB5 = -1.0250950928e+03f,
                RB6 = -4.8351919556e+02f;
    const float SB1 = 3.0338060379e+01f, SB2 = 3.2579251099e+02f, SB3 = 1.5367296143e+03f,
                SB4 = 3.1998581543e+03f, SB5 = 2.5530502930e+03f, SB6 = 4.7452853394e+02f,
                SB7 = -2.2440952301e+01f;
    if (ax < 0x3fa00000u)                     /* |x| < 1.25 */
        return lm_erf_mid(x);
    x = fabsf(x);
    const float s = 1 / (x * x);
    float r, q;
    if (ax < 0x4036db6du) {                  /* |x| < 1/0.35 */
        r = RA0 + s * (RA1 + s * (RA2 + s * (RA3 + s * (RA4 + s * (RA5 + s * (RA6 + s * RA7))))));
        q = 1.0f + s * (SA1 + s * (SA2 + s * (SA3 + s * (SA4 + s * (SA5 + s * (SA6 + s * (SA7 + s * SA8)))))));
    } else {
        r = RB0 + s * (RB1 + s * (RB2 + s * (RB3 + s * (RB4 + s * (RB5 + s * RB6)))));
        q = 1.0f + s * (SB1 + s * (SB2 + s * (SB3 + s * (SB4 + s * (SB5 + s * (SB6 + s * SB7))))));
    }
    const float z = lm_from(lm_bits(x) & 0xffffe000u);
    return ok_expf(-z * z - 0.5625f) * ok_expf((z - x) * (z + x) + r / q) / x;
}

float ok_erff(float x)
{
    const float EFX8 = 1.0270333290e+00f;
    const float P0 = 1.2837916613e-01f, P1 = -3.2504209876e-01f, P2 = -2.8481749818e-02f,
                P3 = -5.7702702470e-03f, P4 = -2.3763017452e-05f;
    const float Q1 = 3.9791721106e-01f, Q2 = 6.5022252500e-02f, Q3 = 5.0813062117e-03f,
                Q4 = 1.3249473704e-04f, Q5 = -3.9602282413e-06f;
    uint32_t ax = lm_bits(x);
    const int neg = (int)(ax >> 31);
    ax &= 0x7fffffffu;
    if (ax >= 0x7f800000u)
        return (float)(1 - 2 * neg) + 1 / x; /* erf(+-inf) = +-1, erf(NaN) = NaN */
    if (ax < 0x3f580000u) {                  /* |x| < 0.84375 */
        if (ax < 0x31800000u)                /* |x| < 2^-28 */
            return 0.125f * (8 * x + EFX8 * x);
        const float z = x * x;
        const float r = P0 + z * (P1 + z * (P2 + z * (P3 + z * P4)));
        const float s = 1 + z * (Q1 + z * (Q2 + z * (Q3 + z * (Q4 + z * Q5))));
        const float y = r / s;
        return x + x * y;
    }
    float y;
    if (ax < 0x40c00000u)                     /* |x| < 6 */
        y = 1 - lm_erfc_tail(ax, x);
    else
        y = 1 - 0x1p-120f;
    return neg ? -y : y;
}

/* ---- sinf / cosf --------------------------------------------------------
 * fdlibm's method in f64 arithmetic (presk_libm.c:672-746 the kernels
 * __sindf/__cosdf, 1372-1447 __rem_pio2f, 749-1189 __rem_pio2_large,
 * 2054-2111 sinf, 2213-2272 cosf): |x| <= pi/4 direct; up to 9pi/4 one
 * subtraction of a multiple of pi/2 rounded to f64; below 2^28*pi/2 the
 * reduction by 25+53 bits of pi/2; beyond it Payne-Hanek with the 24-bit
 * digits of 2/pi (one piece of x, single precision: fdlibm's jk = 3). */

/* minimax polynomials of sin(x) on [-pi/4, pi/4] (odd) and cos(x) (even) */
static float lm_ksin(double x)
{
    const double S1 = -0x15555554cbac77.0p-55, S2 = 0x111110896efbb2.0p-59,
                 S3 = -0x1a00f9e2cae774.0p-65, S4 = 0x16cd878c3b46a7.0p-71;
    const double z = x * x, w = z * z, r = S3 + z * S4, s = z * x;
    return (float)((x + s * (S1 + z * S2)) + s * w * r);
}
static float lm_kcos(double x)
{
    const double C0 = -0x1ffffffd0c5e81.0p-54, C1 = 0x155553e1053a42.0p-57,
                 C2 = -0x16c087e80f1e27.0p-62, C3 = 0x199342e0ee5069.0p-68;
    const double z = x * x, w = z * z, r = C2 + z * C3;
    return (float)(((1.0 + z * C0) + w * C1) + (w * z) * r);
}

/* the first 24-bit digits of 2/pi after the binary point: digit i is
 * ipio2[i] * 2^(-24(i+1)); an f32 argument needs no more than these */
static const int32_t lm_ipio2[] = {
    0xA2F983, 0x6E4E44, 0x1529FC, 0x2757D1, 0xF534DD, 0xC0DB62, 0x95993C, 0x439041, 0xFE5163, 0xABDEBB,
    0xC561B7, 0x246E3A, 0x424DD2, 0xE00649, 0x2EEA09, 0xD1921C, 0xFE1DEB, 0x1CB129, 0xA73EE8, 0x8235F5,
    0x2EBB44, 0x84E99C, 0x7026B4, 0x5F7E41, 0x3991D6, 0x398353, 0x39F49C, 0x845F8B, 0xBDF928, 0x3B1FF8,
};
/* pi/2 cut into 24-bit pieces */
static const double lm_pio2_24[] = {
    1.57079625129699707031e+00, 7.54978941586159635335e-08, 5.39030252995776476554e-15, 3.28200341580791294123e-22,
};

/* x (a positive f32 of exponent e0 + 23, as an integer of 24 bits times
 * 2^e0) reduced mod pi/2: returns the quotient's low bits, the remainder in
 * *y.  The steps of fdlibm's k_rem_pio2 with one piece and jk = 3. */
static int lm_rem_pio2_big(double x0, int e0, double *y)
{
    enum { JK = 3 };
    int32_t iq[20];
    double f[20], q[20], fq[20] = {0};
    int jv = (e0 - 3) / 24;
    if (jv < 0)
        jv = 0;
    int q0 = e0 - 24 * (jv + 1);
    for (int i = 0; i <= JK; i++) {
        const int j = jv + i;
        f[i] = j < 0 ? 0.0 : (double)lm_ipio2[j];
    }
    for (int i = 0; i <= JK; i++)
        q[i] = 0.0 + x0 * f[i];
    int jz = JK, n, ih;
    double z;
    for (;;) {
        /* the product's 24-bit digits, most significant last */
        z = q[jz];
        for (int i = 0, j = jz; j > 0; i++, j--) {
            const double hi = (double)(int32_t)(0x1p-24 * z);
            iq[i] = (int32_t)(z - 0x1p24 * hi);
            z = q[j - 1] + hi;
        }
        /* the integer part mod 8 */
        z = ldexp(z, q0);
        z -= 8.0 * floor(z * 0.125);
        n = (int32_t)z;
        z -= (double)n;
        ih = 0;
        if (q0 > 0) {
            const int32_t top = iq[jz - 1] >> (24 - q0);
            n += top;
            iq[jz - 1] -= top << (24 - q0);
            ih = iq[jz - 1] >> (23 - q0);
        } else if (q0 == 0) {
            ih = iq[jz - 1] >> 23;
        } else if (z >= 0.5) {
            ih = 2;
        }
        if (ih > 0) { /* fraction >= 1/2: take 1 - fraction, n + 1 */
            n += 1;
            int carry = 0;
            for (int i = 0; i < jz; i++) {
                const int32_t d = iq[i];
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
                if (carry != 0)
                    z -= ldexp(1.0, q0);
            }
        }
        /* all digits of the fraction cancelled: take more of 2/pi */
        if (z == 0.0) {
            int32_t any = 0;
            for (int i = jz - 1; i >= JK; i--)
                any |= iq[i];
            if (any == 0) {
                int k = 1;
                while (iq[JK - k] == 0)
                    k++;
                for (int i = jz + 1; i <= jz + k; i++) {
                    f[i] = (double)lm_ipio2[jv + i];
                    q[i] = 0.0 + x0 * f[i];
                }
                jz += k;
                continue;
            }
        }
        break;
    }
    /* drop the zero digits, or split a fraction past 24 bits */
    if (z == 0.0) {
        jz -= 1;
        q0 -= 24;
        while (iq[jz] == 0) {
            jz--;
            q0 -= 24;
        }
    } else {
        z = ldexp(z, -q0);
        if (z >= 0x1p24) {
            const double hi = (double)(int32_t)(0x1p-24 * z);
            iq[jz] = (int32_t)(z - 0x1p24 * hi);
            jz += 1;
            q0 += 24;
            iq[jz] = (int32_t)hi;
        } else {
            iq[jz] = (int32_t)z;
        }
    }
    double fw = ldexp(1.0, q0);
    for (int i = jz; i >= 0; i--) {
        q[i] = fw * (double)iq[i];
        fw *= 0x1p-24;
    }
    /* times pi/2, digit by digit */
    for (int i = jz; i >= 0; i--) {
        fw = 0.0;
        for (int k = 0; k <= JK && k <= jz - i; k++)
            fw += lm_pio2_24[k] * q[i + k];
        fq[jz - i] = fw;
    }
    fw = 0.0;
    for (int i = jz; i >= 0; i--)
        fw += fq[i];
    *y = ih == 0 ? fw : -fw;
    return n;
}

/* x mod pi/2 in *y (f64), the quotient's low bits returned */
static int lm_rem_pio2f(float x, double *y)
{
    const double toint = 1.5 / 0x1p-52, invpio2 = 6.36619772367581382433e-01,
                 pio2_1 = 1.57079631090164184570e+00, pio2_1t = 1.58932547735281966916e-08;
    const uint32_t b = lm_bits(x), ix = b & 0x7fffffffu;
    if (ix < 0x4dc90fdbu) {  /* |x| < 2^28 pi/2: 25 + 53 bits of pi/2 */
        const double fn = (double)x * invpio2 + toint - toint;
        *y = x - fn * pio2_1 - fn * pio2_1t;
        return (int32_t)fn;
    }
    if (ix >= 0x7f800000u) {
        *y = x - x;
        return 0;
    }
    const int e0 = (int)(ix >> 23) - (0x7f + 23);
    double r;
    const int n = lm_rem_pio2_big((double)lm_from(ix - ((uint32_t)e0 << 23)), e0, &r);
    if (b >> 31) {
        *y = -r;
        return -n;
    }
    *y = r;
    return n;
}

float ok_sinf(float x)
{
    const double p1 = 1 * 1.57079632679489661923, p2 = 2 * 1.57079632679489661923,
                 p3 = 3 * 1.57079632679489661923, p4 = 4 * 1.57079632679489661923;
    const uint32_t b = lm_bits(x), ix = b & 0x7fffffffu;
    const int neg = (int)(b >> 31);
    if (ix <= 0x3f490fdau)
        return ix < 0x39800000u ? x : lm_ksin(x);
    if (ix <= 0x407b53d1u) {
        if (ix <= 0x4016cbe3u)
            return neg ? -lm_kcos(x + p1) : lm_kcos(x - p1);
        return lm_ksin(neg ? -(x + p2) : -(x - p2));
    }
    if (ix <= 0x40e231d5u) {
        if (ix <= 0x40afeddfu)
            return neg ? lm_kcos(x + p3) : -lm_kcos(x - p3);
        return lm_ksin(neg ? x + p4 : x - p4);
    }
    if (ix >= 0x7f800000u)
        return x - x;
    double y;
    switch (lm_rem_pio2f(x, &y) & 3) {
    case 0: return lm_ksin(y);
    case 1: return lm_kcos(y);
    case 2: return lm_ksin(-y);
    default: return -lm_kcos(y);
    }
}

float ok_cosf(float x)
{
    const double p1 = 1 * 1.57079632679489661923, p2 = 2 * 1.57079632679489661923,
                 p3 = 3 * 1.57079632679489661923, p4 = 4 * 1.57079632679489661923;
    const uint32_t b = lm_bits(x), ix = b & 0x7fffffffu;
    const int neg = (int)(b >> 31);
    if (ix <= 0x3f490fdau)
        return ix < 0x39800000u ? 1.0f : lm_kcos(x);
    if (ix <= 0x407b53d1u) {
        if (ix > 0x4016cbe3u)
            return -lm_kcos(neg ? x + p2 : x - p2);
        return neg ? lm_ksin(x + p1) : lm_ksin(p1 - x);
    }
    if (ix <= 0x40e231d5u) {
        if (ix > 0x40afeddfu)
            return lm_kcos(neg ? x + p4 : x - p4);
        return neg ? lm_ksin(-x - p3) : lm_ksin(x - p3);
    }
    if (ix >= 0x7f800000u)
        return x - x;
    double y;
    switch ((unsigned)lm_rem_pio2f(x, &y) & 3) {
    case 0: return lm_kcos(y);
    case 1: return lm_ksin(-y);
    case 2: return -lm_kcos(y);
    default: return lm_ksin(y);
    }
}

/* ======================================================================
 * f64: the interpreter's f64 arm (exec.rs:115-130) calls the same crate's
 * double functions, musl 1.1.22's fdlibm code:
 *
 *   ok_exp    follows presk_libm.c:1520-1604 (e_exp)
 *   ok_log    follows presk_libm.c:1738-1810 (e_log)
 *   lm_expm1  follows presk_libm.c:323-435   (s_expm1)
 *   ok_tanh   follows presk_libm.c:1871-1914 (s_tanh)
 *   ok_erf    follows presk_libm.c:2383-2541 (s_erf: erfc1, erfc2, erf)
 *   ok_sin    follows presk_libm.c:1999-2053, ok_cos :2159-2212, with the
 *             kernels :575-690 (k_sin, k_cos), the reduction :1221-1402
 *             (rem_pio2) and its large-argument form :876-1220 at double
 *             precision (prec 1: jk = 4, two result words)
 *
 * Pinned by tests/test_oracle_scalar.py on a fixed sample of 2^24 inputs per
 * function (every class of argument the reductions distinguish), digest
 * against the reference's C compiled into oracle/_ref.
 * ====================================================================== */

static inline uint64_t lm_bits64(double x) { uint64_t b; memcpy(&b, &x, 8); return b; }
static inline double lm_from64(uint64_t b) { double x; memcpy(&x, &b, 8); return x; }

/* y * 2^n in at most two scalings before the final power of two (scalbn) */
static double lm_scalbn(double y, int n)
{
    if (n > 1023) {
        y *= 0x1p1023;
        n -= 1023;
        if (n > 1023) {
            y *= 0x1p1023;
            n -= 1023;
            if (n > 1023)
                n = 1023;
        }
    } else if (n < -1022) {
        /* keep the final scaling below -53 so that a subnormal result is
         * rounded once */
        y *= 0x1p-1022 * 0x1p53;
        n += 1022 - 53;
        if (n < -1022) {
            y *= 0x1p-1022 * 0x1p53;
            n += 1022 - 53;
            if (n < -1022)
                n = -1022;
        }
    }
    return y * lm_from64((uint64_t)(0x3ff + n) << 52);
}

double ok_exp(double x)
{
    /* x = k ln2 + r, |r| <= ln2/2, ln2 split so that k*LN2_HI is exact;
     * exp(r) = 1 + r + r c(r) / (2 - c(r)), c the degree-5 remez of
     * r - r^2 (P1 + ... + P5 r^8) */
    const double LN2_HI = 6.93147180369123816490e-01, LN2_LO = 1.90821492927058770002e-10,
                 INV_LN2 = 1.44269504088896338700e+00;
    const double P1 = 1.66666666666666019037e-01, P2 = -2.77777777770155933842e-03,
                 P3 = 6.61375632143793436117e-05, P4 = -1.65339022054652515390e-06,
                 P5 = 4.13813679705723846039e-08;
    const uint32_t top = (uint32_t)(lm_bits64(x) >> 32);
    const int neg = (int)(top >> 31);
    const uint32_t ax = top & 0x7fffffffu;
    if (ax >= 0x4086232bu) {                 /* |x| >= 708.39 or NaN */
        if (x != x)
            return x;
        if (x > 709.782712893383973096)
            return x * 0x1p1023;              /* overflow */
        if (x < -708.39641853226410622 && x < -745.13321910194110842)
            return 0;                         /* underflow */
    }
    double hi, lo;
    int k;
    if (ax > 0x3fd62e42u) {                  /* |x| > ln2/2 */
        if (ax >= 0x3ff0a2b2u)               /* |x| >= 1.5 ln2 */
            k = (int)(INV_LN2 * x + (neg ? -0.5 : 0.5));
        else
            k = 1 - neg - neg;
        hi = x - k * LN2_HI;
        lo = k * LN2_LO;
        x = hi - lo;
    } else if (ax > 0x3e300000u) {           /* |x| > 2^-28 */
        k = 0;
        hi = x;
        lo = 0;
    } else {
        return 1 + x;
    }
    const double xx = x * x;
    const double c = x - xx * (P1 + xx * (P2 + xx * (P3 + xx * (P4 + xx * P5))));
    const double y = 1 + (x * c / (2 - c) - lo + hi);
    return k == 0 ? y : lm_scalbn(y, k);
}

double ok_log(double x)
{
    /* x = 2^k (1 + f), 1 + f in [sqrt(2)/2, sqrt(2)); log(1+f) = f - hfsq +
     * s (hfsq + R(s^2)), s = f / (2 + f), R the degree-7 remez */
    const double LN2_HI = 6.93147180369123816490e-01, LN2_LO = 1.90821492927058770002e-10;
    const double LG1 = 6.666666666666735130e-01, LG2 = 3.999999999940941908e-01, LG3 = 2.857142874366239149e-01,
                 LG4 = 2.222219843214978396e-01, LG5 = 1.818357216161805012e-01, LG6 = 1.531383769920937332e-01,
                 LG7 = 1.479819860511658591e-01;
    uint64_t b = lm_bits64(x);
    uint32_t top = (uint32_t)(b >> 32);
    int k = 0;
    if (top < 0x00100000u || (top >> 31)) {  /* subnormal, zero or negative */
        if ((b << 1) == 0)
            return -1 / (x * x);              /* log(+-0) = -inf */
        if (top >> 31)
            return (x - x) / 0.0;             /* log(<0) = NaN */
        k -= 54;                              /* subnormal: scale up */
        x *= 0x1p54;
        b = lm_bits64(x);
        top = (uint32_t)(b >> 32);
    } else if (top >= 0x7ff00000u) {
        return x;                             /* inf or NaN */
    } else if (top == 0x3ff00000u && (b << 32) == 0) {
        return 0;                             /* log(1) */
    }
    /* move the mantissa into [sqrt(2)/2, sqrt(2)) */
    top += 0x3ff00000u - 0x3fe6a09eu;
    k += (int)(top >> 20) - 0x3ff;
    top = (top & 0x000fffffu) + 0x3fe6a09eu;
    x = lm_from64((uint64_t)top << 32 | (b & 0xffffffffu));
    const double f = x - 1.0, hfsq = 0.5 * f * f, s = f / (2.0 + f), z = s * s, w = z * z;
    const double t1 = w * (LG2 + w * (LG4 + w * LG6));
    const double t2 = z * (LG1 + w * (LG3 + w * (LG5 + w * LG7)));
    const double R = t2 + t1, dk = k;
    return s * (hfsq + R) + dk * LN2_LO - hfsq + f + dk * LN2_HI;
}

/* e^x - 1: x = k ln2 + r (with the reduction's rounding error c carried),
 * e^r - 1 = r + r^2/2 + r^3/6 * (rational of r^2 with scaled Q1..Q5) */
static double lm_expm1(double x)
{
    const double O_THRESHOLD = 7.09782712893383973096e+02, LN2_HI = 6.93147180369123816490e-01,
                 LN2_LO = 1.90821492927058770002e-10, INV_LN2 = 1.44269504088896338700e+00;
    const double Q1 = -3.33333333333331316428e-02, Q2 = 1.58730158725481460165e-03,
                 Q3 = -7.93650757867487942473e-05, Q4 = 4.00821782732936239552e-06,
                 Q5 = -2.01099218183624371326e-07;
    const uint64_t b = lm_bits64(x);
    const uint32_t ax = (uint32_t)(b >> 32) & 0x7fffffffu;
    const int neg = (int)(b >> 63);
    if (ax >= 0x4043687au) {                 /* |x| >= 56 ln2 or NaN */
        if (x != x)
            return x;
        if (neg)
            return -1;
        if (x > O_THRESHOLD)
            return x * 0x1p1023;
    }
    double hi, lo, c = 0;
    int k;
    if (ax > 0x3fd62e42u) {                  /* |x| > ln2/2 */
        if (ax < 0x3ff0a2b2u) {              /* and < 1.5 ln2 */
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
    } else if (ax < 0x3c900000u) {           /* |x| < 2^-54 */
        return x;
    } else {
        k = 0;
    }
    const double hfx = 0.5 * x, hxs = x * hfx;
    const double r1 = 1.0 + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    const double t = 3.0 - r1 * hfx;
    double e = hxs * ((r1 - t) / (6.0 - x * t));
    if (k == 0)
        return x - (x * e - hxs);
    e = x * (e - c) - c;
    e -= hxs;
    if (k == -1)
        return 0.5 * (x - e) - 0.5;
    if (k == 1) {
        if (x < -0.25)
            return -2.0 * (e - (x + 0.5));
        return 1.0 + 2.0 * (x - e);
    }
    const double twopk = lm_from64((uint64_t)(0x3ff + k) << 52);
    if (k < 0 || k > 56) {
        double y = x - e + 1.0;
        y = k == 1024 ? y * 2.0 * 0x1p1023 : y * twopk;
        return y - 1.0;
    }
    const double twomk = lm_from64((uint64_t)(0x3ff - k) << 52);
    if (k < 20)
        return (x - e + (1 - twomk)) * twopk;
    return (x - (e + twomk) + 1) * twopk;
}

double ok_tanh(double x)
{
    const uint64_t b = lm_bits64(x);
    const int neg = (int)(b >> 63);
    x = lm_from64(b & 0x7fffffffffffffffull);
    const uint32_t w = (uint32_t)(b >> 32) & 0x7fffffffu;
    double t;
    if (w > 0x3fe193eau) {                   /* |x| > log(3)/2 or NaN */
        if (w > 0x40340000u) {               /* |x| > 20 or NaN */
            t = 1 - 0 / x;
        } else {
            t = lm_expm1(2 * x);
            t = 1 - 2 / (t + 2);
        }
    } else if (w > 0x3fd058aeu) {            /* |x| > log(5/3)/2 */
        t = lm_expm1(2 * x);
        t = t / (t + 2);
    } else if (w >= 0x00100000u) {           /* normal */
        t = lm_expm1(-2 * x);
        t = -t / (t + 2);
    } else {
        t = x;                                /* subnormal */
    }
    return neg ? -t : t;
}

/* erfc on [0.84375, 1.25): 1 - erx - P(s)/Q(s), s = |x| - 1 */
static double lm_erfc_mid(double x)
{
    const double ERX = 8.45062911510467529297e-01;
    const double PA0 = -2.36211856075265944077e-03, PA1 = 4.14856118683748331666e-01,
                 PA2 = -3.72207876035701323847e-01, PA3 = 3.18346619901161753674e-01,
                 PA4 = -1.10894694282396677476e-01, PA5 = 3.54783043256182359371e-02,
                 PA6 = -2.16637559486879084300e-03;
    const double QA1 = 1.06420880400844228286e-01, QA2 = 5.40397917702171048937e-01,
                 QA3 = 7.18286544141962662868e-02, QA4 = 1.26171219808761642112e-01,
                 QA5 = 1.36370839120290507362e-02, QA6 = 1.19844998467991074170e-02;
    const double s = fabs(x) - 1;
    const double P = PA0 + s * (PA1 + s * (PA2 + s * (PA3 + s * (PA4 + s * (PA5 + s * PA6)))));
    const double Q = 1 + s * (QA1 + s * (QA2 + s * (QA3 + s * (QA4 + s * (QA5 + s * QA6)))));
    return 1 - ERX - P / Q;
}

/* erfc on [0.84375, 6): the middle piece below 1.25, else
 * exp(-z^2 - 0.5625) exp((z - x)(z + x) + R/S) / x, z = x with its low word
 * cleared, R/S rationals of 1/x^2 on [1.25, 1/0.35) and [1/0.35, 6) */
static double lm_erfc_far(uint32_t ix, double x)
{
    const double RA0 = -9.86494403484714822705e-03, RA1 = -6.93858572707181764372e-01,
                 RA2 = -1.05586262253232909814e+01, RA3 = -6.23753324503260060396e+01,
                 RA4 = -1.62396669462573470355e+02, RA5 = -1.84605092906711035994e+02,
                 RA6 = -8.12874355063065934246e+01, RA7 = -9.81432934416914548592e+00;
    const double SA1 = 1.96512716674392571292e+01, SA2 = 1.37657754143519042600e+02,
                 SA3 = 4.34565877475229228821e+02, SA4 = 6.45387271733267880336e+02,
                 SA5 = 4.29008140027567833386e+02, SA6 = 1.08635005541779435134e+02,
                 SA7 = 6.57024977031928170135e+00, SA8 = -6.04244152148580987438e-02;
    const double RB0 = -9.86494292470009928597e-03, RB1 = -7.99283237680523006574e-01,
                 RB2 = -1.77579549177547519889e+01, RB3 = -1.60636384855821916062e+02,
                 RB4 = -6.37566443368389627722e+02, RB5 = -1.02509513161107724954e+03,
                 RB6 = -4.83519191608651397019e+02;
    const double SB1 = 3.03380607434824582924e+01, SB2 = 3.25792512996573918826e+02,
                 SB3 = 1.53672958608443695994e+03, SB4 = 3.19985821950859553908e+03,
                 SB5 = 2.55305040643316442583e+03, SB6 = 4.74528541206955367215e+02,
                 SB7 = -2.24409524465858183362e+01;
    if (ix < 0x3ff40000u)                    /* |x| < 1.25 */
        return lm_erfc_mid(x);
    x = fabs(x);
    const double s = 1 / (x * x);
    double R, S;
    if (ix < 0x4006db6du) {                  /* |x| < 1/0.35 */
        R = RA0 + s * (RA1 + s * (RA2 + s * (RA3 + s * (RA4 + s * (RA5 + s * (RA6 + s * RA7))))));
        S = 1.0 + s * (SA1 + s * (SA2 + s * (SA3 + s * (SA4 + s * (SA5 + s * (SA6 + s * (SA7 + s * SA8)))))));
    } else {
        R = RB0 + s * (RB1 + s * (RB2 + s * (RB3 + s * (RB4 + s * (RB5 + s * RB6)))));
        S = 1.0 + s * (SB1 + s * (SB2 + s * (SB3 + s * (SB4 + s * (SB5 + s * (SB6 + s * SB7))))));
    }
    const double z = lm_from64(lm_bits64(x) & 0xffffffff00000000ull);
    return ok_exp(-z * z - 0.5625) * ok_exp((z - x) * (z + x) + R / S) / x;
}

double ok_erf(double x)
{
    const double EFX8 = 1.02703333676410069053e+00;
    const double PP0 = 1.28379167095512558561e-01, PP1 = -3.25042107247001499370e-01,
                 PP2 = -2.84817495755985104766e-02, PP3 = -5.77027029648944159157e-03,
                 PP4 = -2.37630166566501626084e-05;
    const double QQ1 = 3.97917223959155352819e-01, QQ2 = 6.50222499887672944485e-02,
                 QQ3 = 5.08130628187576562776e-03, QQ4 = 1.32494738004321644526e-04,
                 QQ5 = -3.96022827877536812320e-06;
    const uint32_t top = (uint32_t)(lm_bits64(x) >> 32);
    const int neg = (int)(top >> 31);
    const uint32_t ix = top & 0x7fffffffu;
    if (ix >= 0x7ff00000u)                   /* NaN, +-inf */
        return 1 - 2 * neg + 1 / x;
    if (ix < 0x3feb0000u) {                  /* |x| < 0.84375 */
        if (ix < 0x3e300000u)                /* |x| < 2^-28 */
            return 0.125 * (8 * x + EFX8 * x);
        const double z = x * x;
        const double r = PP0 + z * (PP1 + z * (PP2 + z * (PP3 + z * PP4)));
        const double s = 1.0 + z * (QQ1 + z * (QQ2 + z * (QQ3 + z * (QQ4 + z * QQ5))));
        return x + x * (r / s);
    }
    const double y = ix < 0x40180000u ? 1 - lm_erfc_far(ix, x) : 1 - 0x1p-1022;
    return neg ? -y : y;
}

/* the minimax kernels of sin and cos on [-pi/4, pi/4] for x + y (y the
 * reduction's tail; iy = 0: y is zero) */
static double lm_ksin64(double x, double y, int iy)
{
    const double S1 = -1.66666666666666324348e-01, S2 = 8.33333333332248946124e-03,
                 S3 = -1.98412698298579493134e-04, S4 = 2.75573137070700676789e-06,
                 S5 = -2.50507602534068634195e-08, S6 = 1.58969099521155010221e-10;
    const double z = x * x, w = z * z;
    const double r = S2 + z * (S3 + z * S4) + z * w * (S5 + z * S6);
    const double v = z * x;
    if (iy == 0)
        return x + v * (S1 + z * r);
    return x - ((z * (0.5 * y - v * r) - y) - v * S1);
}
static double lm_kcos64(double x, double y)
{
    const double C1 = 4.16666666666666019037e-02, C2 = -1.38888888888741095749e-03,
                 C3 = 2.48015872894767294178e-05, C4 = -2.75573143513906633035e-07,
                 C5 = 2.08757232129817482790e-09, C6 = -1.13596475577881948265e-11;
    const double z = x * x;
    double w = z * z;
    const double r = z * (C1 + z * (C2 + z * C3)) + w * w * (C4 + z * (C5 + z * C6));
    const double hz = 0.5 * z;
    w = 1.0 - hz;
    return w + (((1.0 - w) - hz) + (z * r - x * y));
}

/* the 24-bit digits of 2/pi after the binary point (digit i weighs
 * 2^(-24(i+1))), as far as an f64 argument needs them */
static const int32_t lm_ipio2_64[] = {
    0xA2F983, 0x6E4E44, 0x1529FC, 0x2757D1, 0xF534DD, 0xC0DB62, 0x95993C, 0x439041, 0xFE5163, 0xABDEBB,
    0xC561B7, 0x246E3A, 0x424DD2, 0xE00649, 0x2EEA09, 0xD1921C, 0xFE1DEB, 0x1CB129, 0xA73EE8, 0x8235F5,
    0x2EBB44, 0x84E99C, 0x7026B4, 0x5F7E41, 0x3991D6, 0x398353, 0x39F49C, 0x845F8B, 0xBDF928, 0x3B1FF8,
    0x97FFDE, 0x05980F, 0xEF2F11, 0x8B5A0A, 0x6D1F6D, 0x367ECF, 0x27CB09, 0xB74F46, 0x3F669E, 0x5FEA2D,
    0x7527BA, 0xC7EBE5, 0xF17B3D, 0x0739F7, 0x8A5292, 0xEA6BFB, 0x5FB11F, 0x8D5D08, 0x560330, 0x46FC7B,
    0x6BABF0, 0xCFBC20, 0x9AF436, 0x1DA9E3, 0x91615E, 0xE61B08, 0x659985, 0x5F14A0, 0x68408D, 0xFFD880,
    0x4D7327, 0x310606, 0x1556CA, 0x73A8C9, 0x60E27B, 0xC08C6B,
};
/* pi/2 in 24-bit pieces */
static const double lm_pio2_24_64[] = {
    1.57079625129699707031e+00, 7.54978941586159635335e-08, 5.39030252995776476554e-15,
    3.28200341580791294123e-22, 1.27065575308067607349e-29,
};

/* x (nx pieces of 24 bits, x[0] times 2^e0 the leading one) reduced mod
 * pi/2 to y[0] + y[1]: the steps of fdlibm's k_rem_pio2 at double precision
 * (jk = 4 digits of the product kept, more taken when the fraction cancels);
 * returns the quotient's low 3 bits */
static int lm_rem_pio2_large(const double *x, double *y, int e0, int nx)
{
    enum { JK = 4 };
    int32_t iq[20];
    double f[20], q[20], fq[20] = {0};
    const int jx = nx - 1;
    int jv = (e0 - 3) / 24;
    if (jv < 0)
        jv = 0;
    int q0 = e0 - 24 * (jv + 1);
    for (int i = 0, j = jv - jx; i <= jx + JK; i++, j++)
        f[i] = j < 0 ? 0.0 : (double)lm_ipio2_64[j];
    for (int i = 0; i <= JK; i++) {
        double fw = 0.0;
        for (int j = 0; j <= jx; j++)
            fw += x[j] * f[jx + i - j];
        q[i] = fw;
    }
    int jz = JK, n, ih;
    double z;
    for (;;) {
        z = q[jz];
        for (int i = 0, j = jz; j > 0; i++, j--) {
            const double hi = (double)(int32_t)(0x1p-24 * z);
            iq[i] = (int32_t)(z - 0x1p24 * hi);
            z = q[j - 1] + hi;
        }
        z = lm_scalbn(z, q0);
        z -= 8.0 * floor(z * 0.125);
        n = (int32_t)z;
        z -= (double)n;
        ih = 0;
        if (q0 > 0) {
            const int32_t top = iq[jz - 1] >> (24 - q0);
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
            for (int i = 0; i < jz; i++) {
                const int32_t d = iq[i];
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
                if (carry != 0)
                    z -= lm_scalbn(1.0, q0);
            }
        }
        if (z == 0.0) {
            int32_t any = 0;
            for (int i = jz - 1; i >= JK; i--)
                any |= iq[i];
            if (any == 0) {
                int k = 1;
                while (iq[JK - k] == 0)
                    k++;
                for (int i = jz + 1; i <= jz + k; i++) {
                    f[jx + i] = (double)lm_ipio2_64[jv + i];
                    double fw = 0.0;
                    for (int j = 0; j <= jx; j++)
                        fw += x[j] * f[jx + i - j];
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
            jz--;
            q0 -= 24;
        }
    } else {
        z = lm_scalbn(z, -q0);
        if (z >= 0x1p24) {
            const double hi = (double)(int32_t)(0x1p-24 * z);
            iq[jz] = (int32_t)(z - 0x1p24 * hi);
            jz += 1;
            q0 += 24;
            iq[jz] = (int32_t)hi;
        } else {
            iq[jz] = (int32_t)z;
        }
    }
    double fw = lm_scalbn(1.0, q0);
    for (int i = jz; i >= 0; i--) {
        q[i] = fw * (double)iq[i];
        fw *= 0x1p-24;
    }
    for (int i = jz; i >= 0; i--) {
        fw = 0.0;
        for (int k = 0; k <= JK && k <= jz - i; k++)
            fw += lm_pio2_24_64[k] * q[i + k];
        fq[jz - i] = fw;
    }
    fw = 0.0;
    for (int i = jz; i >= 0; i--)
        fw += fq[i];
    y[0] = ih == 0 ? fw : -fw;
    fw = fq[0] - fw;
    for (int i = 1; i <= jz; i++)
        fw += fq[i];
    y[1] = ih == 0 ? fw : -fw;
    return n & 7;
}

/* x mod pi/2 as y[0] + y[1], the quotient's low bits returned (the caller
 * handles |x| <= pi/4): one subtraction of n pi/2 (n <= 4, 33 + 53 bits of
 * pi/2) up to 9pi/4 outside the cancelling points, rounds of 33 bits of
 * pi/2 up to 2^20 pi/2, Payne-Hanek beyond */
static int lm_rem_pio2(double x, double *y)
{
    const double TOINT = 1.5 / 0x1p-52, INVPIO2 = 6.36619772367581382433e-01,
                 PIO2_1 = 1.57079632673412561417e+00, PIO2_1T = 6.07710050650619224932e-11,
                 PIO2_2 = 6.07710050630396597660e-11, PIO2_2T = 2.02226624879595063154e-21,
                 PIO2_3 = 2.02226624871116645580e-21, PIO2_3T = 8.47842766036889956997e-32;
    const uint64_t b = lm_bits64(x);
    const int neg = (int)(b >> 63);
    const uint32_t ix = (uint32_t)(b >> 32) & 0x7fffffffu;
    int near = 0;    /* the multiple of pi/2 one subtraction removes, 0: none */
    if (ix <= 0x400f6a7au) {                             /* |x| <= 5pi/4 */
        if ((ix & 0xfffffu) != 0x921fbu)                 /* not near pi/2, pi */
            near = ix <= 0x4002d97cu ? 1 : 2;            /* 3pi/4 */
    } else if (ix <= 0x401c463bu) {                      /* |x| <= 9pi/4 */
        if (ix <= 0x4015fdbcu) {                         /* 7pi/4 */
            if (ix != 0x4012d97cu)                       /* not near 3pi/2 */
                near = 3;
        } else if (ix != 0x401921fbu) {                  /* not near 2pi */
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
    if (ix < 0x413921fbu) {                              /* |x| < 2^20 pi/2 */
        const double fn = x * INVPIO2 + TOINT - TOINT;
        const int n = (int32_t)fn;
        double r = x - fn * PIO2_1;
        double w = fn * PIO2_1T;
        y[0] = r - w;
        const int ex = (int)(ix >> 20);
        int ey = (int)(lm_bits64(y[0]) >> 52 & 0x7ff);
        if (ex - ey > 16) {                              /* second round, 118 bits */
            double t = r;
            w = fn * PIO2_2;
            r = t - w;
            w = fn * PIO2_2T - ((t - r) - w);
            y[0] = r - w;
            ey = (int)(lm_bits64(y[0]) >> 52 & 0x7ff);
            if (ex - ey > 49) {                          /* third round, 151 bits */
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
    if (ix >= 0x7ff00000u) {                             /* inf or NaN */
        y[0] = y[1] = x - x;
        return 0;
    }
    /* |x| as up to three 24-bit pieces, the first scaled into [2^23, 2^24) */
    double z = lm_from64((b & (~0ull >> 12)) | ((uint64_t)(0x3ff + 23) << 52));
    double tx[3], ty[2];
    int i;
    for (i = 0; i < 2; i++) {
        tx[i] = (double)(int32_t)z;
        z = (z - tx[i]) * 0x1p24;
    }
    tx[i] = z;
    while (tx[i] == 0.0)
        i--;
    const int n = lm_rem_pio2_large(tx, ty, (int)(ix >> 20) - (0x3ff + 23), i + 1);
    if (neg) {
        y[0] = -ty[0];
        y[1] = -ty[1];
        return -n;
    }
    y[0] = ty[0];
    y[1] = ty[1];
    return n;
}

double ok_sin(double x)
{
    const uint32_t ix = (uint32_t)(lm_bits64(x) >> 32) & 0x7fffffffu;
    if (ix <= 0x3fe921fbu)                   /* |x| <= pi/4 */
        return ix < 0x3e500000u ? x : lm_ksin64(x, 0.0, 0);
    if (ix >= 0x7ff00000u)
        return x - x;
    double y[2];
    switch ((unsigned)lm_rem_pio2(x, y) & 3) {
    case 0: return lm_ksin64(y[0], y[1], 1);
    case 1: return lm_kcos64(y[0], y[1]);
    case 2: return -lm_ksin64(y[0], y[1], 1);
    default: return -lm_kcos64(y[0], y[1]);
    }
}

double ok_cos(double x)
{
    const uint32_t ix = (uint32_t)(lm_bits64(x) >> 32) & 0x7fffffffu;
    if (ix <= 0x3fe921fbu)                   /* |x| <= pi/4 */
        return ix < 0x3e46a09eu ? 1.0 : lm_kcos64(x, 0);
    if (ix >= 0x7ff00000u)
        return x - x;
    double y[2];
    switch ((unsigned)lm_rem_pio2(x, y) & 3) {
    case 0: return lm_kcos64(y[0], y[1]);
    case 1: return -lm_ksin64(y[0], y[1], 1);
    case 2: return -lm_kcos64(y[0], y[1]);
    default: return lm_ksin64(y[0], y[1], 1);
    }
}
