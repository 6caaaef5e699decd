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
