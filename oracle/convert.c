/* oracle/convert.c -- TEST INFRASTRUCTURE ONLY (the parity oracle).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * include, link or run anything under oracle/.  The product (presk_amd/) never
 * does.
 *
 * The host's conversion of a buffer at a kernel's edge, restated:
 * Buf::of(to, b.to_f64()) (crates/presk-rt/src/lib.rs:868-876, the call at
 * crates/presk-kernel/src/host.rs:793-829).  A buffer of the kernel's own type
 * is lent, its bits as they are; otherwise every element is widened to f64
 * exactly and stored as `to` stores an f64: f32 rounds once, bf16 rounds to
 * f32 and then to bf16 (two roundings), binary16 and e8m15 round once from
 * the f64.  The guard: storing a finite value at or past binary16's or
 * e8m15's overflow threshold (presk_rt::codes::overflows).
 *
 * Type numbers: 0 f64, 1 f32, 2 bf16, 4 f16, 5 e8m15 (i64 is 3, never
 * converted).  Pinned by tests/test_oracle_convert.py against the reference's
 * own presk_convert (crates/presk-export-c/c/presk_rt.c, built into
 * oracle/_ref by oracle/Makefile) on every pair and the special values.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "codes.h"

static size_t width(int t)
{
    switch (t) {
    case 0: return 8;
    case 1: return 4;
    case 2: case 4: return 2;
    case 5: return 3;
    }
    return 0;
}

static double load_f64(const void *src, int from, size_t i)
{
    const unsigned char *p = (const unsigned char *)src;
    switch (from) {
    case 0: { double x; memcpy(&x, p + 8 * i, 8); return x; }
    case 1: { float x; memcpy(&x, p + 4 * i, 4); return (double)x; }
    case 2: { uint16_t c; memcpy(&c, p + 2 * i, 2); return (double)oc_bf16_to_f32(c); }
    case 4: { uint16_t c; memcpy(&c, p + 2 * i, 2); return (double)oc_f16_to_f32(c); }
    case 5: {
        uint32_t c = (uint32_t)p[3 * i] | ((uint32_t)p[3 * i + 1] << 8) | ((uint32_t)p[3 * i + 2] << 16);
        return (double)oc_e8m15_to_f32(c);
    }
    }
    return 0.0;
}

static void store_f64(void *dst, int to, size_t i, double x)
{
    unsigned char *p = (unsigned char *)dst;
    switch (to) {
    case 0: memcpy(p + 8 * i, &x, 8); return;
    case 1: { float f = (float)x; memcpy(p + 4 * i, &f, 4); return; }
    case 2: { uint16_t c = oc_f32_to_bf16((float)x); memcpy(p + 2 * i, &c, 2); return; }
    case 4: { uint16_t c = oc_f64_to_f16(x); memcpy(p + 2 * i, &c, 2); return; }
    case 5: {
        uint32_t c = oc_f64_to_e8m15(x);
        p[3 * i] = (unsigned char)c;
        p[3 * i + 1] = (unsigned char)(c >> 8);
        p[3 * i + 2] = (unsigned char)(c >> 16);
        return;
    }
    }
}

/* n elements of type `from` at src stored as `to` at dst; returns the guard. */
uint32_t po_convert(void *dst, int to, const void *src, int from, size_t n)
{
    if (to == from) {
        memmove(dst, src, n * width(to));
        return 0;
    }
    uint32_t o = 0;
    for (size_t i = 0; i < n; i++) {
        const double x = load_f64(src, from, i);
        if (to == 4) o |= (uint32_t)oc_overflows_f16(x);
        if (to == 5) o |= (uint32_t)oc_overflows_e8m15(x);
        store_f64(dst, to, i, x);
    }
    return o;
}

/* ---- .psk.d leaves (crates/presk-data/src/lib.rs:205-219, Enc::decode) ----
 * A code of a float format given by its parameters is the f64 it denotes
 * (crates/presk-format/src/lib.rs:460-476, Float::decode): sign, exponent
 * field biased by 1 - emin, p - 1 trailing bits; the top field holds the
 * infinities and NaNs (IEEE) or only the NaN of the top trailing code (NaN
 * only); field 0 the subnormals or, without them, zero.  exp2 is exact
 * (lib.rs:170-176).  Pinned by tests/test_oracle_pskd.py: binary16 against
 * numpy over every code, the reference's own E4M3 codes of 480, -0.375, 2^-9
 * and -0 (crates/presk-data/tests/data.rs:235-236), E2M1's eight magnitudes
 * from its definition, bf16 and f32 against their bit layouts. */
static double po_exp2i(int k)
{
    uint64_t b = k >= -1022 ? (uint64_t)(k + 1023) << 52 : 1ull << (k + 1074);
    double x;
    memcpy(&x, &b, 8);
    return x;
}

double po_format_decode(uint64_t code, int p, int emin, int emax, int subnormals, int specials)
{
    const int t = p - 1;
    const uint64_t ncodes = (uint64_t)(emax - emin + 2) + (specials == 0 ? 1 : 0);
    int ebits = 0;
    while ((1ull << ebits) < ncodes) ebits++;
    const int bits = 1 + ebits + t;
    const int negative = (int)((code >> (bits - 1)) & 1);
    const uint64_t top = (1ull << ebits) - 1, tmask = (1ull << t) - 1;
    const uint64_t field = (code >> t) & top, trailing = code & tmask;
    double v;
    uint64_t nan = 0x7ff8000000000000ull;
    if (specials == 0 && field == top) {
        if (trailing == 0) v = INFINITY;
        else memcpy(&v, &nan, 8);
    } else if (specials == 1 && field == top && trailing == tmask) {
        memcpy(&v, &nan, 8);
    } else if (field == 0) {
        v = subnormals ? (double)trailing * po_exp2i(emin - t) : 0.0;
    } else {
        v = (double)((1ull << t) | trailing) * po_exp2i((int)field - (1 - emin) - t);
    }
    if (negative) {
        uint64_t b;
        memcpy(&b, &v, 8);
        b ^= 0x8000000000000000ull;
        memcpy(&v, &b, 8);
    }
    return v;
}

/* n elements of a real leaf: enc 0 f64, 1 f32, 2 bf16 (the conversion from
 * that type), 3 codes of `width` bytes of the format (p, emin, emax,
 * subnormals, specials); stored as `to` stores an f64.  Returns the guard. */
uint32_t po_pskd_decode(void *dst, int to, const void *src, int enc, int width, int p, int emin, int emax,
                        int subnormals, int specials, size_t n)
{
    if (enc != 3) return po_convert(dst, to, src, enc, n);
    const unsigned char *b = (const unsigned char *)src;
    uint32_t o = 0;
    for (size_t i = 0; i < n; i++) {
        uint64_t code = 0;
        for (int k = 0; k < width; k++) code |= (uint64_t)b[i * width + k] << (8 * k);
        const double x = po_format_decode(code, p, emin, emax, subnormals, specials);
        if (to == 4) o |= (uint32_t)oc_overflows_f16(x);
        if (to == 5) o |= (uint32_t)oc_overflows_e8m15(x);
        store_f64(dst, to, i, x);
    }
    return o;
}

/* n elements of an idx leaf of `width` bytes, little-endian, as i64 */
void po_pskd_idx(int64_t *dst, const void *src, int width, size_t n)
{
    const unsigned char *b = (const unsigned char *)src;
    for (size_t i = 0; i < n; i++) {
        uint64_t v = 0;
        for (int k = 0; k < width; k++) v |= (uint64_t)b[i * width + k] << (8 * k);
        dst[i] = (int64_t)v;
    }
}
