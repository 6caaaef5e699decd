/* oracle/digest.c -- TEST INFRASTRUCTURE ONLY (the parity oracle).
 *
 * Digests of a scalar function over its whole domain (every f32, every code)
 * or over a fixed sample, so that two implementations can be compared without
 * storing 2^32 outputs.  Built twice by oracle/Makefile:
 *   -DIMPL_ORACLE  the oracle's restatement (oracle/libm.c, oracle/codes.h)
 *                  -> oracle/liboracle.so
 *   -DIMPL_REF     the reference's own C runtime (presk_rt.h, presk_libm.c
 *                  from crates/presk-export-c/c) -> oracle/_ref/libpresk_ref.so
 * The GPU side computes the same digest with the product's device functions
 * (presk_amd/csrc/selftest.hip), and tests/golden/digests.json holds the
 * reference's values.
 *
 * digest = sum over inputs i of mix64((i << 32) | out_i)  (mod 2^64)
 * where mix64 is the splitmix64 finalizer (a bijection of u64): an order-free
 * sum, so that any partition of the domain gives the same value.
 */
#include <stdint.h>
#include <string.h>
#include <stddef.h>

#if defined(IMPL_REF)
#include "presk_rt.h"
#define F_EXP presk_expf
#define F_LOG presk_logf
#define F_TANH presk_tanhf
#define F_ERF presk_erff
#define F_SIN presk_sinf
#define F_COS presk_cosf
#define D_EXP presk_exp
#define D_LOG presk_log
#define D_TANH presk_tanh
#define D_ERF presk_erf
#define D_SIN presk_sin
#define D_COS presk_cos
static inline uint16_t C_BF16(float x) { return presk_f32_to_bf16(x); }
static inline uint16_t C_F16(float x) { return presk_f32_to_f16(x); }
static inline uint32_t C_E8(float x) { return presk_f32_to_e8m15_code(x); }
static inline float W_BF16(uint16_t c) { return presk_bf16_to_f32(c); }
static inline float W_F16(uint16_t c) { return presk_f16_to_f32(c); }
static inline float W_E8(uint32_t c) { return presk_e8m15_code_to_f32(c); }
static inline uint16_t D_F16(double x) { return presk_f64_to_f16(x); }
static inline uint32_t D_E8(double x) { return presk_e8m15_code(presk_f64_to_e8m15(x)); }
static inline uint32_t O_F16(float x) { return presk_overflows(x, 0x477ff000u); }
static inline uint32_t O_E8(float x) { return presk_overflows(x, 0x7f7fff80u); }
#else
#include "codes.h"
float ok_expf(float);
float ok_logf(float);
float ok_tanhf(float);
float ok_erff(float);
float ok_sinf(float);
float ok_cosf(float);
double ok_exp(double);
double ok_log(double);
double ok_tanh(double);
double ok_erf(double);
double ok_sin(double);
double ok_cos(double);
#define D_EXP ok_exp
#define D_LOG ok_log
#define D_TANH ok_tanh
#define D_ERF ok_erf
#define D_SIN ok_sin
#define D_COS ok_cos
#define F_SIN ok_sinf
#define F_COS ok_cosf
#define F_EXP ok_expf
#define F_LOG ok_logf
#define F_TANH ok_tanhf
#define F_ERF ok_erff
static inline uint16_t C_BF16(float x) { return oc_f32_to_bf16(x); }
static inline uint16_t C_F16(float x) { return oc_f32_to_f16(x); }
static inline uint32_t C_E8(float x) { return oc_f32_to_e8m15(x); }
static inline float W_BF16(uint16_t c) { return oc_bf16_to_f32(c); }
static inline float W_F16(uint16_t c) { return oc_f16_to_f32(c); }
static inline float W_E8(uint32_t c) { return oc_e8m15_to_f32(c); }
static inline uint16_t D_F16(double x) { return oc_f64_to_f16(x); }
static inline uint32_t D_E8(double x) { return oc_f64_to_e8m15(x); }
static inline uint32_t O_F16(float x) { return (uint32_t)oc_overflows_f16((double)x); }
static inline uint32_t O_E8(float x) { return (uint32_t)oc_overflows_e8m15((double)x); }
#endif

static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static inline float f_of(uint32_t b) { float x; memcpy(&x, &b, 4); return x; }
static inline uint32_t b_of(float x) { uint32_t b; memcpy(&b, &x, 4); return b; }

/* The f64 sample for the narrowings from f64: sample i.  Three in four have an
 * exponent within [-40, 24] so that the f16/e8m15 roundings, subnormals and
 * overflows are all reached; one in four is any f64 bit pattern. */
uint64_t pd_sample_f64_bits(uint64_t i)
{
    uint64_t r = mix64(i * 0x9e3779b97f4a7c15ull + 0x632be59bd9b4e019ull);
    if ((i & 3) == 3)
        return r;
    uint64_t e = 1023 - 40 + (r >> 52) % 65;          /* biased exponent */
    uint64_t frac = r & ((1ull << 52) - 1);
    if ((i & 3) == 2)                                    /* a narrow code's tie region */
        frac &= ~((1ull << 28) - 1) | (r >> 40 & 1);
    return (r & (1ull << 63)) | (e << 52) | frac;
}

/* The argument sample of f64 function fn (40 + 0..5), sample i: one in
 * eight any bit pattern (NaNs, infinities, subnormals, zeros), one in eight
 * any exponent, the rest exponents in [-30, 12] (|x| from 1e-9 to 8192,
 * where the reductions' branches lie), mantissa and sign uniform. */
uint64_t pd_sample_f64_arg(int fn, uint64_t i)
{
    const uint64_t r = mix64(i * 0x9e3779b97f4a7c15ull + 0x2545f4914f6cdd1dull * (uint64_t)(fn + 1));
    const uint64_t cls = i & 7;
    if (cls == 0)
        return r;
    const uint64_t m = mix64(r);
    const uint64_t e = cls == 1 ? m % 2047 : 1023 - 30 + m % 43;
    return (r & (1ull << 63)) | (e << 52) | (r & ((1ull << 52) - 1));
}

static inline double d_of(uint64_t b) { double x; memcpy(&x, &b, 8); return x; }
static inline uint64_t bd_of(double x) { uint64_t b; memcpy(&b, &x, 8); return b; }

/* an f64 function's value at x */
static inline double evald(int fn, double x, int *ok)
{
    *ok = 1;
    switch (fn) {
    case 40: return D_EXP(x);
    case 41: return D_LOG(x);
    case 42: return D_TANH(x);
    case 43: return D_ERF(x);
    case 44: return D_SIN(x);
    case 45: return D_COS(x);
    default: *ok = 0; return 0;
    }
}

/* Function ids: 0 expf, 1 logf, 2 tanhf, 3 erff, 4 sinf, 5 cosf (every f32);
 * 10 f32->bf16, 11 f32->f16, 12 f32->e8m15, 32 f16 guard, 33 e8m15 guard
 * (every f32); 20 bf16->f32, 21 f16->f32 (every code of 16 bits),
 * 22 e8m15->f32 (every 24-bit code); 30 f64->f16, 31 f64->e8m15 (the sample);
 * 40 exp, 41 log, 42 tanh, 43 erf, 44 sin, 45 cos of f64 (their argument
 * sample; the result's 64 bits folded to 32 by the top half of mix64). */
static inline uint32_t eval1(int fn, uint64_t i, int *ok)
{
    *ok = 1;
    switch (fn) {
    case 0: return b_of(F_EXP(f_of((uint32_t)i)));
    case 1: return b_of(F_LOG(f_of((uint32_t)i)));
    case 2: return b_of(F_TANH(f_of((uint32_t)i)));
    case 3: return b_of(F_ERF(f_of((uint32_t)i)));
    case 4: return b_of(F_SIN(f_of((uint32_t)i)));
    case 5: return b_of(F_COS(f_of((uint32_t)i)));
    case 10: return C_BF16(f_of((uint32_t)i));
    case 11: return C_F16(f_of((uint32_t)i));
    case 12: return C_E8(f_of((uint32_t)i));
    case 20: return b_of(W_BF16((uint16_t)i));
    case 21: return b_of(W_F16((uint16_t)i));
    case 22: return b_of(W_E8((uint32_t)i));
    case 30: { uint64_t b = pd_sample_f64_bits(i); double x; memcpy(&x, &b, 8); return D_F16(x); }
    case 31: { uint64_t b = pd_sample_f64_bits(i); double x; memcpy(&x, &b, 8); return D_E8(x); }
    case 32: return O_F16(f_of((uint32_t)i));
    case 33: return O_E8(f_of((uint32_t)i));
    case 40: case 41: case 42: case 43: case 44: case 45:
        return (uint32_t)(mix64(bd_of(evald(fn, d_of(pd_sample_f64_arg(fn, i)), ok))) >> 32);
    default: *ok = 0; return 0;
    }
}

uint64_t pd_digest(int fn, uint64_t lo, uint64_t hi)
{
    uint64_t acc = 0;
    int bad = 0;
    #pragma omp parallel for reduction(+:acc) reduction(|:bad) schedule(static)
    for (int64_t i = (int64_t)lo; i < (int64_t)hi; i++) {
        int ok;
        uint32_t o = eval1(fn, (uint64_t)i, &ok);
        bad |= !ok;
        acc += mix64(((uint64_t)i << 32) | o);
    }
    return bad ? 0 : acc;
}

/* The outputs at given inputs (for sample vectors and for reporting which
 * inputs differ). */
int pd_eval(int fn, const uint64_t *in, uint32_t *out, size_t n)
{
    for (size_t k = 0; k < n; k++) {
        int ok;
        out[k] = eval1(fn, in[k], &ok);
        if (!ok)
            return -1;
    }
    return 0;
}

/* An f64 function at given arguments, the results' bits. */
int pd_eval_f64(int fn, const double *in, uint64_t *out, size_t n)
{
    for (size_t k = 0; k < n; k++) {
        int ok;
        out[k] = bd_of(evald(fn, in[k], &ok));
        if (!ok)
            return -1;
    }
    return 0;
}
