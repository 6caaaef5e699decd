/* oracle/rng.c -- TEST INFRASTRUCTURE ONLY (the parity oracle).
 *
 * Presk's keys and their draws, restated: the generator is rand_chacha
 * 0.9's ChaCha20Rng (crates/presk-interp/src/key.rs:1-60, a dependency
 * absent from /root/reference; its C twin is
 * crates/presk-export-c/c/presk_rt.c:767-930): Bernstein's ChaCha20 with
 * twenty rounds, state words 0-3 the constant "expand 32-byte k", 4-11 the
 * key (32 bytes as little-endian words), 12-13 a 64-bit block counter from 0,
 * 14-15 a 64-bit stream number 0; the output read a word at a time in block
 * order, a u64 as two words, the low one first.  From it:
 *   po_word(key, w)        word w of the stream (block w / 16, word w % 16)
 *   po_uniform01_at(key,e) uniform01's e-th draw: (u64 e >> 11) / 2^53
 *                          (key.rs:53-55), u64 e = words 2e, 2e + 1
 *   po_key_split(k, l)     key l of split(n): stream bytes 32l..32l+31
 *                          (key.rs:19-29)
 *   po_key_child(k, t)     split 0 of the key whose first 8 bytes are k's
 *                          xor t, little-endian (key.rs:33-42)
 *   po_key_from_seed(s)    the first 32 stream bytes of seed_from_u64(s):
 *                          rand_core's PCG32 fill of the seed (key.rs:12-17)
 *   po_dropout_mask(...)   the training mask of n elements: element e is
 *                          1/(1-rate) where uniform e < 1-rate, else 0, in
 *                          the site's type as crates/presk-kernel/src/
 *                          host.rs:1893-1926 rounds it (f32: the f64 value
 *                          as f32; bf16: that f32 rounded to bf16; f16 and
 *                          e8m15: the f64 narrowed once, Buf::of).
 * Pinned by tests/test_oracle_rng.py: against the reference's own golden
 * normals of Key::from_seed(0) (key.rs:85-93, with the reference's f64 log
 * and cos from oracle/_ref) and against oracle/_ref's presk_rt.c.
 */
#include <stdint.h>
#include <string.h>

#include "codes.h"

static uint32_t rotl(uint32_t x, int n) { return (x << n) | (x >> (32 - n)); }

#define QR(a, b, c, d)                    \
    a += b; d ^= a; d = rotl(d, 16);      \
    c += d; b ^= c; b = rotl(b, 12);      \
    a += b; d ^= a; d = rotl(d, 8);       \
    c += d; b ^= c; b = rotl(b, 7);

static void block(const uint8_t key[32], uint64_t counter, uint32_t out[16])
{
    uint32_t s[16], x[16];
    s[0] = 0x61707865u; s[1] = 0x3320646eu; s[2] = 0x79622d32u; s[3] = 0x6b206574u;
    for (int i = 0; i < 8; ++i)
        s[4 + i] = (uint32_t)key[4 * i] | ((uint32_t)key[4 * i + 1] << 8) | ((uint32_t)key[4 * i + 2] << 16) |
                   ((uint32_t)key[4 * i + 3] << 24);
    s[12] = (uint32_t)counter;
    s[13] = (uint32_t)(counter >> 32);
    s[14] = 0;
    s[15] = 0;
    memcpy(x, s, sizeof x);
    for (int r = 0; r < 10; ++r) {
        QR(x[0], x[4], x[8], x[12]);
        QR(x[1], x[5], x[9], x[13]);
        QR(x[2], x[6], x[10], x[14]);
        QR(x[3], x[7], x[11], x[15]);
        QR(x[0], x[5], x[10], x[15]);
        QR(x[1], x[6], x[11], x[12]);
        QR(x[2], x[7], x[8], x[13]);
        QR(x[3], x[4], x[9], x[14]);
    }
    for (int i = 0; i < 16; ++i) out[i] = x[i] + s[i];
}

uint32_t po_word(const uint8_t key[32], uint64_t w)
{
    uint32_t b[16];
    block(key, w / 16, b);
    return b[w % 16];
}

static uint64_t u64_at(const uint8_t key[32], uint64_t e)
{
    uint32_t b[16];
    block(key, (2 * e) / 16, b);
    const unsigned i = (unsigned)((2 * e) % 16);
    return (uint64_t)b[i] | ((uint64_t)b[i + 1] << 32);
}

double po_uniform01_at(const uint8_t key[32], uint64_t e)
{
    return (double)(u64_at(key, e) >> 11) / 9007199254740992.0;
}

/* n stream bytes from word w0 on, each word little-endian */
static void stream_bytes(const uint8_t key[32], uint64_t w0, uint8_t *out, unsigned n)
{
    for (unsigned i = 0; i < n; i += 4) {
        const uint32_t w = po_word(key, w0 + i / 4);
        for (unsigned j = 0; j < 4 && i + j < n; ++j) out[i + j] = (uint8_t)(w >> (8 * j));
    }
}

void po_key_split(const uint8_t key[32], uint64_t l, uint8_t out[32]) { stream_bytes(key, 8 * l, out, 32); }

void po_key_child(const uint8_t key[32], uint64_t t, uint8_t out[32])
{
    uint8_t seed[32];
    memcpy(seed, key, 32);
    for (int i = 0; i < 8; ++i) seed[i] ^= (uint8_t)(t >> (8 * i));
    stream_bytes(seed, 0, out, 32);
}

void po_key_from_seed(uint64_t state, uint8_t out[32])
{
    /* rand_core's seed_from_u64: PCG32 (multiplier 6364136223846793005,
       increment 11634580027462260723), XSH RR output, 8 words LE */
    uint8_t seed[32];
    const uint64_t mul = 6364136223846793005ull, inc = 11634580027462260723ull;
    for (int i = 0; i < 8; ++i) {
        state = state * mul + inc;
        const uint64_t x = state;
        const uint32_t xs = (uint32_t)(((x >> 18) ^ x) >> 27);
        const unsigned rot = (unsigned)(x >> 59);
        const uint32_t v = (xs >> rot) | (xs << ((32 - rot) & 31));
        for (int j = 0; j < 4; ++j) seed[4 * i + j] = (uint8_t)(v >> (8 * j));
    }
    stream_bytes(seed, 0, out, 32);
}

/* dtype codes as po_convert's: 0 f64, 1 f32, 2 bf16, 4 f16, 5 e8m15 */
void po_dropout_mask(const uint8_t key[32], double rate, int dtype, uint64_t n, void *out)
{
    const double keep = 1.0 - rate, scale = 1.0 / (1.0 - rate);
    for (uint64_t e = 0; e < n; ++e) {
        const double v = po_uniform01_at(key, e) < keep ? scale : 0.0;
        switch (dtype) {
        case 0: ((double *)out)[e] = v; break;
        case 1: ((float *)out)[e] = (float)v; break;
        case 2: ((uint16_t *)out)[e] = oc_f32_to_bf16((float)v); break;
        case 4: ((uint16_t *)out)[e] = oc_f64_to_f16(v); break;
        case 5: {
            const uint32_t c = oc_f64_to_e8m15(v);
            uint8_t *p = (uint8_t *)out + 3 * e;
            p[0] = (uint8_t)c; p[1] = (uint8_t)(c >> 8); p[2] = (uint8_t)(c >> 16);
            break;
        }
        }
    }
}
