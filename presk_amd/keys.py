"""Presk's keys on the host (crates/presk-interp/src/key.rs): 32 bytes each,
derived by rand_chacha 0.9's ChaCha20Rng -- Bernstein's ChaCha20, twenty
rounds, state words 0-3 the constant, 4-11 the key as little-endian words,
12-13 a 64-bit block counter from 0, 14-15 a 64-bit stream number 0, the
output bytes the words in order, each little-endian.  The host derives the
keys of a call's dropout sites from the step's key (split_key in the
program, `Key::child` per training step); the device draws the masks from
them (presk_hip_dropout_mask).  Keys are few and short, so plain Python."""
from __future__ import annotations

import struct

_M32 = 0xFFFFFFFF


def _rotl(x: int, n: int) -> int:
    return ((x << n) | (x >> (32 - n))) & _M32


def _block(key: bytes, counter: int) -> list:
    s = [0x61707865, 0x3320646E, 0x79622D32, 0x6B206574, *struct.unpack("<8I", key),
         counter & _M32, (counter >> 32) & _M32, 0, 0]
    x = list(s)

    def qr(a, b, c, d):
        x[a] = (x[a] + x[b]) & _M32; x[d] = _rotl(x[d] ^ x[a], 16)
        x[c] = (x[c] + x[d]) & _M32; x[b] = _rotl(x[b] ^ x[c], 12)
        x[a] = (x[a] + x[b]) & _M32; x[d] = _rotl(x[d] ^ x[a], 8)
        x[c] = (x[c] + x[d]) & _M32; x[b] = _rotl(x[b] ^ x[c], 7)

    for _ in range(10):
        qr(0, 4, 8, 12); qr(1, 5, 9, 13); qr(2, 6, 10, 14); qr(3, 7, 11, 15)
        qr(0, 5, 10, 15); qr(1, 6, 11, 12); qr(2, 7, 8, 13); qr(3, 4, 9, 14)
    return [(a + b) & _M32 for a, b in zip(x, s)]


def stream(key: bytes, nbytes: int, word0: int = 0) -> bytes:
    """nbytes of the key's keystream from word `word0` on."""
    out = bytearray()
    w = word0
    while len(out) < nbytes:
        blk = _block(key, w // 16)
        out += struct.pack("<I", blk[w % 16])
        w += 1
    return bytes(out[:nbytes])


def split(key: bytes, n: int) -> list:
    """`split_key`'s n keys (Key::split): consecutive 32-byte pieces of the stream."""
    return [stream(key, 32, 8 * l) for l in range(n)]


def child(key: bytes, t: int) -> bytes:
    """Key::child(t): split 0 of the key whose first eight bytes are xored with t."""
    seed = bytes(a ^ b for a, b in zip(key[:8], struct.pack("<Q", t & 0xFFFFFFFFFFFFFFFF))) + key[8:]
    return stream(seed, 32)


def seed_key(seed: int) -> bytes:
    """The key of rand_core's seed_from_u64 for ChaCha20Rng: eight PCG32
    outputs (XSH RR), each little-endian."""
    mul, inc = 6364136223846793005, 11634580027462260723
    state = seed & 0xFFFFFFFFFFFFFFFF
    words = []
    for _ in range(8):
        state = (state * mul + inc) & 0xFFFFFFFFFFFFFFFF
        xs = (((state >> 18) ^ state) >> 27) & _M32
        rot = state >> 59
        words.append(((xs >> rot) | (xs << ((32 - rot) & 31))) & _M32)
    return struct.pack("<8I", *words)


def from_seed(seed: int) -> bytes:
    """Key::from_seed: the first 32 stream bytes of seed_from_u64's generator."""
    return stream(seed_key(seed), 32)
