"""Inputs for the edge-conversion parity tests: for each source type, the
special values (zeros, subnormals, the largest finite numbers, the
infinities, NaNs with payloads, the rounding ties and the overflow
thresholds of every target) and a seeded random set, as storage bytes."""
import numpy as np

TYPES = {"f64": 0, "f32": 1, "bf16": 2, "f16": 4, "e8m15": 5}
WIDTH = {"f64": 8, "f32": 4, "bf16": 2, "f16": 2, "e8m15": 3}


def _doubles(rng, n):
    ties = []
    for m in (1.0, 1.5, 1024.0, 2.0 ** -14, 2.0 ** -24, 2.0 ** -126, 2.0 ** -133, 65504.0, 3.0e38):
        for t in (-53, -25, -24, -12, -11, -9, -8, -16, -17):
            ties += [m * (1 + 2.0 ** t), m * (1 + 3 * 2.0 ** t), m * (1 - 2.0 ** t)]
    special = [0.0, -0.0, 5e-324, -5e-324, 2.2250738585072014e-308, 1.7976931348623157e308, -1.7976931348623157e308,
               np.inf, -np.inf, np.nan, 65504.0, 65519.99, 65520.0, 65520.0000001, -65520.0, 65535.9,
               3.4028234663852886e38, 3.4028235677973366e38, 3.4028236e38, 3.3895313892515355e38, 3.3895314e38,
               1.401298464324817e-45, 7e-46, 5.960464477539063e-08, 2.9802322387695312e-08, 2.98023224e-08, 1e-40]
    vals = np.array(special + ties + [-x for x in ties], np.float64)
    bits = vals.view(np.uint64).copy()
    nan_bits = np.array([0x7ff8000000000001, 0x7ff0000000000001, 0xfff4000000000000, 0x7ffffffffffffff0, 0x7ff0000020000000], np.uint64)
    rnd = (rng.standard_normal(n) * np.exp2(rng.integers(-150, 130, n))).view(np.uint64)
    rbits = rng.integers(0, 2 ** 63, n, dtype=np.uint64) | (rng.integers(0, 2, n, dtype=np.uint64) << np.uint64(63))
    return np.concatenate([bits, nan_bits, rnd, rbits]).view(np.uint8)


def _floats(rng, n):
    special = np.array([0, 0x80000000, 1, 0x80000001, 0x007fffff, 0x00800000, 0x7f7fffff, 0xff7fffff, 0x7f800000, 0xff800000,
                        0x7fc00000, 0x7f800001, 0x7fa00001, 0xffc00123, 0x477fe000, 0x477ff000, 0x477fefff, 0x7f7fff80,
                        0x7f7fff7f, 0x33800000, 0x33000000, 0x33000001, 0x387fc000, 0x38800000, 0x3f808000, 0x3f818000],
                       np.uint32)
    rnd = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([special, rnd]).view(np.uint8)


def source_bytes(ty: str, seed: int = 0, n: int = 200000):
    rng = np.random.default_rng(seed)
    if ty == "f64":
        return _doubles(rng, n)
    if ty == "f32":
        return _floats(rng, n)
    if ty in ("bf16", "f16"):
        return np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.uint8)
    # e8m15: every 24-bit code
    c = np.arange(1 << 24, dtype=np.uint32)
    return np.stack([c & 0xff, (c >> 8) & 0xff, c >> 16], axis=1).astype(np.uint8).ravel()
