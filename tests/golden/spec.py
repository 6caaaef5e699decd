"""The functions, domains and blocks of tests/golden/digests.json (shared by
the fixture writer and the tests)."""

# name -> (function id of oracle/digest.c and the device self-test, domain size)
FUNCTIONS = {
    "expf": (0, 1 << 32),
    "logf": (1, 1 << 32),
    "tanhf": (2, 1 << 32),
    "erff": (3, 1 << 32),
    "sinf": (4, 1 << 32),
    "cosf": (5, 1 << 32),
    "f32_to_bf16": (10, 1 << 32),
    "f32_to_f16": (11, 1 << 32),
    "f32_to_e8m15": (12, 1 << 32),
    "bf16_to_f32": (20, 1 << 16),
    "f16_to_f32": (21, 1 << 16),
    "e8m15_to_f32": (22, 1 << 24),
    "f64_to_f16": (30, 1 << 26),
    "f64_to_e8m15": (31, 1 << 26),
    "guard_f16": (32, 1 << 32),
    "guard_e8m15": (33, 1 << 32),
}


def blocks(domain):
    """256 equal blocks of a domain of 2^32 inputs, else one block."""
    if domain == 1 << 32:
        step = domain // 256
        return [(i * step, (i + 1) * step) for i in range(256)]
    return [(0, domain)]


def sample_inputs(domain, n=512):
    """Fixed sample inputs: special values and a spread of the domain."""
    if domain == 1 << 32:
        special = [0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x7F800001, 1, 0x807FFFFF,
                   0x3F800000, 0xBF800000, 0x477FEFFF, 0x477FF000, 0x47800000, 0x7F7FFF7F, 0x7F7FFF80, 0x42B17218,
                   0xC2CFF1B5, 0x3F580000, 0x40C00000, 0x3EB17218, 0x33000000, 0x38800000, 0x387FFFFF]
    else:
        special = [0, 1, domain - 1, domain // 2, domain // 2 - 1]
    ins = list(dict.fromkeys(x % domain for x in special))
    k = 0
    while len(ins) < n:
        k += 1
        ins.append((k * 0x9E3779B97F4A7C15 >> 17) % domain)
    return ins[:n]


# f64 functions (the interpreter's f64 arm): name -> function id of
# oracle/digest.c and the device self-test, each over its argument sample
# (pd_sample_f64_arg) of F64_DOMAIN inputs in 16 blocks
F64 = {"exp": 40, "log": 41, "tanh": 42, "erf": 43, "sin": 44, "cos": 45}
F64_DOMAIN = 1 << 24


def f64_blocks():
    step = F64_DOMAIN // 16
    return [(i * step, (i + 1) * step) for i in range(16)]


def f64_specials():
    """Arguments at the f64 functions' branch points, overflow and underflow
    thresholds, reduction boundaries and near multiples of pi/2, their
    negatives and next doubles up."""
    import math
    import numpy as np
    base = [0.0, 1.0, 5e-324, 1e-320, 2.2250738585072014e-308, 1e-300, 2.0 ** -54, 2.0 ** -28, 3.0e-10, 0.25541281188299536,
            0.5493061443340549, 0.84375, 1.25, 1 / 0.35, 6.0, 20.0, 28.0, 0.5 * math.log(2), 1.5 * math.log(2),
            56 * math.log(2), 708.3964185322641, 709.782712893383973096, 709.7827128933841, 745.1332191019411,
            745.1332191019412, 0.7853981633974483, math.pi / 2, math.pi, 3 * math.pi / 2, 2 * math.pi, 5 * math.pi / 4,
            9 * math.pi / 4, 2 ** 20 * math.pi / 2, 1e22, 1e300, 2.0 ** 1023, 1.7976931348623157e308, math.inf, math.nan]
    out = base + [-x for x in base]
    with np.errstate(over="ignore"):
        out += [float(np.nextafter(x, math.inf)) for x in base if math.isfinite(x)]
    return out
