"""numpy encoders/decoders of the storage formats for test inputs and expected
values (IEEE rounding via numpy for f16; the top-bits rounding for bf16 and
e8m15, crates/presk-rt/src/lib.rs:228-241, crates/presk-rt/src/codes.rs:89-110).
NaN payloads are not needed by these helpers' callers."""
import numpy as np


def encode(x, ty):
    """float32 values -> storage array of type `ty`."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if ty == "f32":
        return x.ravel().copy()
    if ty == "f64":
        return x.astype(np.float64).ravel()
    b = x.view(np.uint32).astype(np.uint64).ravel()
    if ty == "bf16":
        return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    if ty == "f16":
        with np.errstate(over="ignore"):
            return x.astype(np.float16).view(np.uint16).ravel()
    if ty == "e8m15":
        c = ((b + 0x7F + ((b >> 8) & 1)) >> 8).astype(np.uint32)
        out = np.empty(c.size * 3, dtype=np.uint8)
        out[0::3], out[1::3], out[2::3] = c & 0xFF, (c >> 8) & 0xFF, (c >> 16) & 0xFF
        return out
    raise ValueError(ty)


def decode(a, ty):
    """storage array -> float32 values (float64 for f64)."""
    if ty in ("f32", "f64"):
        return a
    if ty == "bf16":
        return (a.astype(np.uint32) << 16).view(np.float32)
    if ty == "f16":
        return a.view(np.float16).astype(np.float32)
    if ty == "e8m15":
        c = a[0::3].astype(np.uint32) | (a[1::3].astype(np.uint32) << 8) | (a[2::3].astype(np.uint32) << 16)
        return (c << 8).view(np.float32)
    raise ValueError(ty)


def roundtrip(x, ty):
    """float32 values rounded to `ty` and widened back."""
    return decode(encode(x, ty), ty).reshape(np.shape(x))
