"""bf16 and OCP fp8 e4m3fn codecs in numpy (oracle; test infrastructure only).

bf16: the reference's default dtype is bfloat16 (nanovllm/engine/model_runner.py:70-72),
so every tensor it stores is rounded to bf16 with IEEE round-to-nearest-even.

e4m3fn: the OCP 8-bit float used by gfx950 (1 sign, 4 exponent bits with bias 7,
3 mantissa bits, no infinities, a single NaN pattern S.1111.111, max finite 448,
smallest subnormal 2^-9). The reference has no fp8 path; this codec defines the
quantised variant's arithmetic (round-to-nearest-even, saturating to +-448).
"""
import numpy as np

__all__ = [
    "bf16_bits", "bf16_from_bits", "bf16_round", "bf16_ulp",
    "E4M3_MAX", "e4m3_decode", "e4m3_encode", "e4m3_values",
]


def bf16_bits(x):
    """float32 -> bf16 bit patterns (uint16), round-to-nearest-even; NaN -> 0x7fc0."""
    u = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    r[nan] = np.uint16(0x7FC0)
    return r


def bf16_from_bits(b):
    """bf16 bit patterns (uint16) -> float32 values."""
    b = np.ascontiguousarray(np.asarray(b, dtype=np.uint16))
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_round(x):
    """Round float32 values to the nearest bf16 value (returned as float32)."""
    return bf16_from_bits(bf16_bits(x))


def bf16_ulp(x):
    """Spacing of bf16 numbers at |x| (x already bf16-representable, finite)."""
    x = np.abs(np.asarray(x, dtype=np.float32))
    e = np.floor(np.log2(np.maximum(x, np.float32(2.0 ** -126))))
    return np.exp2(e - 7).astype(np.float32)


E4M3_MAX = 448.0


def _e4m3_table():
    vals = np.empty(256, dtype=np.float64)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            vals[c] = np.nan
        elif e == 0:
            vals[c] = s * (m / 8.0) * 2.0 ** -6
        else:
            vals[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


_E4M3 = _e4m3_table()
_E4M3_POS = _E4M3[:127]          # codes 0x00..0x7e: 0 .. 448, strictly increasing


def e4m3_values():
    """Decoded value of every e4m3fn code (float64, NaN at 0x7f/0xff)."""
    return _E4M3.copy()


def e4m3_decode(codes):
    """e4m3fn codes (uint8) -> float32 values."""
    return _E4M3[np.asarray(codes, dtype=np.uint8)].astype(np.float32)


def e4m3_encode(x):
    """float32 -> e4m3fn codes (uint8): round-to-nearest-even, saturate to +-448, NaN -> 0x7f."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64).ravel()
    lo = np.searchsorted(_E4M3_POS, a, side="right") - 1       # v[lo] <= a
    lo = np.clip(lo, 0, 126)
    hi = np.minimum(lo + 1, 126)
    dlo = a - _E4M3_POS[lo]
    dhi = _E4M3_POS[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (lo % 2 == 1))
    code = np.where(pick_hi & (hi != lo), hi, lo).astype(np.uint8)
    code = np.where(a >= E4M3_MAX, np.uint8(126), code)
    sign = (np.signbit(x.ravel())).astype(np.uint8) << 7
    out = (code | sign).astype(np.uint8)
    out[np.isnan(x.ravel())] = np.uint8(0x7F)
    return out.reshape(x.shape)
