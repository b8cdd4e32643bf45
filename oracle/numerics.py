"""Bit-level number formats used by the oracle (test infrastructure only).

bfloat16 values are carried as float32 arrays whose low 16 bits are zero;
float16 values as float32 arrays holding exactly representable values.
float8_e4m3fn values are carried as uint8 codes.
"""

from __future__ import annotations

import numpy as np

BF16_NAN_BITS = np.uint16(0x7FC0)
E4M3_MAX = 448.0


def f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32)


def bf16_round(a) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32.

    Same rule as c10::BFloat16's round_to_nearest_even: add 0x7FFF plus the
    lowest kept bit, truncate. NaN maps to a quiet NaN.
    """
    a = f32(a)
    bits = a.view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    out = ((bits + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    out = np.where(np.isnan(a), np.float32(np.nan), out)
    return out.astype(np.float32)


def f16_round(a) -> np.ndarray:
    """float32 -> nearest IEEE binary16 (ties to even, subnormals kept,
    overflow to infinity), returned as float32: numpy's float32 -> float16
    conversion, the textbook correctly rounded one. NaN stays NaN."""
    a = f32(a)
    with np.errstate(over="ignore", invalid="ignore"):
        return a.astype(np.float16).astype(np.float32)


def f16_from_bits(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def bf16_bits(a) -> np.ndarray:
    """float32 holding bf16 values -> uint16 bit patterns (exact, no rounding)."""
    a = f32(a)
    return (a.view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits) -> np.ndarray:
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def e4m3_encode(a) -> np.ndarray:
    """float32 -> float8_e4m3fn code with round-to-nearest-even.

    e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits, no infinities, one
    NaN code per sign (0x7F / 0xFF), max finite 448, smallest subnormal 2^-9.
    A value whose rounded magnitude exceeds 448 (|v| > 464, infinities) and NaN
    become the NaN code with the input's sign bit, as torch's conversion does.
    Derived from the format definition, not from any library's bit tricks.
    """
    a = f32(a)
    sign = ((a.view(np.uint32) >> 24) & 0x80).astype(np.uint8)
    finite = np.isfinite(a)
    with np.errstate(invalid="ignore"):
        mag = np.where(finite, np.abs(a.astype(np.float64)), 0.0)

    sub = finite & (mag < 2.0 ** -6)
    # Subnormal range: quantum 2^-9; np.rint rounds half to even. A result of 8
    # is the smallest normal (code 0x08), which is consistent with the layout.
    code = np.rint(np.where(sub, mag, 0.0) * 512.0).astype(np.int64)

    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        e = np.floor(np.log2(np.where(sub, 1.0, mag + np.where(finite, 0.0, 1.0))))
        # Guard against log2 rounding at exact powers of two.
        m = np.where(sub | ~finite, 1.0, mag / np.exp2(e))
        fix_lo = m < 1.0
        e = np.where(fix_lo, e - 1, e)
        m = np.where(fix_lo, m * 2.0, m)
        fix_hi = m >= 2.0
        e = np.where(fix_hi, e + 1, e)
        m = np.where(fix_hi, m / 2.0, m)
        q = np.rint(m * 8.0)  # 8..16, ties to even on the 3-bit mantissa
        carry = q >= 16.0
        e = np.where(carry, e + 1, e)
        q = np.where(carry, 8.0, q)
        ecode = (e + 7).astype(np.int64)
        ncode = (ecode << 3) | (q.astype(np.int64) - 8)
    code = np.where(sub, code, ncode)
    overflow = (~sub) & ((ecode > 15) | (ncode >= 0x7F))
    nan = np.isnan(a) | np.isinf(a) | overflow
    code = np.where(nan, 0x7F, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def e4m3_decode(codes) -> np.ndarray:
    """float8_e4m3fn code -> float32 (exact)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7))
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return (sign * val).astype(np.float32)


def round_to(v, dt: str) -> np.ndarray:
    """float32 values rounded to dtype `dt` ('bf16', 'f16' or 'f32')."""
    if dt == "bf16":
        return bf16_round(v)
    if dt == "f16":
        return f16_round(v)
    return f32(v)


class T:
    """A tensor value as torch would hold it: float32 data plus a dtype tag.

    dtype is 'bf16', 'f16' or 'f32'. `dim0` marks a 0-dim tensor, which does
    not take part in dtype promotion against dimensioned tensors of the same
    category (torch's rule: bf16_tensor * f32_0dim -> bf16).
    """

    __slots__ = ("v", "dt", "dim0")

    def __init__(self, v, dt: str, dim0: bool = False):
        assert dt in ("bf16", "f16", "f32")
        self.v = f32(v)
        self.dt = dt
        self.dim0 = dim0

    def to(self, dt: str) -> "T":
        if dt == self.dt:
            return self
        return T(round_to(self.v, dt), dt, self.dim0)


def _promote(a: T, b: T) -> str:
    if a.dim0 and not b.dim0:
        return b.dt
    if b.dim0 and not a.dim0:
        return a.dt
    if a.dt == b.dt:
        return a.dt
    return "f32"  # f32 with anything, and bf16 with f16 (torch.promote_types)


def _finish(v: np.ndarray, dt: str, dim0: bool) -> T:
    return T(round_to(f32(v), dt), dt, dim0)


def add(a: T, b: T) -> T:
    return _finish(a.v + b.v, _promote(a, b), a.dim0 and b.dim0)


def sub(a: T, b: T) -> T:
    return _finish(a.v - b.v, _promote(a, b), a.dim0 and b.dim0)


def mul(a: T, b: T) -> T:
    return _finish(a.v * b.v, _promote(a, b), a.dim0 and b.dim0)


def add_scalar(a: T, s: float) -> T:
    """`s + a` with a Python scalar: the result keeps a's dtype."""
    return _finish(np.float32(s) + a.v, a.dt, a.dim0)


def clamp(a: T, lo: float, hi: float) -> T:
    v = np.minimum(np.maximum(a.v, np.float32(lo)), np.float32(hi))
    v = np.where(np.isnan(a.v), a.v, v)
    return T(v, a.dt, a.dim0)
