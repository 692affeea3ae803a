"""bfloat16 emulation on uint16 bit patterns (test infrastructure).

NumPy has no bfloat16.  A bfloat16 value is the upper 16 bits of a float32;
widening is exact, narrowing rounds to nearest even (RNE).

Pinned by: torch's CPU float32->bfloat16 conversion (an RNE library
routine) on random, tie and special values; exhaustive round-trip of all
65536 patterns; float64->bfloat16 against exact rational rounding
(``fractions.Fraction``) on random and tie values.
"""

from __future__ import annotations

import numpy as np


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bfloat16 bit patterns to float32."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    """RNE float32 -> bfloat16 bit patterns; NaN stays NaN (quieted, sign kept)."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    nan = (bits & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    rounded = ((bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    quiet = ((bits >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return np.where(nan, quiet, rounded)


def round_bf16(values: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16 (returned as float32)."""
    return bf16_to_f32(f32_to_bf16(values))


def f64_to_bf16(values: np.ndarray) -> np.ndarray:
    """Single correct rounding float64 -> bfloat16 (bit patterns).

    Normal bfloat16 results: integer round-to-nearest-even on the float64 bit
    pattern (drop 45 of the 52 fraction bits, re-bias the exponent; a carry
    out of the fraction bumps the exponent, overflow gives infinity).  Zero,
    subnormal results, NaN and infinities take the exact scalar path.
    """
    values = np.asarray(values, dtype=np.float64)
    flat = values.reshape(-1)
    bits = flat.view(np.uint64)
    sign = ((bits >> np.uint64(63)).astype(np.uint16) << np.uint16(15)).astype(np.uint16)
    exponent = ((bits >> np.uint64(52)) & np.uint64(0x7FF)).astype(np.int64) - 1023
    fraction = bits & np.uint64((1 << 52) - 1)
    normal = (exponent >= -126) & (exponent <= 127)
    rebased = np.where(normal, exponent + 127, 1).astype(np.uint64)
    full = (rebased << np.uint64(52)) | fraction
    rounded = (full + np.uint64((1 << 44) - 1) + ((full >> np.uint64(45)) & np.uint64(1))) >> np.uint64(45)
    rounded = np.minimum(rounded, np.uint64(0x7F80)).astype(np.uint16)
    out = (sign | rounded).astype(np.uint16)
    special = ~normal
    if special.any():
        for index in np.flatnonzero(special):
            out[index] = _f64_to_bf16_scalar(float(flat[index]), 0)
    return out.reshape(values.shape)


def f64_to_bf16_exact(value: float) -> int:
    """Reference scalar rounding used by the pins: exact walk over neighbours."""
    return _f64_to_bf16_scalar(float(value), 0)


def _bf16_value(bits: int) -> float:
    return float(np.array([bits << 16], dtype=np.uint32).view(np.float32)[0])


def _f64_to_bf16_scalar(value: float, guess: int) -> int:
    if value != value:
        return 0x7FC0 | (0x8000 if np.signbit(value) else 0)
    sign = 0x8000 if (value < 0 or (value == 0 and np.signbit(value))) else 0
    magnitude = abs(value)
    largest = _bf16_value(0x7F7F)
    # Values at or beyond the midpoint between the largest finite bf16 and
    # 2**128 round to infinity.
    if magnitude >= largest + (2.0 ** 128 - largest) / 2:
        return sign | 0x7F80
    with np.errstate(over="ignore"):
        truncated = int(np.array([magnitude], dtype=np.float32).view(np.uint32)[0]) >> 16
    candidate = max(guess & 0x7FFF, truncated)
    if candidate >= 0x7F80:
        candidate = 0x7F7F
    # Walk to the pair (lo, hi) of adjacent bf16 magnitudes around `magnitude`.
    while candidate > 0 and _bf16_value(candidate) > magnitude:
        candidate -= 1
    while candidate < 0x7F7F and _bf16_value(candidate + 1) <= magnitude:
        candidate += 1
    lo = candidate
    lo_value = _bf16_value(lo)
    if lo_value == magnitude or lo == 0x7F7F:
        return sign | lo
    hi_value = _bf16_value(lo + 1)
    mid = lo_value + (hi_value - lo_value) / 2
    if magnitude < mid:
        return sign | lo
    if magnitude > mid:
        return sign | (lo + 1)
    return sign | (lo if lo % 2 == 0 else lo + 1)


def round_to(dtype: str, values64: np.ndarray) -> np.ndarray:
    """Round float64 values once to `dtype` ('float16', 'float32', 'float64'
    or 'bfloat16'); returns float32/float16/float64 arrays, bf16 as float32."""
    values64 = np.asarray(values64, dtype=np.float64)
    if dtype == "bfloat16":
        return bf16_to_f32(f64_to_bf16(values64))
    with np.errstate(over="ignore", invalid="ignore"):
        return values64.astype(dtype)
