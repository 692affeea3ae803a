"""Property tests (hypothesis) of the roundings and closed forms the step
relies on, on the CPU: the oracle's and the host package's conversions
against exact rational rounding, the norm against its exact value and its
power-of-two scaling, and the loss-scale state machine against an integer
model of its exponent.

The expected values come from ``fractions.Fraction`` arithmetic or from
NumPy's scalar constructors (what the reference's ``_scalar`` calls,
optim/_common.py:39-47), never from the code under test."""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from namitorch_amd.dtype import DType
from namitorch_amd.optim._common import _round_scalar
from namitorch_amd.tensor import _bf16_bits_from_f64
from oracle import clip as oclip
from oracle import lowp
from oracle import scaler as oscaler

SETTINGS = settings(max_examples=300, deadline=None, suppress_health_check=[HealthCheck.too_slow])
FINITE = st.floats(allow_nan=False, allow_infinity=False, width=64)

# (stored fraction bits, smallest normal exponent, largest exponent)
FORMATS = {"bfloat16": (7, -126, 127), "float16": (10, -14, 15), "float32": (23, -126, 127)}


def nearest_even(x: float, fmt: str) -> float:
    """`x` rounded once to `fmt`, ties to even, by exact rational
    arithmetic: the grid spacing at |x| (subnormal spacing below the
    smallest normal), Python's round() of the exact quotient (ties to even),
    infinity past the largest finite value."""
    if x == 0:
        return x
    bits, emin, emax = FORMATS[fmt]
    sign = -1.0 if x < 0 else 1.0
    _, e = math.frexp(abs(x))                      # |x| in [2**(e-1), 2**e)
    ulp = Fraction(2) ** (max(e - 1, emin) - bits)
    value = round(Fraction(abs(x)) / ulp) * ulp
    largest = (2 - Fraction(2) ** -bits) * Fraction(2) ** emax
    return sign * (math.inf if value > largest else float(value))


def bf16_bits(value: float) -> int:
    return int(np.array([value], dtype=np.float32).view(np.uint32)[0]) >> 16


@st.composite
def bf16_ties(draw):
    """float64 values exactly halfway between two adjacent finite bfloat16
    values (either sign), where ties-to-even decides."""
    low = draw(st.integers(0, 0x7F7E))
    a = Fraction(float(lowp.bf16_to_f32(np.array([low], np.uint16))[0]))
    b = Fraction(float(lowp.bf16_to_f32(np.array([low + 1], np.uint16))[0]))
    value = float((a + b) / 2)                     # 9 significant bits: exact in float64
    return -value if draw(st.booleans()) else value


@SETTINGS
@given(st.one_of(FINITE, bf16_ties(), st.floats(min_value=3.38e38, max_value=3.41e38)))
def test_bf16_from_f64_is_one_nearest_even_rounding(x):
    want = bf16_bits(nearest_even(x, "bfloat16"))
    assert int(lowp.f64_to_bf16(np.array([x]))[0]) == want, x
    assert int(_bf16_bits_from_f64(np.array([x]))[0]) == want, x


@SETTINGS
@given(st.one_of(st.floats(allow_nan=False, allow_infinity=False, width=32), bf16_ties()))
def test_bf16_from_f32_is_one_nearest_even_rounding(x):
    assert int(lowp.f32_to_bf16(np.array([x], np.float32))[0]) == bf16_bits(nearest_even(x, "bfloat16")), x


@SETTINGS
@given(FINITE)
def test_fp16_and_fp32_rounding_is_nearest_even(x):
    """lowp.round_to (the oracle's clip/unscale rounding) for the IEEE formats."""
    for fmt in ("float16", "float32"):
        got = float(lowp.round_to(fmt, np.array([x]))[0])
        want = nearest_even(x, fmt)
        assert got == want and math.copysign(1.0, got) == math.copysign(1.0, want), (fmt, x)


@SETTINGS
@given(st.one_of(FINITE, st.floats(min_value=6.5e4, max_value=6.6e4), st.floats(min_value=3.40e38, max_value=3.41e38)))
def test_optimizer_scalars_round_like_numpy_scalar_constructors(x):
    """The host's coefficient rounding (_round_scalar) equals the reference's
    dtype.type(value) wherever the reference accepts the value, and refuses
    it (ValueError) wherever the reference does."""
    for dtype, numpy_type in ((DType.float32, np.float32), (DType.float16, np.float16), (DType.float64, np.float64)):
        if abs(x) > float(np.finfo(numpy_type).max):
            with pytest.raises(ValueError, match="must be representable"):
                _round_scalar(dtype, x)
            continue
        with np.errstate(over="ignore", under="ignore"):
            want = float(numpy_type(x))
        got = _round_scalar(dtype, x)
        assert got == want and math.copysign(1.0, got) == math.copysign(1.0, want), (dtype, x)


@SETTINGS
@given(st.lists(st.floats(min_value=-1e3, max_value=1e3, allow_nan=False), min_size=1, max_size=40),
       st.floats(min_value=2.0 ** -30, max_value=2.0 ** 30))
def test_clip_apply_rounds_the_float64_product_once(values, coefficient):
    """clip_grad_norm_ multiplies in float64 and copies into the gradient
    dtype (clip_grad.py:108-111): the exact product rounded to float64, then
    that rounded once to the gradient dtype."""
    gradient = np.array(values, dtype=np.float64)
    for fmt in ("bfloat16", "float16", "float32"):
        got = oclip.clip_apply(gradient, coefficient, fmt).astype(np.float64)
        for g, value in zip(values, got):
            product = float(Fraction(g) * Fraction(coefficient))
            assert value == nearest_even(product, fmt), (fmt, g, coefficient)


GRADIENTS = st.lists(st.lists(st.floats(min_value=-1e6, max_value=1e6, allow_nan=False, allow_subnormal=False),
                              min_size=0, max_size=120), min_size=1, max_size=4)


@SETTINGS
@given(GRADIENTS, st.sampled_from([np.float32, np.float64]))
def test_total_norm_is_close_to_the_exact_2_norm(lists, dtype):
    gradients = [np.array(values, dtype=dtype) for values in lists]
    exact = sum((Fraction(float(v)) ** 2 for g in gradients for v in g), Fraction(0))
    norm = oclip.total_norm(gradients)
    if exact == 0:
        assert norm == 0.0
        return
    assert abs(Fraction(norm) ** 2 / exact - 1) <= Fraction(1, 10 ** 13), (norm, float(exact))


@SETTINGS
@given(GRADIENTS, st.integers(-20, 20), st.sampled_from([1.0, 2.0, 3.0, math.inf]))
def test_total_norm_scales_exactly_by_powers_of_two(lists, k, order):
    """The max-abs prescale divides any power-of-two factor out exactly
    (clip_grad.py:63-79), so scaling every gradient by 2**k scales the norm
    by exactly 2**k: a dropped prescale or a wrong final multiply breaks it."""
    gradients = [np.array(values, dtype=np.float64) for values in lists]
    factor = 2.0 ** k
    assert oclip.total_norm([g * factor for g in gradients], order) == factor * oclip.total_norm(gradients, order)


@SETTINGS
@given(st.lists(st.booleans(), max_size=80), st.integers(1, 6), st.integers(-40, 40))
def test_scaler_follows_the_exponent_model(found, interval, start):
    """With growth 2, backoff 0.5 and a power-of-two start clear of the
    float32 range ends, the scale is 2**e: e falls by one at every
    non-finite iteration and rises by one after every `interval`
    consecutive finite ones (amp.py:225-233)."""
    scaler = oscaler.Scaler(2.0 ** start, growth_factor=2.0, backoff_factor=0.5, growth_interval=interval)
    exponent, run = start, 0
    for bad in found:
        scaler.update(bad)
        if bad:
            exponent, run = exponent - 1, 0
        else:
            run += 1
            if run == interval:
                exponent, run = exponent + 1, 0
        assert scaler.scale == 2.0 ** exponent
        assert scaler.growth_tracker == run
