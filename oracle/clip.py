"""NumPy restatement of gradient norms and clipping (test infrastructure).

``total_norm`` follows ``_total_norm`` (optim/clip_grad.py:63-79): the
max-abs prescale over all gradients (NaN propagates through np.maximum), an
early return of that prescale when it is non-finite or zero or p is
infinite, else ``scale * (sum over grads of sum((|g|/scale)**p))**(1/p)`` in
float64 with the exp/log fallback when that overflows.
``clip_coefficient``/``clip_apply`` follow clip_grad.py:106-111: coef =
max_norm / (norm + 1e-6); when coef < 1 every gradient becomes
``to_grad_dtype(float64(g) * coef)`` (one rounding; bfloat16 via
lowp.f64_to_bf16).

Pinned by: golden fixtures from the reference's clip_grad_norm_ (norms for
p = 2, 1, 3, inf and clipped float32/float16 gradients, including the
non-finite cases); the L2 norm against math.fsum/np.linalg.norm in float64;
special cases (all-zero grads -> 0, an inf element -> inf, a NaN -> NaN,
norm below max_norm -> no change).
"""

from __future__ import annotations

import numpy as np

from . import lowp


def total_norm(gradients, norm_type: float = 2.0) -> float:
    scale = np.asarray(0.0, dtype=np.float64)
    for gradient in gradients:
        scale = np.maximum(scale, np.max(np.abs(gradient), initial=0))
    if not bool(np.isfinite(scale)) or bool(scale == 0) or np.isinf(norm_type):
        return float(scale)
    total = np.asarray(0.0, dtype=np.float64)
    with np.errstate(over="ignore", divide="ignore", invalid="ignore", under="ignore"):
        for gradient in gradients:
            scaled = np.abs(np.asarray(gradient, dtype=np.float64)) / scale
            total = total + np.sum(np.power(scaled, norm_type), dtype=np.float64)
        result = scale * np.power(total, 1 / norm_type)
        if not bool(np.isfinite(result)):
            result = np.exp(np.log(scale) + np.log(total) / norm_type)
    return float(result)


def clip_coefficient(max_norm: float, norm: float) -> float:
    with np.errstate(invalid="ignore", divide="ignore"):
        return float(np.divide(np.float64(max_norm), np.add(np.float64(norm), 1e-6)))


def clip_apply(gradient: np.ndarray, coefficient: float, dtype: str | None = None) -> np.ndarray:
    """float64 multiply, one rounding to the gradient dtype."""
    dtype = dtype or gradient.dtype.name
    with np.errstate(invalid="ignore", over="ignore", under="ignore"):
        product = np.multiply(np.asarray(gradient, dtype=np.float64), coefficient)
    return lowp.round_to(dtype, product)


def clip_grad_norm(gradients, max_norm: float, norm_type: float = 2.0, dtype: str | None = None):
    """Returns (norm, clipped gradients) like clip_grad_norm_ (clip_grad.py:96-112)."""
    norm = total_norm(gradients, norm_type)
    coefficient = clip_coefficient(max_norm, norm)
    if coefficient < 1:
        return norm, [clip_apply(gradient, coefficient, dtype) for gradient in gradients]
    return norm, [np.array(gradient, copy=True) for gradient in gradients]
