"""NumPy restatement of GradScaler's arithmetic (test infrastructure).

* ``unscale`` — amp.py:186-191: float16 gradients are widened to float32,
  divided by the (float32-representable) scale in float32 and stored back
  rounded to the gradient dtype; bfloat16 gradients (extension) the same way.
* ``finite`` — amp.py:152-167: every element of every unscaled gradient finite.
* ``Scaler.update`` — amp.py:219-234: backoff on any non-finite step, growth
  after ``growth_interval`` consecutive finite steps, both in float64 then
  rounded to float32 by ``_scale_value`` (amp.py:114-119) within
  [float32 tiny, float32 max].

Pinned by: golden scale/finite sequences from the reference's GradScaler
(tests/golden/make_golden.py); closed form of the sequence (s -> s/2 on a
non-finite step, s -> 2s after `interval` finite steps, clamped);
unscale by a power of two is exact (g/2**k == g*2**-k) and by other
scales equals float32 true division (checked against Python float
division rounded through numpy).
"""

from __future__ import annotations

import numpy as np

from . import lowp

_MIN = float(np.finfo(np.float32).tiny)
_MAX = float(np.finfo(np.float32).max)


def unscale(gradient: np.ndarray, scale: float, dtype: str | None = None) -> np.ndarray:
    dtype = dtype or gradient.dtype.name
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        if dtype == "float64":
            return np.divide(gradient, scale)
        data = np.asarray(gradient, dtype=np.float32)
        quotient = np.divide(data, np.float32(scale))
    if dtype == "bfloat16":
        return lowp.round_bf16(quotient)
    if dtype == "float16":
        with np.errstate(over="ignore"):
            return quotient.astype(np.float16)
    return quotient


def finite(gradients) -> bool:
    return all(bool(np.all(np.isfinite(gradient))) for gradient in gradients)


class Scaler:
    """Host state machine of GradScaler.update."""

    def __init__(self, init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=2000):
        self.scale = float(np.float32(init_scale))
        self.growth_factor = float(growth_factor)
        self.backoff_factor = float(backoff_factor)
        self.growth_interval = int(growth_interval)
        self.growth_tracker = 0

    def update(self, found_inf: bool) -> None:
        if found_inf:
            self.scale = float(np.float32(max(_MIN, self.scale * self.backoff_factor)))
            self.growth_tracker = 0
        else:
            self.growth_tracker += 1
            if self.growth_tracker == self.growth_interval:
                self.scale = float(np.float32(min(_MAX, self.scale * self.growth_factor)))
                self.growth_tracker = 0
