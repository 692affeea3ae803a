"""NumPy restatement of gradient accumulation (test infrastructure).

``accumulate(existing, incoming, dtype)`` — autograd.accumulate_gradient
(autograd.py:198-205): the incoming gradient is cast to the leaf dtype
(NumPy cast, round to nearest even); without a stored gradient the result is
that cast copy, otherwise ``np.add`` of the stored and the cast gradient in
the leaf dtype.  ``"bfloat16"`` (extension, no reference counterpart) casts
with round-to-nearest-even and adds in float32 with one rounding, like
NumPy's float16 add.

Pinned by: the reference's own accumulate_gradient outputs for leaf dtypes
float32/16/64 and incoming float16/32/64 with special values
(tests/golden/accumulate.npz); for bfloat16, torch's RNE conversion and the
exactness of float32 sums of bfloat16 values whose exponents differ by at
most 15 (tests/test_oracle.py).
"""

from __future__ import annotations

import numpy as np

from . import lowp


def accumulate(existing: np.ndarray | None, incoming: np.ndarray, dtype) -> np.ndarray:
    if isinstance(dtype, str) and dtype == "bfloat16":
        converted = lowp.round_to("bfloat16", np.asarray(incoming, dtype=np.float64))
        if existing is None:
            return converted.copy()
        with np.errstate(over="ignore", invalid="ignore"):
            total = np.asarray(existing, dtype=np.float32) + converted.astype(np.float32)
        return lowp.round_bf16(total)
    dtype = np.dtype(dtype)
    with np.errstate(over="ignore", invalid="ignore"):
        converted = np.asarray(incoming, dtype=dtype)
        if existing is None:
            return np.array(converted, copy=True, order="C")
        return np.asarray(np.add(existing, converted), dtype=dtype)
