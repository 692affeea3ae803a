"""NumPy restatement of Tensor-by-scalar arithmetic (test infrastructure).

``scalar_op(values, operand, op)`` follows the reference's
``Tensor._binary_operation`` with a scalar operand (tensor.py:585-646,
_backend.py:54-72): the scalar becomes an array of its own dtype (bool ->
bool, int -> int64, float -> float32, a NumPy scalar keeps its dtype;
dtype.py:177-188), both operands are cast to the promoted dtype
(dtype.py:94-109, 204-208; for a floating array only a wider float operand
changes it) and one NumPy ufunc computes the result in that dtype.  This is
what ``GradScaler.scale`` (amp.py:137-138) and the training loop's
``loss / grad_accum_steps`` (runner.py:246) compute.

Pinned by: tests/golden/scalar_ops.npz, written by the reference's own
GradScaler.scale and Tensor operators for float16/32/64 losses (scales
65536, 3000, 0.125; int, float, float16 and float64 divisors and factors).
"""

from __future__ import annotations

import numpy as np

_RANK = {np.dtype(np.float16): 1, np.dtype(np.float32): 2, np.dtype(np.float64): 3}


def operand_dtype(value) -> np.dtype:
    if isinstance(value, np.generic):
        return value.dtype
    if isinstance(value, bool):
        return np.dtype(np.bool_)
    if isinstance(value, int):
        return np.dtype(np.int64)
    return np.dtype(np.float32)


def result_dtype(values_dtype, value) -> np.dtype:
    mine = np.dtype(values_dtype)
    other = operand_dtype(value)
    if other.kind != "f" or _RANK[other] <= _RANK[mine]:
        return mine
    return other


def scalar_op(values: np.ndarray, value, op: str) -> np.ndarray:
    """``values * value`` (op "mul") or ``values / value`` (op "div")."""
    values = np.asarray(values)
    compute = result_dtype(values.dtype, value)
    with np.errstate(over="ignore", under="ignore", invalid="ignore", divide="ignore"):
        left = values.astype(compute)
        right = np.asarray(value, dtype=operand_dtype(value)).astype(compute)
        ufunc = np.multiply if op == "mul" else np.true_divide
        return ufunc(left, right, dtype=compute)


def scale_loss(loss: np.ndarray, scale: float) -> np.ndarray:
    """GradScaler.scale: ``loss * scale`` with the scale a Python float."""
    return scalar_op(loss, float(scale), "mul")
