"""Data types of the optimizer-step path.

Mirrors ``namitorch/dtype.py:16-25`` (float16/32/64, int8/16/32/64, uint8,
bool) and adds ``bfloat16``, which the reference does not have: it is needed
for the low-precision model copies, moments and gradients of mixed-precision
training.  Each dtype knows its NumPy dtype (bfloat16 has none; its host
form is float32 values or uint16 bit patterns) and its code in the C ABI.
The package does not need PyTorch; ``torch_dtype`` and the acceptance of
``torch.dtype`` values are for callers that hand in PyTorch arrays.
"""

from __future__ import annotations

from enum import Enum

import numpy as np

from . import _native


class UnsupportedDTypeError(TypeError):
    def __init__(self, value: object):
        supported = ", ".join(dtype.value for dtype in DType)
        super().__init__(f"Unsupported NamiTorch dtype: {value!r}. Supported: {supported}.")


class DType(Enum):
    float16 = "float16"
    float32 = "float32"
    float64 = "float64"
    bfloat16 = "bfloat16"
    int8 = "int8"
    int16 = "int16"
    int32 = "int32"
    int64 = "int64"
    uint8 = "uint8"
    bool = "bool"

    # Members are singletons compared by identity: hash them by identity too
    # (C-level), since dtypes key dictionaries in the per-tensor step loop.
    __hash__ = object.__hash__

    @classmethod
    def _missing_(cls, value: object) -> "DType":
        raise UnsupportedDTypeError(value)

    def __repr__(self) -> str:
        return f"namitorch.{self.value}"

    def __str__(self) -> str:
        return repr(self)

    @property
    def itemsize(self) -> int:
        return _ITEMSIZE[self]

    @property
    def bits(self) -> int:
        return self.itemsize * 8

    @property
    def numpy_dtype(self) -> np.dtype:
        if self is DType.bfloat16:
            raise TypeError("bfloat16 has no NumPy dtype; use float32 values or uint16 bit patterns.")
        return np.dtype(self.value)

    @property
    def torch_dtype(self):
        """The matching ``torch.dtype`` (imports PyTorch)."""
        return _torch_table()[0][self]

    @property
    def code(self) -> int:
        """C-ABI storage code (NT_F32 ...); NT_DTYPE_NONE for non-floating types."""
        return self._code

    @property
    def is_floating_point(self) -> bool:
        return self._floating

    @property
    def is_integer(self) -> bool:
        return self in (DType.int8, DType.int16, DType.int32, DType.int64, DType.uint8)

    @property
    def can_require_grad(self) -> bool:
        return self.is_floating_point

    @property
    def finfo_max(self) -> float:
        if self is DType.bfloat16:
            return float.fromhex("0x1.fep127")
        return float(np.finfo(self.numpy_dtype).max)


float16 = DType.float16
float32 = DType.float32
float64 = DType.float64
bfloat16 = DType.bfloat16
int8 = DType.int8
int16 = DType.int16
int32 = DType.int32
int64 = DType.int64
uint8 = DType.uint8
bool_ = DType.bool

_ITEMSIZE = {float16: 2, float32: 4, float64: 8, bfloat16: 2, int8: 1, int16: 2, int32: 4, int64: 8, uint8: 1, bool_: 1}
_TORCH_TABLE: list = []


def _torch_table():
    """(DType -> torch.dtype, torch.dtype -> DType), built on first use."""
    if not _TORCH_TABLE:
        import torch
        forward = {member: getattr(torch, "bool" if member is bool_ else member.value) for member in DType}
        _TORCH_TABLE.extend((forward, {value: key for key, value in forward.items()}))
    return _TORCH_TABLE


def _is_torch_dtype(value: object) -> bool:
    return type(value).__module__ == "torch" and type(value).__name__ == "dtype"


_CODES = {float32: _native.NT_F32, float16: _native.NT_F16, bfloat16: _native.NT_BF16, float64: _native.NT_F64}
for _member in DType:
    # Plain attributes (not enum lookups) because the step loop reads them per tensor.
    _member._code = _CODES.get(_member, _native.NT_DTYPE_NONE)
    _member._floating = _member in _CODES
del _member


def normalize_dtype(value: object) -> DType:
    if isinstance(value, DType):
        return value
    if _is_torch_dtype(value):
        return from_torch_dtype(value)
    if isinstance(value, str):
        return DType("bool" if value == "bool_" else value)
    try:
        return from_numpy_dtype(np.dtype(value))
    except TypeError:
        raise UnsupportedDTypeError(value) from None


def from_numpy_dtype(value: np.dtype) -> DType:
    name = np.dtype(value).name
    try:
        return DType(name)
    except UnsupportedDTypeError:
        raise
    except ValueError:
        raise UnsupportedDTypeError(value) from None


def from_torch_dtype(value) -> DType:
    found = _torch_table()[1].get(value)
    if found is None:
        raise UnsupportedDTypeError(value)
    return found


# ---- promotion of a floating Tensor with a scalar operand ------------------------------
# The reference wraps a Python scalar in a Tensor (bool -> bool, int -> int64,
# float -> float32, a NumPy scalar keeps its dtype; dtype.py:177-188) and
# promotes the two dtypes with its table (dtype.py:94-109, 204-208): for a
# floating Tensor the result is the Tensor's dtype unless the scalar's dtype
# is a wider float.  bfloat16 (no reference counterpart) ranks with float16:
# integers keep it, float16 and float32 promote it to float32.
_FLOAT_RANK = {float16: 1, bfloat16: 1, float32: 2, float64: 3}


def scalar_dtype(value: object) -> DType:
    """The dtype a scalar operand gets when the reference wraps it in a Tensor."""
    if isinstance(value, np.generic):
        return from_numpy_dtype(value.dtype)
    if isinstance(value, bool):
        return bool_
    if isinstance(value, int):
        if not -(1 << 63) <= value < (1 << 63):
            raise OverflowError("Python integer is outside the supported int64 range.")
        return int64
    if isinstance(value, float):
        return float32
    raise TypeError(f"Unsupported scalar operand type {type(value).__name__}.")


def promote_with_scalar(tensor_dtype: DType, operand: DType) -> DType:
    """Result dtype of a floating Tensor combined with a scalar of `operand` dtype."""
    mine = _FLOAT_RANK[tensor_dtype]
    other = _FLOAT_RANK.get(operand, 0)
    if other == 0 or (other == mine and operand is tensor_dtype):
        return tensor_dtype
    if other <= mine and mine >= 2:
        return tensor_dtype
    if other == mine:                      # float16 with bfloat16
        return float32
    return operand if other > mine else tensor_dtype


def round_scalar(value: object, operand: DType, target: DType) -> float:
    """The scalar as the reference computes with it: stored in its own dtype
    (NumPy cast, round to nearest even), then cast to the compute dtype."""
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        stored = np.asarray(value, dtype=operand.numpy_dtype)
        if target is bfloat16:
            # One correct rounding from the value widened to float64.
            from .tensor import _bf16_bits_from_f64
            bits = _bf16_bits_from_f64(stored.astype(np.float64).reshape(1))
            return float((bits.astype(np.uint32) << 16).view(np.float32)[0])
        return float(stored.astype(target.numpy_dtype))


__all__ = ["DType", "UnsupportedDTypeError", "normalize_dtype", "from_numpy_dtype", "from_torch_dtype",
           "float16", "float32", "float64", "bfloat16"]
