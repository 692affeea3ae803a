"""Tensor and Parameter: the storage holder the optimizer-step path needs.

This is not a general tensor library.  It keeps the parts of
``namitorch/tensor.py`` the hot path touches: a contiguous storage array
(``_data``), ``dtype``/``shape``/``device``, ``requires_grad`` and ``grad``,
the in-place version counter (``tensor.py:71-76``) and ``copy_`` /
``__setitem__(...)`` that convert to the destination dtype and bump the
version (``tensor.py:1269-1287``).

Storage is a contiguous ``torch.Tensor`` (device memory on HIP devices):
torch is used for allocation and streams only, never for the step's
arithmetic.

Deferred gradient transforms.  ``GradScaler.unscale_`` and
``clip_grad_norm_`` rewrite gradients in place in the reference
(``amp.py:191``, ``optim/clip_grad.py:111``).  Here the rewrite is recorded
on the gradient as a pending :class:`GradTransform` and fused into the next
kernel that reads the gradient (the AdamW pass); any other access to
``_data`` first writes the transformed values back with a kernel, so every
observer sees exactly the values the reference would have stored.
"""

from __future__ import annotations

import builtins
import threading
from contextlib import contextmanager
from dataclasses import dataclass
from numbers import Real

import numpy as np
import torch

from .backends._graph_capture import reject_during_capture
from .device import Device
from .dtype import (
    DType,
    bfloat16,
    float16,
    float32,
    from_numpy_dtype,
    from_torch_dtype,
    int64,
    normalize_dtype,
    promote_with_scalar,
    round_scalar,
    scalar_dtype,
)


class _VersionCounter:
    __slots__ = ("value",)

    def __init__(self, value: int = 0):
        self.value = value

    def increment(self) -> None:
        self.value += 1


# Device-decided optimizer steps (namitorch_amd.amp.fused_step) whose host
# bookkeeping (version counters, step counts) is still optimistic, oldest
# first; each removes itself when reconciled.
_unsettled_steps: list = []


def _settle_device_steps() -> None:
    while _unsettled_steps:
        _unsettled_steps[0].reconcile()


# ---- grad mode (namitorch/autograd.py:15-42) -----------------------------------------
_grad_mode = threading.local()
# One immutable Device per torch device: tensors on one device share it, so
# device comparisons between them are identity checks.
_DEVICES: dict = {}


def _storage_device(place: torch.device) -> Device:
    found = _DEVICES.get(place)
    if found is None:
        found = Device("cpu") if place.type == "cpu" else Device("cuda", place.index)
        _DEVICES[place] = found
    return found


def is_grad_enabled() -> bool:
    return getattr(_grad_mode, "enabled", True)


@contextmanager
def _grad_enabled(mode: bool):
    previous = is_grad_enabled()
    _grad_mode.enabled = mode
    try:
        yield
    finally:
        _grad_mode.enabled = previous


def no_grad():
    return _grad_enabled(False)


def enable_grad():
    return _grad_enabled(True)


@dataclass(frozen=True)
class GradTransform:
    """Pending in-place rewrite of a gradient: ``g <- clip(unscale(g))``.

    ``scale``: divide by this fp32 loss scale and round to the grad dtype
    (``amp.py:190-191``); ``clip``: multiply by this fp64 coefficient and
    round to the grad dtype (``optim/clip_grad.py:111``).  ``None`` = absent.
    ``device``: the scale, the clip decision and its coefficient live in the
    control block of a device-decided step (``namitorch_amd.amp.DeviceStep``)
    instead; compared by identity.
    """

    scale: float | None = None
    clip: float | None = None
    device: object = None

    def then_clip(self, coefficient: float) -> "GradTransform":
        return GradTransform(self.scale, coefficient, self.device)


# ---- host-side conversions used when creating storage ---------------------------------
def _bf16_bits_from_f64(values: np.ndarray) -> np.ndarray:
    """Correctly rounded (RNE) float64 -> bfloat16 bit patterns.

    Rounds to float32 with round-to-odd first (exact for the second rounding
    because float32 keeps 16 more significand bits than bfloat16), then RNE.
    """
    values = np.asarray(values, dtype=np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        nearest = values.astype(np.float32)
        back = nearest.astype(np.float64)
    bits = nearest.view(np.uint32).copy()
    inexact = (back != values) & ~np.isnan(values)
    away = inexact & (np.abs(back) > np.abs(values))
    bits -= away.astype(np.uint32)
    bits |= inexact.astype(np.uint32)
    return _bf16_bits_from_f32_bits(bits)


def _bf16_bits_from_f32_bits(bits: np.ndarray) -> np.ndarray:
    bits = np.asarray(bits, dtype=np.uint32)
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    quiet = ((bits >> 16) | 0x40).astype(np.uint16)
    return np.where(nan, quiet, rounded)


def _host_array(data: object, dtype: DType) -> torch.Tensor:
    """Host data -> CPU torch tensor of `dtype`, rounded once like NumPy's cast."""
    if dtype is bfloat16:
        array = np.asarray(data)
        if array.dtype == np.float32:
            bits = _bf16_bits_from_f32_bits(array.view(np.uint32))
        else:
            bits = _bf16_bits_from_f64(array.astype(np.float64))
        return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        array = np.array(data, dtype=dtype.numpy_dtype, copy=True, order="C")
    return torch.from_numpy(array)


def _resolve_dtype(data: object, dtype: object) -> DType:
    if dtype is not None:
        return normalize_dtype(dtype)
    if isinstance(data, Tensor):
        return data.dtype
    if isinstance(data, torch.Tensor):
        return from_torch_dtype(data.dtype)
    if isinstance(data, (np.ndarray, np.generic)):
        return from_numpy_dtype(data.dtype)
    if isinstance(data, builtins.bool):
        return DType.bool
    if isinstance(data, int):
        return int64
    if isinstance(data, (float, Real)):
        return float32
    array = np.asarray(data)
    if array.dtype.kind == "f":
        return float32
    return from_numpy_dtype(array.dtype)


def _make_storage(data: object, dtype: DType, device: Device) -> torch.Tensor:
    source = data._data if isinstance(data, Tensor) else data
    if isinstance(source, torch.Tensor):
        if source.dtype == torch.float64 and dtype in (float16, bfloat16) and source.device.type != "cpu":
            raise TypeError("Device float64 -> float16/bfloat16 conversions must go through the host for exact rounding.")
        if source.dtype == torch.float64 and dtype in (float16, bfloat16):
            host = _host_array(source.numpy(), dtype)
            return host.to(device.torch, copy=True).contiguous()
        return source.to(device=device.torch, dtype=dtype.torch_dtype, copy=True).contiguous()
    host = _host_array(source, dtype)
    return host.to(device.torch, copy=True).contiguous()


class Tensor:
    __slots__ = (
        "_storage", "_dtype", "_device", "_requires_grad", "_grad", "_version_counter",
        "_writable", "_pending", "_is_leaf", "_ptr", "_numel", "_clean_version", "_finite_version", "__weakref__",
    )

    def __init__(self, data: object, dtype: object = None, requires_grad: builtins.bool = False, *, device=None):
        resolved = _resolve_dtype(data, dtype)
        if device is None:
            if isinstance(data, Tensor):
                target = data.device
            elif isinstance(data, torch.Tensor):
                target = Device(str(data.device)) if data.device.type == "cpu" else Device("cuda", data.device.index)
            else:
                target = Device("cpu")
        else:
            target = Device(device)
        self._initialize(_make_storage(data, resolved, target), requires_grad)

    def _initialize(self, storage: torch.Tensor, requires_grad: builtins.bool, version_counter: _VersionCounter | None = None):
        if not isinstance(storage, torch.Tensor) or not storage.is_contiguous():
            raise TypeError("Tensor storage must be a contiguous array.")
        self._storage = storage
        self._dtype = from_torch_dtype(storage.dtype)
        self._device = _storage_device(storage.device)
        if requires_grad and not self._dtype.can_require_grad:
            raise TypeError(f"Only floating Tensors can require gradients, got {self._dtype.name}.")
        self._requires_grad = requires_grad
        self._grad = None
        self._version_counter = version_counter if version_counter is not None else _VersionCounter()
        self._writable = True
        self._pending = None
        self._is_leaf = True
        self._ptr = storage.data_ptr() if storage.device.type != "cpu" else None
        self._numel = storage.numel()
        self._clean_version = None      # version at which a state buffer was last known nonnegative
        self._finite_version = None     # version at which GradScaler last knew the gradient's finiteness

    @classmethod
    def _from_storage(cls, storage: torch.Tensor, requires_grad: builtins.bool = False, version_counter=None) -> "Tensor":
        instance = cls.__new__(cls)
        Tensor._initialize(instance, storage, requires_grad, version_counter)
        return instance

    # ---- storage access --------------------------------------------------------------
    @property
    def _data(self) -> torch.Tensor:
        if self._pending is not None:
            self._materialize()
        return self._storage

    def _materialize(self) -> None:
        """Write a pending gradient transform back into storage."""
        pending = self._pending
        if pending is None:
            return
        from .backends import get_backend
        get_backend(self).apply_grad_transform([self], pending)
        self._pending = None

    @property
    def device(self) -> Device:
        return self._device

    @property
    def shape(self) -> tuple[int, ...]:
        return tuple(self._storage.shape)

    @property
    def ndim(self) -> int:
        return self._storage.dim()

    @property
    def size(self) -> int:
        return self._numel

    def numel(self) -> int:
        return self._numel

    @property
    def dtype(self) -> DType:
        return self._dtype

    @property
    def nbytes(self) -> int:
        return self.size * self._dtype.itemsize

    @property
    def requires_grad(self) -> builtins.bool:
        return self._requires_grad

    @requires_grad.setter
    def requires_grad(self, value: builtins.bool) -> None:
        if type(value) is not builtins.bool:
            raise TypeError("requires_grad must be a Python bool.")
        if value and not self._dtype.can_require_grad:
            raise TypeError(f"Only floating Tensors can require gradients, got {self._dtype.name}.")
        if not self._is_leaf:
            raise ValueError("requires_grad can only be changed on leaf tensors.")
        self._requires_grad = value

    def requires_grad_(self, mode: builtins.bool = True) -> "Tensor":
        self.requires_grad = mode
        return self

    @property
    def grad(self) -> "Tensor | None":
        return self._grad

    @grad.setter
    def grad(self, value: "Tensor | None") -> None:
        # The reference stores gradients through autograd (tensor.py:445-450);
        # this setter is how callers hand in gradients computed elsewhere.
        if value is not None and not isinstance(value, Tensor):
            raise TypeError("Parameter gradients must be NamiTorch Tensors.")
        self._grad = value

    @property
    def grad_fn(self):
        return None

    @property
    def is_leaf(self) -> builtins.bool:
        return self._is_leaf

    @property
    def _version(self) -> int:
        """In-place version (tensor.py:71-76).  A fused step decided on the
        device bumps versions before its outcome is known; reading a version
        settles such steps first, so a skipped step reads as never taken."""
        if _unsettled_steps:
            _settle_device_steps()
        return self._version_counter.value

    # ---- in-place updates (tensor.py:1252-1287) ------------------------------------------
    def _ensure_inplace_allowed(self) -> None:
        reject_during_capture("In-place Tensor updates")
        self._check_inplace()

    def _check_inplace(self) -> None:
        """The per-tensor half of ``_ensure_inplace_allowed``, for loops that
        have already checked for graph capture once."""
        if self._requires_grad and is_grad_enabled():
            raise RuntimeError("In-place assignment is not allowed on a Tensor with requires_grad=True.")
        if not self._writable:
            raise RuntimeError("Cannot assign to read-only Tensor storage.")

    def copy_(self, src: object) -> "Tensor":
        self._ensure_inplace_allowed()
        if isinstance(src, Tensor) and src.requires_grad and is_grad_enabled():
            raise RuntimeError("copy_ from a Tensor with requires_grad=True must run inside no_grad().")
        self[...] = src
        return self

    def __setitem__(self, index: object, value: object) -> None:
        if index is not Ellipsis:
            raise NotImplementedError("namitorch_amd Tensors support only whole-tensor assignment (t[...] = value).")
        self._ensure_inplace_allowed()
        if isinstance(value, Tensor) and value.device != self.device:
            raise RuntimeError(f"Operands are on different devices: {self.device}, {value.device}; use an explicit .to() transfer.")
        converted = _make_storage(value, self._dtype, self._device)
        if converted.numel() == 1 and self.size != 1:
            converted = converted.reshape(()).expand(self.shape)
        elif tuple(converted.shape) != self.shape:
            converted = converted.reshape(self.shape) if converted.numel() == self.size else converted.expand(self.shape)
        self._pending = None
        self._storage.copy_(converted)
        self._version_counter.increment()

    def _accumulate_grad(self, gradient: "Tensor") -> None:
        """Add `gradient` (cast to this leaf's dtype) into ``self.grad``, or
        make it the gradient (tensor.py:443-450); see ``grads.accumulate_grads``."""
        from .grads import accumulate_grads
        accumulate_grads([self], [gradient])

    def zero_(self) -> "Tensor":
        return self.fill_(0)

    def fill_(self, value: object) -> "Tensor":
        self._ensure_inplace_allowed()
        if isinstance(value, Tensor) and value.ndim != 0:
            raise ValueError("fill_ requires a scalar value or a zero-dimensional Tensor.")
        self[...] = value
        return self

    # ---- conversions ---------------------------------------------------------------------
    def numpy(self) -> np.ndarray:
        """Host copy; bfloat16 is returned as (exact) float32 values."""
        reject_during_capture("Host Tensor reads")
        storage = self._data
        if self._dtype is bfloat16:
            storage = storage.to(torch.float32)
        return storage.detach().cpu().numpy().copy()

    def bits(self) -> np.ndarray:
        """Host copy of the raw bit patterns (uint16 for 16-bit types)."""
        reject_during_capture("Host Tensor reads")
        storage = self._data
        view = {2: torch.int16, 4: torch.int32, 8: torch.int64, 1: torch.uint8}[self._dtype.itemsize]
        unsigned = {2: np.uint16, 4: np.uint32, 8: np.uint64, 1: np.uint8}[self._dtype.itemsize]
        return storage.view(view).cpu().numpy().view(unsigned).copy()

    def item(self):
        reject_during_capture("Host Tensor reads")
        if self.size != 1:
            raise ValueError(f"item() requires exactly one element, got {self.size}.")
        return self._data.reshape(()).item()

    def detach(self) -> "Tensor":
        result = Tensor._from_storage(self._data, False, self._version_counter)
        return result

    def clone(self) -> "Tensor":
        return Tensor._from_storage(self._data.clone(), False)

    def to(self, device=None, dtype=None) -> "Tensor":
        target = self.device if device is None else Device(device)
        kind = self._dtype if dtype is None else normalize_dtype(dtype)
        if target == self.device and kind is self._dtype:
            return self
        return Tensor(self, dtype=kind, device=target)

    def _scalar_arithmetic(self, other, op: int) -> "Tensor":
        """``self * other`` or ``self / other`` for a scalar ``other``, with the
        reference's promotion (tensor.py:585-646: the scalar becomes a Tensor of
        its own dtype, both operands are cast to the promoted dtype and one
        NumPy ufunc computes the result in it)."""
        if isinstance(other, Tensor):
            return NotImplemented
        if not isinstance(other, (builtins.bool, builtins.int, builtins.float, np.generic)):
            raise TypeError(
                f"Operators require Tensor, Python scalar or NumPy scalar operands, got {type(other).__name__}. "
                "Convert sequences and ndarrays explicitly with tensor() or as_tensor()."
            )
        if not self._dtype.is_floating_point:
            raise TypeError("Only floating Tensors support scalar arithmetic on the device.")
        operand = scalar_dtype(other)
        result = promote_with_scalar(self._dtype, operand)
        from .backends import get_backend
        return get_backend(self).scalar_arithmetic(self, round_scalar(other, operand, result), op, result)

    def __mul__(self, other):
        from ._native import NT_OP_MUL
        return self._scalar_arithmetic(other, NT_OP_MUL)

    __rmul__ = __mul__

    def __truediv__(self, other):
        from ._native import NT_OP_DIV
        return self._scalar_arithmetic(other, NT_OP_DIV)

    def __len__(self) -> int:
        if self.ndim == 0:
            raise TypeError("len() is not defined for a scalar Tensor.")
        return self.shape[0]

    def __repr__(self) -> str:
        location = "" if self.device.type == "cpu" else f", device='{self.device}'"
        if self.size <= 8:
            values = np.array2string(self.numpy(), separator=", ")
        else:
            values = f"<{self.size} elements>"
        return f"tensor({values}, shape={self.shape}, dtype={self.dtype.name}{location}, requires_grad={self.requires_grad})"


class Parameter(Tensor):
    __slots__ = ()

    def __init__(self, data: object, requires_grad: builtins.bool | None = None, *, dtype: object = None, device=None):
        super().__init__(data, dtype=dtype, device=data.device if device is None and isinstance(data, Tensor) else device)
        self.requires_grad = self.dtype.can_require_grad if requires_grad is None else requires_grad

    def __repr__(self) -> str:
        return f"Parameter({super().__repr__()})"


def tensor(data: object, dtype: object = None, requires_grad: builtins.bool = False, *, device=None) -> Tensor:
    return Tensor(data, dtype=dtype, requires_grad=requires_grad, device=device)


__all__ = ["Tensor", "Parameter", "tensor", "no_grad", "enable_grad", "is_grad_enabled", "GradTransform"]
