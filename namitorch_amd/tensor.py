"""Tensor and Parameter: the storage holder the optimizer-step path needs.

This is not a general tensor library.  It keeps the parts of
``namitorch/tensor.py`` the hot path touches: a contiguous storage array
(``_data``), ``dtype``/``shape``/``device``, ``requires_grad`` and ``grad``,
the in-place version counter (``tensor.py:71-76``) and ``copy_`` /
``__setitem__(...)`` that convert to the destination dtype and bump the
version (``tensor.py:1269-1287``).

Storage is contiguous: a NumPy array on the host (bfloat16 as uint16 bit
patterns) and a :class:`namitorch_amd.array.DeviceArray` on HIP devices,
memory of the library's own allocator or, wrapped without a copy, a device
array of another framework.

Deferred gradient transforms.  ``GradScaler.unscale_`` and
``clip_grad_norm_`` rewrite gradients in place in the reference
(``amp.py:191``, ``optim/clip_grad.py:111``).  Here the rewrite is recorded
on the gradient as a pending :class:`GradTransform` and fused into the next
kernel that reads the gradient (the AdamW pass); any other access to
``_data`` first writes the transformed values back with a kernel, so every
observer sees exactly the values the reference would have stored.

Deferred accumulation.  ``accumulate_grads(..., defer=True)`` records the
last micro-batch's gradient on the stored gradient (``_incoming``) instead
of adding it; the pre-pass and the AdamW pass add it as they read the
gradient, and any other access writes the sum back first.  The addition
comes before a pending transform, as in the reference's order of events.
"""

from __future__ import annotations

import builtins
import threading
from contextlib import contextmanager
from dataclasses import dataclass
from numbers import Real

import numpy as np

from .array import DeviceArray, is_device_array
from .backends._graph_capture import reject_during_capture
from .device import Device
from .dtype import (
    DType,
    bfloat16,
    float32,
    from_numpy_dtype,
    from_torch_dtype,
    int64,
    normalize_dtype,
    promote_with_scalar,
    round_scalar,
    scalar_dtype,
)

_CPU = Device("cpu")
_UNSIGNED = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}


class _VersionCounter:
    __slots__ = ("value",)

    def __init__(self, value: int = 0):
        self.value = value

    def increment(self) -> None:
        """One in-place write.  Device-decided steps still pending settle
        first, so the optimistic bumps they undo are never mixed with this
        write's."""
        if _unsettled_steps:
            _settle_device_steps()
        self.value += 1


# Device-decided optimizer steps (namitorch_amd.amp.fused_step) whose host
# bookkeeping (version counters, step counts) is still optimistic, oldest
# first; each removes itself when reconciled.  Entries are added by a plain
# append and removed one by one, so threads never lose each other's entries.
_unsettled_steps: list = []

# Held while a step is reconciled or its control block is read: each step's
# rollback runs once, whichever thread settles it (its own optimizer's next
# step, a result access, or an in-place write on any thread).  Re-entrant:
# settling all pending steps holds it around each step's own reconcile.
_settle_lock = threading.RLock()


# Bumped whenever ``requires_grad`` changes on an existing Tensor (its only
# route after creation), so memoized checks of the flag can skip re-reading
# it while the count is unchanged.
_requires_grad_changes = _VersionCounter()
_requires_grad_lock = threading.Lock()


def _settle_device_steps() -> None:
    with _settle_lock:
        while _unsettled_steps:
            _unsettled_steps[0].reconcile()


def check_addends(gradients) -> None:
    """Raise if the incoming gradient of a deferred accumulation
    (``accumulate_grads(..., defer=True)``) changed after it was deferred:
    its values are read only when the accumulation is consumed."""
    for gradient in gradients:
        incoming = gradient._incoming
        if incoming is not None and incoming[0]._version_counter.value != incoming[1]:
            raise RuntimeError("An incoming gradient of a deferred accumulation was modified in place before the "
                               "accumulation ran; keep it unchanged until the next step or read of the gradient.")


# ---- grad mode (namitorch/autograd.py:15-42) -----------------------------------------
_grad_mode = threading.local()


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


def _values(storage: np.ndarray, dtype: DType) -> np.ndarray:
    """The values a host storage array holds (bfloat16 bits widened exactly to float32)."""
    if dtype is bfloat16:
        return (np.ascontiguousarray(storage).astype(np.uint32) << 16).view(np.float32)
    return storage


def _host_framework_array(data) -> np.ndarray | None:
    """Values of another framework's host array (PyTorch-style ``numpy()``),
    bfloat16 widened exactly; None for anything else."""
    place = getattr(data, "device", None)
    if getattr(place, "type", None) != "cpu" or not callable(getattr(data, "numpy", None)):
        return None
    if str(getattr(data, "dtype", "")).endswith("bfloat16"):
        return data.float().numpy()
    return data.numpy()


def _host_array(data: object, dtype: DType) -> np.ndarray:
    """Host data -> a NumPy array in `dtype`'s storage format (bfloat16 as
    uint16 bit patterns), rounded once like NumPy's cast."""
    framework = _host_framework_array(data)
    if framework is not None:
        data = framework
    if dtype is bfloat16:
        array = np.ascontiguousarray(data)
        if array.dtype == np.float32:
            return np.ascontiguousarray(_bf16_bits_from_f32_bits(array.view(np.uint32)))
        return np.ascontiguousarray(_bf16_bits_from_f64(array.astype(np.float64)))
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        return np.array(data, dtype=dtype.numpy_dtype, copy=True, order="C")


def _resolve_dtype(data: object, dtype: object) -> DType:
    if dtype is not None:
        return normalize_dtype(dtype)
    if isinstance(data, Tensor):
        return data.dtype
    if isinstance(data, DeviceArray):
        return data.dtype
    if not isinstance(data, (np.ndarray, np.generic)) and type(getattr(data, "dtype", None)).__module__ == "torch":
        return from_torch_dtype(data.dtype)
    if is_device_array(data):
        return DeviceArray.wrap(data).dtype
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


def _make_storage(data: object, dtype: DType, device: Device):
    """New storage of `dtype` on `device` holding `data`'s values, each
    rounded once to `dtype` (NumPy's cast; on the device ``nt_cast``)."""
    if isinstance(data, Tensor):
        source, source_dtype = data._data, data._dtype
    else:
        source, source_dtype = data, None
    if isinstance(source, DeviceArray) or (not isinstance(source, np.ndarray) and is_device_array(source)):
        array = DeviceArray.wrap(source)
        if device is array.device and (array.dtype is dtype or (array.dtype._floating and dtype._floating)):
            return DeviceArray.empty(array.shape, dtype, device).copy_from(array)
        source = _values(array.download(), array.dtype)
    elif source_dtype is not None:
        source = _values(source, source_dtype)
    host = _host_array(source, dtype)
    if device.type == "cpu":
        return host
    return DeviceArray.empty(host.shape, dtype, device).upload(host)


def _device_of(data: object) -> Device:
    """Where data handed to the Tensor constructor lives."""
    if isinstance(data, Tensor):
        return data.device
    if isinstance(data, DeviceArray):
        return data.device
    if not isinstance(data, np.ndarray) and is_device_array(data):
        return DeviceArray.wrap(data).device
    return _CPU


def _on_device(value: object) -> bool:
    return isinstance(value, DeviceArray) or (not isinstance(value, np.ndarray) and is_device_array(value))


def _assign_device(target: DeviceArray, source: object, dtype: DType) -> None:
    """``target[...] = source`` for device storage: device sources are copied
    (and converted between floating dtypes) on the device; host values are
    converted on the host and uploaded, a single value as a fill."""
    if _on_device(source):
        array = DeviceArray.wrap(source)
        if array.device != target.device:
            raise RuntimeError(f"Operands are on different devices: {target.device}, {array.device}; "
                               "use an explicit .to() transfer.")
        if array.numel() == target.numel() and (array.dtype is dtype or (array.dtype._floating and dtype._floating)):
            if array.data_ptr() != target.data_ptr():
                target.copy_from(array)
            return
        source = _values(array.download(), array.dtype)
    host = _host_array(source, dtype)
    if host.size == 1 and target.numel() != 1:
        target.fill_bits(int(host.reshape(-1).view(_UNSIGNED[dtype.itemsize])[0]))
        return
    if host.size != target.numel():
        host = np.ascontiguousarray(np.broadcast_to(host, target.shape))
    target.upload(host)


def _assign_host(target: np.ndarray, source: object, dtype: DType, source_dtype: DType | None) -> None:
    """``target[...] = source`` for host storage; `source_dtype` names the
    dtype of a Tensor's storage handed in as `source`."""
    if source_dtype is not None:
        source = _values(source, source_dtype)
    elif _on_device(source):
        array = DeviceArray.wrap(source)
        source = _values(array.download(), array.dtype)
    host = _host_array(source, dtype)
    if host.size == target.size:
        host = host.reshape(target.shape)
    np.copyto(target, np.broadcast_to(host, target.shape))


class Tensor:
    __slots__ = (
        "_storage", "_dtype", "_device", "_requires_grad", "_grad", "_version_counter",
        "_pending", "_incoming", "_is_leaf", "_ptr", "_numel", "_shape", "_clean_version",
        "_finite_version", "_known_item", "__weakref__",
    )
    # Every Tensor here may be written in place: device storage always, and
    # host arrays through NumPy, which refuses writes to read-only arrays by
    # itself.  The reference's read-only Tensors (expand views, read-only
    # arrays; tensor.py:348,1012) do not exist, so the flag is a class
    # constant that no instance can change, and the per-step paths do not
    # test it.
    _writable = True

    def __init__(self, data: object, dtype: object = None, requires_grad: builtins.bool = False, *, device=None):
        resolved = _resolve_dtype(data, dtype)
        target = _device_of(data) if device is None else Device(device)
        self._initialize(_make_storage(data, resolved, target), requires_grad, dtype=resolved)

    def _initialize(self, storage, requires_grad: builtins.bool, version_counter: _VersionCounter | None = None,
                    dtype: DType | None = None):
        """Adopt `storage` without a copy: a C-contiguous NumPy array (bfloat16
        as uint16 bits, with ``dtype=bfloat16``), a DeviceArray, or another
        framework's contiguous device array (wrapped)."""
        if isinstance(storage, np.ndarray):
            if not storage.flags.c_contiguous:
                raise TypeError("Tensor storage must be a contiguous array.")
            kind = from_numpy_dtype(storage.dtype) if dtype is None else normalize_dtype(dtype)
            expected = np.dtype(np.uint16) if kind is bfloat16 else kind.numpy_dtype
            if storage.dtype != expected:
                raise TypeError(f"{kind.name} host storage must be a {expected.name} array, got {storage.dtype.name}.")
            self._device = _CPU
            self._ptr = None
            self._numel = storage.size
        else:
            try:
                storage = DeviceArray.wrap(storage)
            except ValueError as error:
                raise TypeError(f"Tensor storage must be a contiguous array: {error}") from None
            kind = storage.dtype
            if dtype is not None and normalize_dtype(dtype) is not kind:
                raise TypeError(f"Storage of dtype {kind.name} cannot back a {normalize_dtype(dtype).name} Tensor.")
            self._device = storage.device
            self._ptr = storage.data_ptr()
            self._numel = storage.numel()
        self._storage = storage
        self._shape = tuple(storage.shape)     # storage is fixed for the Tensor's life
        self._dtype = kind
        if requires_grad and not self._dtype.can_require_grad:
            raise TypeError(f"Only floating Tensors can require gradients, got {self._dtype.name}.")
        self._requires_grad = requires_grad
        self._grad = None
        self._version_counter = version_counter if version_counter is not None else _VersionCounter()
        self._pending = None
        self._incoming = None
        self._is_leaf = True
        self._clean_version = None      # version at which a state buffer was last known nonnegative
        self._finite_version = None     # version at which GradScaler last knew the gradient's finiteness
        self._known_item = None         # (value, version): the host knows the value this device scalar was filled with

    @classmethod
    def _from_storage(cls, storage, requires_grad: builtins.bool = False, version_counter=None,
                      dtype: DType | None = None) -> "Tensor":
        instance = cls.__new__(cls)
        Tensor._initialize(instance, storage, requires_grad, version_counter, dtype)
        return instance

    # ---- storage access --------------------------------------------------------------
    @property
    def _data(self):
        if self._pending is not None or self._incoming is not None:
            self._materialize()
        return self._storage

    def _materialize(self) -> None:
        """Write a deferred accumulation, then a pending gradient transform,
        back into storage."""
        incoming = self._incoming
        if incoming is not None:
            check_addends([self])
            self._incoming = None
            from .backends import get_backend
            get_backend(self).accumulate_tensors([self], [incoming[0]], assign=False)
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
        return self._shape

    @property
    def ndim(self) -> int:
        return len(self._shape)

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
        with _requires_grad_lock:            # no increment lost to another thread's
            _requires_grad_changes.value += 1

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
        source = value._data if isinstance(value, Tensor) else value
        self._pending = None
        self._incoming = None
        if isinstance(self._storage, DeviceArray):
            _assign_device(self._storage, source, self._dtype)
        else:
            _assign_host(self._storage, source, self._dtype, value._dtype if isinstance(value, Tensor) else None)
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
        host = storage.download() if isinstance(storage, DeviceArray) else storage.copy()
        return _values(host, self._dtype)

    def bits(self) -> np.ndarray:
        """Host copy of the raw bit patterns (uint16 for 16-bit types)."""
        reject_during_capture("Host Tensor reads")
        storage = self._data
        if isinstance(storage, DeviceArray):
            return storage.raw_bits()
        return storage.view(_UNSIGNED[self._dtype.itemsize]).copy()

    def item(self):
        reject_during_capture("Host Tensor reads")
        if self.size != 1:
            raise ValueError(f"item() requires exactly one element, got {self.size}.")
        # A device scalar filled from a host value (the norm clip_grad_norm_
        # returns) and not written since: the same value without a device
        # round trip.  Every write through this package bumps the version.
        known = self._known_item
        if known is not None and known[1] == self._version_counter.value:
            return known[0]
        return self.numpy().reshape(()).item()

    def detach(self) -> "Tensor":
        return Tensor._from_storage(self._data, False, self._version_counter, self._dtype)

    def clone(self) -> "Tensor":
        return Tensor._from_storage(self._data.clone() if isinstance(self._data, DeviceArray) else self._data.copy(),
                                    False, dtype=self._dtype)

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


__all__ = ["Tensor", "Parameter", "tensor", "no_grad", "enable_grad", "is_grad_enabled", "GradTransform",
           "check_addends"]
