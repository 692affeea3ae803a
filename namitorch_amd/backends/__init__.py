"""Device-backend registry (mirrors namitorch/backends/__init__.py:12-131).

``get_backend(x)`` returns one backend object per device.  Backend arrays
are NumPy arrays on the host and :class:`namitorch_amd.array.DeviceArray`
on HIP devices (``cuda:N``); device arrays of other frameworks are accepted
wherever a backend array is and are wrapped without a copy.  The HIP backend
carries the reference's optional kernel attribute ``adamw``
(``supports``/``run``, backends/cuda/adamw.py:32-73) plus the multi-tensor
entry points the optimizer step uses.  The CPU backend exists so that
host-side validation and errors behave as in the reference, but it performs
no optimizer arithmetic: this package computes the step only on the MI355X.
"""

from __future__ import annotations

from contextlib import nullcontext
from functools import wraps
from threading import RLock

import numpy as np

from ..array import DeviceArray, is_device_array
from ..device import Device
from ._settings import enable_fused_kernels, fused_kernels_enabled

_lock = RLock()
_backends: dict = {}
_CPU = Device("cpu")


class CPUBackend:
    """Host backend (backends/cpu.py): NumPy arrays; validation only, every
    optimizer compute request raises."""

    device = _CPU
    array_type = np.ndarray
    module = np
    namespace = np
    adamw = None

    def _unsupported(self, what: str):
        raise RuntimeError(
            f"{what} runs only on HIP devices (cuda:N) in namitorch_amd; "
            "move parameters, gradients and states to the GPU first."
        )

    def context(self, *operands):
        return nullcontext()

    def result(self, value):
        return value

    def ready_for_host(self, array):
        return array

    def array(self, value, dtype=None, copy=True, *, non_blocking=False):
        from ..dtype import normalize_dtype
        from ..tensor import _host_array
        if isinstance(value, np.ndarray) and not copy and (dtype is None or np.dtype(value.dtype) == np.dtype(normalize_dtype(dtype).numpy_dtype)):
            return value
        kind = None if dtype is None else normalize_dtype(dtype)
        if kind is None:
            return np.array(value, copy=True)
        return _host_array(value, kind)

    def item(self, array):
        return array.item()

    def to_numpy(self, array):
        return np.asarray(array)

    def writable(self, array):
        return bool(getattr(array, "flags", None) is None or array.flags.writeable)

    def readonly(self, array):
        view = np.asarray(array).view()
        view.flags.writeable = False
        return view

    def apply_grad_transform(self, tensors, transform):
        self._unsupported("Gradient unscale/clip")

    def scalar_arithmetic(self, tensor, operand, op, dtype, ctrl=None):
        self._unsupported("Tensor arithmetic")

    def __repr__(self):
        return "CPUBackend()"


def is_array(value) -> bool:
    """A backend array: a NumPy array or a (wrappable) device array."""
    return isinstance(value, (np.ndarray, DeviceArray)) or is_device_array(value)


def array_device(value) -> Device:
    if isinstance(value, np.ndarray):
        return _CPU
    if isinstance(value, DeviceArray):
        return value.device
    if is_device_array(value):
        return DeviceArray.wrap(value).device
    raise TypeError(f"Tensor storage must be a registered backend array, got {type(value).__name__}.")


def get_backend(value=None):
    """Backend of a Tensor, a backend array, a Device or a device string."""
    if value is None or isinstance(value, (np.generic, bool, int, float)):
        target = _CPU
    elif isinstance(value, (str, Device)):
        target = Device(value)
    elif isinstance(getattr(value, "device", None), Device) and hasattr(value, "_storage"):
        target = value.device
    elif is_array(value):
        target = array_device(value)
    else:
        raise TypeError("Expected a Tensor, backend array or Device.")
    backend = _backends.get(target)
    if backend is not None:
        return backend
    with _lock:
        if target not in _backends:
            if target.type == "cpu":
                _backends[target] = CPUBackend()
            else:
                from .hip import HIPBackend
                _backends[target] = HIPBackend(target)
        return _backends[target]


def namespace(value=None):
    """The array namespace of `value`'s backend (backends/__init__.py:79-80):
    NumPy on the host, ``HIPNamespace`` on a HIP device."""
    return get_backend(value).namespace


def ensure_same_device(*values, _active=None):
    active = set() if _active is None else _active
    devices = []
    for value in values:
        if value is None:
            continue
        if isinstance(value, (tuple, list)):
            if id(value) in active:
                raise ValueError("Operand sequences cannot contain cycles.")
            active.add(id(value))
            nested = ensure_same_device(*value, _active=active)
            active.remove(id(value))
            if nested is not None:
                devices.append(nested)
        elif isinstance(getattr(value, "device", None), Device) and hasattr(value, "_storage"):
            devices.append(value.device)
        elif isinstance(value, (np.ndarray, DeviceArray)) or is_device_array(value):
            devices.append(array_device(value))
    if devices and any(value != devices[0] for value in devices[1:]):
        raise RuntimeError(f"Operands are on different devices: {', '.join(map(str, devices))}; use an explicit .to() transfer.")
    return devices[0] if devices else None


def same_device(function):
    @wraps(function)
    def checked(*args, **kwargs):
        target = ensure_same_device(*args, *kwargs.values())
        backend = get_backend(target)
        with backend.context(args, kwargs):
            return backend.result(function(*args, **kwargs))
    return checked


def transfer(array, target, dtype=None, copy=True, *, non_blocking=False):
    """Copy a backend array to `target`'s device (backends/__init__.py:121-128)."""
    if type(copy) is not bool or type(non_blocking) is not bool:
        raise TypeError("Transfer copy and non_blocking arguments must be Python bools.")
    source = get_backend(array)
    destination = get_backend(target)
    if source.device.type != destination.device.type and destination.device.type == "cpu":
        array = source.to_numpy(array)
    return destination.array(array, dtype=dtype, copy=copy, non_blocking=non_blocking)


def writable(array) -> bool:
    return get_backend(array).writable(array)


def readonly(array):
    return get_backend(array).readonly(array)


__all__ = ["get_backend", "namespace", "ensure_same_device", "same_device", "transfer", "is_array", "array_device",
           "enable_fused_kernels", "fused_kernels_enabled", "CPUBackend"]
