"""Device-backend registry (mirrors namitorch/backends/__init__.py:12-131).

``get_backend(x)`` returns one backend object per device.  The HIP backend
(``cuda:N`` devices) carries the reference's optional kernel attribute
``adamw`` (``supports``/``run``, backends/cuda/adamw.py:32-73) plus the
multi-tensor entry points the optimizer step uses.  The CPU backend exists
so that host-side validation and errors behave as in the reference, but it
performs no optimizer arithmetic: this package computes the step only on
the MI355X.
"""

from __future__ import annotations

from functools import wraps
from threading import RLock

import torch

from ..device import Device
from ._settings import enable_fused_kernels, fused_kernels_enabled

_lock = RLock()
_backends: dict = {}


class CPUBackend:
    """Host backend: validation only; every compute request raises."""

    device = Device("cpu")
    adamw = None

    def _unsupported(self, what: str):
        raise RuntimeError(
            f"{what} runs only on HIP devices (cuda:N) in namitorch_amd; "
            "move parameters, gradients and states to the GPU first."
        )

    def context(self, *operands):
        from contextlib import nullcontext
        return nullcontext()

    def result(self, value):
        return value

    def item(self, array):
        return array.item()

    def writable(self, array):
        return True

    def apply_grad_transform(self, tensors, transform):
        self._unsupported("Gradient unscale/clip")

    def scalar_arithmetic(self, tensor, operand, op, dtype, ctrl=None):
        self._unsupported("Tensor arithmetic")

    def __repr__(self):
        return "CPUBackend()"


def get_backend(value=None):
    """Backend of a Tensor, a torch storage array, a Device or a device string."""
    if value is None:
        target = Device("cpu")
    elif isinstance(value, (str, Device)):
        target = Device(value)
    elif isinstance(value, torch.Tensor):
        target = Device("cpu") if value.device.type == "cpu" else Device("cuda", value.device.index)
    else:
        device = getattr(value, "device", None)
        if not isinstance(device, Device):
            raise TypeError("Expected a Tensor, backend array or Device.")
        target = device
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


def is_array(value) -> bool:
    return isinstance(value, torch.Tensor)


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
        elif isinstance(value, torch.Tensor):
            devices.append(get_backend(value).device)
        elif isinstance(getattr(value, "device", None), Device) and hasattr(value, "_storage"):
            devices.append(value.device)
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


def writable(array) -> bool:
    return True


__all__ = ["get_backend", "ensure_same_device", "same_device", "enable_fused_kernels", "fused_kernels_enabled", "CPUBackend"]
