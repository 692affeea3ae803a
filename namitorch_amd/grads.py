"""Gradient producer edges of the optimizer step.

``accumulate_grads(parameters, gradients)`` is ``Tensor._accumulate_grad``
(namitorch/tensor.py:443-450 over autograd.accumulate_gradient,
autograd.py:198-205) for many leaves at once: one device launch per
(stored dtype, incoming dtype) instead of one NumPy/CuPy expression per
leaf.  A leaf without a gradient receives a new gradient Tensor holding the
incoming values cast to its dtype; a leaf with one has the cast values added
in place (a ``copy_``: its version counter advances).  Validation order and
messages are the reference's.  ``Optimizer.zero_grad(set_to_none=False)``
uses ``zero_grads``, one launch per dtype.
"""

from __future__ import annotations

from .array import DeviceArray

from .backends import ensure_same_device, get_backend
from .backends._graph_capture import reject_during_capture
from .tensor import Tensor

_GRADIENT_DTYPES = ("float16", "bfloat16", "float32", "float64")


def _validate(parent: Tensor, gradient, operation: str, exact_dtype: bool = False) -> None:
    """validate_gradient (autograd.py:176-187)."""
    if not isinstance(gradient, Tensor):
        raise RuntimeError(f"{operation} must be a registered backend gradient array.")
    if gradient.shape != parent.shape:
        raise RuntimeError(f"{operation} has invalid gradient shape {gradient.shape}; expected {parent.shape}.")
    if not parent.dtype.can_require_grad or gradient.dtype.value not in _GRADIENT_DTYPES:
        raise RuntimeError(f"{operation} requires supported floating gradients and a floating parent, "
                           f"got {gradient.dtype.value} and {parent.dtype}.")
    ensure_same_device(parent, gradient)
    if exact_dtype and gradient.dtype is not parent.dtype:
        raise RuntimeError(f"{operation} has gradient dtype {gradient.dtype.value}; expected {parent.dtype}.")


def _validate_accumulation(parent: Tensor, gradient) -> None:
    """validate_accumulation (autograd.py:190-195)."""
    _validate(parent, gradient, "Gradient accumulation")
    existing = parent._grad
    if existing is not None:
        _validate(parent, existing, "Stored gradient", exact_dtype=True)
        if existing.requires_grad:
            raise RuntimeError("Stored gradients must be detached from autograd.")


def accumulate_grads(parameters, gradients, *, defer: bool = False) -> None:
    """For each (leaf, incoming gradient): ``leaf.grad`` becomes the incoming
    gradient cast to the leaf's dtype, or has it added in the leaf's dtype.
    Every pair is validated before anything is written.

    ``defer=True`` (the last micro-batch before a step): where the leaf has
    a gradient of the incoming gradient's dtype (float16, bfloat16 or
    float32), the addition is recorded instead of launched, and the step's
    pre-pass and AdamW pass add the incoming values as they read the
    gradient, which saves writing the sum and reading it back.  Any other
    read of the gradient adds first, so every observer sees the accumulated
    values; the version counter advances as for the addition.  The incoming
    gradients must stay unchanged until then (a RuntimeError names a
    violation)."""
    if type(defer) is not bool:
        raise TypeError("accumulate_grads defer must be a Python bool.")
    parameters = list(parameters)
    gradients = list(gradients)
    if len(parameters) != len(gradients):
        raise ValueError("accumulate_grads needs one gradient per parameter.")
    reject_during_capture("In-place Tensor updates")
    for parameter, gradient in zip(parameters, gradients):
        if not isinstance(parameter, Tensor):
            raise TypeError("accumulate_grads requires NamiTorch Tensors.")
        _validate_accumulation(parameter, gradient)
        if parameter._grad is not None:
            parameter._grad._check_inplace()
    # A leaf listed twice accumulates twice, in order: split into rounds in
    # which every leaf appears once (one launch cannot update a leaf twice).
    rounds: list = []
    seen_in: dict = {}
    for parameter, gradient in zip(parameters, gradients):
        index = seen_in.get(id(parameter), -1) + 1
        seen_in[id(parameter)] = index
        if index == len(rounds):
            rounds.append([])
        rounds[index].append((parameter, gradient))
    for members in rounds:
        _accumulate_round(members, defer)


_DEFERRABLE = ("float16", "bfloat16", "float32")


def _deferrable(stored: Tensor, gradient: Tensor) -> bool:
    """The step's kernels can add `gradient` into `stored` as they read it:
    same 16/32-bit dtype, and a 16-byte aligned incoming array (so it never
    breaks the vector path of the stored gradient's plan)."""
    return (gradient._dtype is stored._dtype and stored._dtype.value in _DEFERRABLE and stored._numel > 0
            and gradient is not stored and gradient._ptr is not None and gradient._ptr % 16 == 0
            and gradient._ptr != stored._ptr)


def _accumulate_round(members, defer: bool = False) -> None:
    by_backend: dict = {}
    for parameter, gradient in members:
        by_backend.setdefault(get_backend(parameter), []).append((parameter, gradient))
    for backend, pairs in by_backend.items():
        if getattr(backend, "adamw", None) is None:
            backend._unsupported("Gradient accumulation")
        fresh, existing, deferred = [], [], []
        for parameter, gradient in pairs:
            if gradient._pending is not None or gradient._incoming is not None:
                gradient._materialize()
            stored = parameter._grad
            if stored is None:
                with backend.context():
                    storage = DeviceArray.empty(parameter.shape, parameter.dtype, parameter.device)
                parameter._grad = Tensor._from_storage(storage)
                fresh.append((parameter._grad, gradient))
            else:
                if stored._pending is not None or stored._incoming is not None:
                    stored._materialize()
                if defer and _deferrable(stored, gradient):
                    deferred.append((stored, gradient))
                else:
                    existing.append((stored, gradient))
        if fresh:
            backend.accumulate_tensors([s for s, _ in fresh], [g for _, g in fresh], assign=True)
        if existing:
            backend.accumulate_tensors([s for s, _ in existing], [g for _, g in existing], assign=False)
            for stored, _ in existing:
                stored._version_counter.increment()
        for stored, gradient in deferred:
            stored._incoming = (gradient, gradient._version_counter.value)
            stored._version_counter.increment()


def zero_grads(gradients) -> None:
    """``grad.zero_()`` for every gradient: device gradients in one launch
    per (device, dtype); host gradients through ``Tensor.zero_``."""
    by_backend: dict = {}
    reject_during_capture("In-place Tensor updates")
    for gradient in gradients:
        gradient._check_inplace()
        if gradient.device.type == "cpu":
            gradient.zero_()
            continue
        by_backend.setdefault(get_backend(gradient), []).append(gradient)
    for backend, members in by_backend.items():
        for gradient in members:
            gradient._incoming = None        # overwritten whole: nothing left to add
        backend.zero_tensors(members)
        for gradient in members:
            gradient._pending = None
            gradient._version_counter.increment()


__all__ = ["accumulate_grads", "zero_grads"]
