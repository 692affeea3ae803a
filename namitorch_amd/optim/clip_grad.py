"""Gradient norm and clipping (namitorch/optim/clip_grad.py) on the MI355X.

``clip_grad_norm_``/``get_grad_norm`` keep the reference's argument checks,
errors and return value (a 0-d float64 Tensor on the gradients' device).
The norm follows ``_total_norm`` (clip_grad.py:63-79): a non-finite or zero
max-abs prescale is itself the result (and the result for norm_type=inf);
otherwise the p-norm in float64.  For p = 2 the device reduces sum(g*g) in
float64 in one pass: squares of float32/float16/bfloat16 values cannot
overflow or underflow float64, and float64 gradients take the reference's
prescaled form with a second pass whenever max|g| lies outside
[2**-480, 2**480].  The norm therefore agrees with NumPy's to a few float64
ulps rather than bit for bit: NumPy sums the prescaled squares pairwise and
takes ``power(total, 0.5)``, whose last bit depends on the host (SVML's pow
on AVX-512 CPUs, libm's elsewhere), so no device formula can match it on
every host.  Other p use the prescaled form with a second pass.  The
reduction order is fixed, so the result is deterministic.

Clipping multiplies each gradient by ``max_norm / (norm + 1e-6)`` in
float64 and rounds once to the gradient dtype (clip_grad.py:106-111).  The
rewrite is recorded on the gradients (see ``GradTransform``) and fused into
the next kernel that reads them.  When nothing is pending on the gradients
and ``error_if_nonfinite`` is False, the norm, the ``coefficient < 1``
decision and the coefficient stay on the device (``_clip_on_device``): the
call queues two kernels and returns without waiting, and the AdamW pass
that follows reads the decision from the device.  ``get_grad_norm`` takes
the same device path (``_norm_on_device``) and records nothing on the
gradients; ``.item()`` on either result waits for it.
"""

from __future__ import annotations

import ctypes
import math
from numbers import Real
from itertools import repeat
from operator import attrgetter, eq, is_

import numpy as np

from .. import _native, runtime
from ..array import DeviceArray
from ..backends import ensure_same_device, get_backend
from ..backends._graph_capture import reject_during_capture
from ..dtype import float64
from ..tensor import GradTransform, Tensor, no_grad

_NORM_EPS = 1e-6
# max|g| range in which the direct float64 sum of squares neither overflows
# nor loses small terms (the device's NT_NORM_POW_GUARD uses the same bounds).
_DIRECT_L2_LOW = 2.0 ** -480
_DIRECT_L2_HIGH = 2.0 ** 480


def _nonnegative(value: object, name: str) -> float:
    if isinstance(value, (bool, np.bool_)) or not isinstance(value, Real):
        raise TypeError(f"{name} must be a finite nonnegative real scalar.")
    try:
        value = float(value)
    except OverflowError:
        raise ValueError(f"{name} must be finite.") from None
    if not math.isfinite(value) or value < 0:
        raise ValueError(f"{name} must be finite and nonnegative.")
    return value


def _norm_type(value: object) -> float:
    if isinstance(value, (bool, np.bool_)) or not isinstance(value, Real):
        raise TypeError("norm_type must be a positive real scalar or positive infinity.")
    try:
        value = float(value)
    except OverflowError:
        raise ValueError("norm_type is outside the supported range.") from None
    if math.isnan(value) or value <= 0:
        raise ValueError("norm_type must be positive or positive infinity.")
    return value


_GRAD_OF = attrgetter("_grad")
_DEVICE_OF = attrgetter("_device")
_SHAPE_OF = attrgetter("_shape")
_FLOATING_OF = attrgetter("_dtype._floating")


def _gradients_bulk(parameters) -> list[Tensor] | None:
    """``_gradients`` for the common case, in C-level passes: every entry a
    Tensor whose gradient is a distinct floating Tensor of its shape on its
    (identical) Device object.  None when anything else holds, so that the
    per-parameter loop skips, deduplicates or raises exactly as the
    reference does."""
    if not all(map(isinstance, parameters, repeat(Tensor))):
        return None
    gradients = list(map(_GRAD_OF, parameters))
    if (not all(map(isinstance, gradients, repeat(Tensor))) or not all(map(_FLOATING_OF, gradients))
            or not all(map(is_, map(_DEVICE_OF, gradients), map(_DEVICE_OF, parameters)))
            or not all(map(eq, map(_SHAPE_OF, gradients), map(_SHAPE_OF, parameters)))
            or len(set(map(id, gradients))) != len(gradients)):
        return None
    return gradients


def _gradients(parameters) -> list[Tensor]:
    if isinstance(parameters, Tensor):
        parameters = (parameters,)
    if isinstance(parameters, (dict, str, bytes, set, frozenset)):
        raise TypeError("parameters must be a Tensor or an ordered iterable of Tensors.")
    if type(parameters) in (list, tuple):
        gradients = _gradients_bulk(parameters)
        if gradients is not None:
            return gradients
    try:
        parameters = iter(parameters)
    except TypeError:
        raise TypeError("parameters must be a Tensor or an ordered iterable of Tensors.") from None
    gradients = []
    seen = set()
    for parameter in parameters:
        if not isinstance(parameter, Tensor):
            raise TypeError("parameters must contain only NamiTorch Tensors.")
        gradient = parameter.grad
        if gradient is None or id(gradient) in seen:
            continue
        if not isinstance(gradient, Tensor) or not gradient.dtype.is_floating_point:
            raise TypeError("Gradients must be floating NamiTorch Tensors.")
        if gradient.shape != parameter.shape:
            raise ValueError(f"Gradient shape {gradient.shape} does not match parameter shape {parameter.shape}.")
        ensure_same_device(parameter, gradient)
        seen.add(id(gradient))
        gradients.append(gradient)
    return gradients


class GradStats:
    """float64 sum of squares, max |g| and non-finite flags of a gradient set."""

    __slots__ = ("sumsq", "amax", "has_nan", "has_inf")

    def __init__(self, sumsq=0.0, amax=0.0, has_nan=False, has_inf=False):
        self.sumsq, self.amax, self.has_nan, self.has_inf = sumsq, amax, has_nan, has_inf

    def merge(self, other: "GradStats") -> None:
        self.sumsq += other.sumsq
        self.amax = max(self.amax, other.amax)
        self.has_nan |= other.has_nan
        self.has_inf |= other.has_inf

    @property
    def finite(self) -> bool:
        return not (self.has_nan or self.has_inf)

    def prescale(self) -> float:
        """The reference's max-abs prescale including NaN/inf propagation."""
        if self.has_nan:
            return math.nan
        if self.has_inf:
            return math.inf
        return self.amax


# Statistics of the last device pre-pass, reused by clip_grad_norm_ when it
# sees the same gradients at the same versions with the same pending
# transform: at most one entry, (snapshot, stats) under the key "last".
_last_stats: dict = {}


_PENDING = attrgetter("_pending")
_VERSION_VALUE = attrgetter("_version_counter.value")
_FINITE_VERSION = attrgetter("_finite_version")
_COUNTER = attrgetter("_version_counter")
_VALUE_OF = attrgetter("value")


def _stats_snapshot(gradients) -> tuple:
    """The gradients (held, so their identities cannot be reused), the set
    of their identities, their version counters with the values they hold,
    and their pending transforms."""
    held = tuple(gradients)
    counters = tuple(map(_COUNTER, held))
    return held, frozenset(map(id, held)), counters, tuple(map(_VALUE_OF, counters)), tuple(map(_PENDING, held))


def _remember_stats(snapshot: tuple, stats: GradStats) -> None:
    """Cache `stats` with the ``_stats_snapshot`` taken when the pre-pass was
    queued, unless a version counter has moved since the snapshot (a settled
    device step may lower one, after which the snapshot's value could come
    back with other contents)."""
    _last_stats.clear()
    held, ids, counters, versions, pendings = snapshot
    if tuple(map(_VALUE_OF, counters)) == versions:
        _last_stats["last"] = (snapshot, stats)


def _cached_stats(gradients) -> GradStats | None:
    """The cached statistics when `gradients` are the cached set (in any
    order) at the same versions with the same pending transforms."""
    entry = _last_stats.get("last")
    if entry is None:
        return None
    (held, ids, counters, versions, pendings), stats = entry
    if (len(gradients) != len(held) or frozenset(map(id, gradients)) != ids
            or tuple(map(_VALUE_OF, counters)) != versions or not all(map(is_, map(_PENDING, held), pendings))):
        return None
    return stats


_DEVICE = attrgetter("_device")
_DTYPE = attrgetter("_dtype")


def _device_groups(gradients) -> dict:
    """Gradients grouped by (backend, dtype), in order."""
    if gradients:
        # Common case: one device and one dtype, checked by identity in
        # C-level passes (Tensors share one Device object per device, and
        # dtypes are singletons).
        first = gradients[0]
        if (all(map(is_, map(_DEVICE, gradients), repeat(first._device)))
                and all(map(is_, map(_DTYPE, gradients), repeat(first._dtype)))):
            return {(get_backend(first), first._dtype): list(gradients)}
    groups: dict = {}
    for gradient in gradients:
        groups.setdefault((get_backend(gradient), gradient.dtype), []).append(gradient)
    return groups


def grad_stats(gradients, norm_type: float = 2.0, remember: bool = True) -> tuple[GradStats, dict]:
    """Run the device pre-pass over `gradients` (with their deferred
    accumulations and pending unscale) and return the merged statistics;
    also, per (backend, dtype) group, its members, control block and scale."""
    stats = GradStats()
    blocks = {}
    launched = []
    for (backend, dtype), members in _device_groups(gradients).items():
        if backend.adamw is None:
            backend._unsupported("Gradient norms")
        transforms = {gradient._pending for gradient in members}
        # The pre-pass applies at most one host-known unscale.  Anything else
        # (mixed transforms, a pending clip, or a fused step's device-decided
        # unscale/clip) is written back first, so the statistics are those of
        # the values the reference would hold.
        if len(transforms) > 1 or any(t is not None and (t.clip is not None or t.device is not None)
                                      for t in transforms):
            for gradient in members:
                gradient._materialize()
            scale = None
        else:
            transform = next(iter(transforms))
            scale = None if transform is None else transform.scale
        plan = backend.grad_plan(members, dtype, incoming=True)
        block = backend.empty_ctrl()                     # written whole by the finalize
        backend.grad_prepass(plan, scale)
        # The finalize also writes the block to a host mirror, which the host
        # waits for below (no copy back, nothing recorded on the stream).
        mirror = runtime.take_mirror()
        try:
            backend.grad_finalize(plan, block.data_ptr(), norm_type=2.0, carry_ptr=backend.neutral_ctrl().data_ptr(),
                                  mirror=mirror)
        except BaseException:
            runtime.give_mirror(mirror, launched=False)
            raise
        launched.append((backend, dtype, members, block, scale, mirror, backend.stream()))
    # Host work that does not need the results runs while the device works.
    snapshot = _stats_snapshot(gradients) if remember else None
    for backend, dtype, members, block, scale, mirror, stream in launched:
        if not mirror.ready:
            with backend.context():
                _native.call("nt_mirror_wait", ctypes.addressof(mirror), stream)
        ctrl = _native.AmpCtrl.from_buffer_copy(mirror)
        runtime.give_mirror(mirror)
        stats.merge(GradStats(ctrl.sumsq, ctrl.amax, bool(ctrl.has_nan), bool(ctrl.found_inf and not ctrl.has_nan)))
        blocks[(backend, dtype)] = (members, block, scale)
    if remember:
        _remember_stats(snapshot, stats)
    return stats, blocks


def _pow_total(blocks, amax: float, order: float) -> float:
    """Sum over gradients of (|g|/amax)^p in float64 (clip_grad.py:73-76)."""
    total = 0.0
    for (backend, dtype), (members, block, scale) in blocks.items():
        plan = backend.grad_plan(members, dtype)         # deferred accumulations written back first
        ctrl = backend.read_ctrl(block)
        ctrl.amax = amax
        with backend.context():
            _native.call("nt_memcpy_h2d", block.data_ptr(), ctypes.addressof(ctrl), ctypes.sizeof(ctrl), backend.stream())
        backend.grad_norm_pow(plan, block.data_ptr(), order, -1.0, scale)
        total += backend.read_ctrl(block).sumsq
    return total


def _total_norm(gradients: list[Tensor], norm_type: float) -> float:
    reject_during_capture("Host Tensor reads")          # the norm comes back to the host
    if not gradients:
        return 0.0
    cached = _cached_stats(gradients)
    if cached is not None and (norm_type == 2 or math.isinf(norm_type)):
        stats, blocks = cached, None
    else:
        stats, blocks = grad_stats(gradients)
    scale = stats.prescale()
    if not math.isfinite(scale) or scale == 0 or math.isinf(norm_type):
        return scale
    if norm_type == 2 and _DIRECT_L2_LOW <= scale <= _DIRECT_L2_HIGH:
        return math.sqrt(stats.sumsq)
    # Other p, and p = 2 where squares of float64 gradients may leave the
    # float64 range: the reference's prescaled sum (clip_grad.py:73-78).
    if blocks is None:
        stats, blocks = grad_stats(gradients)
    total = _pow_total(blocks, scale, norm_type)
    with np.errstate(over="ignore", divide="ignore", invalid="ignore", under="ignore"):
        result = float(np.float64(scale) * np.power(np.float64(total), 1 / norm_type))
        if not math.isfinite(result):
            result = float(np.exp(np.log(np.float64(scale)) + np.log(np.float64(total)) / norm_type))
    return result


def _norm_tensor(norm: float, gradients) -> Tensor:
    device = gradients[0].device if gradients else None
    if device is None or device.type == "cpu":
        return Tensor._from_storage(np.array(norm, dtype=np.float64), False)
    # A fill with the value's bits as a kernel argument: no host-to-device copy to wait for.
    storage = DeviceArray.empty((), float64, device)
    value = np.float64(norm)
    storage.fill_bits(int(value.view(np.uint64)))
    result = Tensor._from_storage(storage, False)
    result._known_item = (value.item(), result._version_counter.value)   # .item() needs no device read
    return result


def get_grad_norm(parameters, norm_type: float = 2) -> Tensor:
    order = _norm_type(norm_type)
    gradients = _gradients(parameters)
    launched = _norm_on_device(gradients, order, -1.0)
    if launched is not None:
        return Tensor._from_storage(launched[2], False)       # read on the device; .item() waits
    return _norm_tensor(_total_norm(gradients, order), gradients)


_VALUE = attrgetter("value")
# Device-decided clips not yet settled by an optimizer step or a version
# read: past this many, the oldest is settled at the next clip (its finalize
# ran long before), which bounds the host buffers they hold.
_UNSETTLED_LIMIT = 64


def _settle_oldest(pending: list) -> None:
    try:
        oldest = pending[0]
    except IndexError:                    # another thread settled them all meanwhile
        return
    oldest.reconcile()


def _norm_on_device(gradients, order: float, maximum: float, with_mirror: bool = False):
    """Queue the pre-pass and a finalize over `gradients` and a device copy
    of the norm, with no host wait: (backend, control block, 0-d float64
    norm array, host mirror of the block or None), or None when the host
    path must answer.  With `maximum` >= 0 the finalize also takes the clip
    decision by the reference's rule (clip when ``max_norm / (norm + 1e-6)
    < 1``, also for a non-finite norm).  With `with_mirror` the finalize
    also writes the finished block to a ``runtime.take_mirror()``.

    Eligible: norm_type 2 or inf; one device and one float16, bfloat16 or
    float32 gradient dtype (float64 may need the prescaled second pass);
    nothing pending on the gradients; and no cached statistics for them
    (then the host path answers without waiting)."""
    if order != 2.0 and not math.isinf(order):
        return None
    if not gradients or any(map(_PENDING, gradients)):
        return None
    if _cached_stats(gradients) is not None:
        return None
    groups = _device_groups(gradients)
    if len(groups) != 1:
        return None
    (backend, dtype), _ = next(iter(groups.items()))
    if backend.adamw is None or dtype is float64:
        return None
    reject_during_capture("Host Tensor reads")           # as the host path: nothing under capture
    plan = backend.grad_plan(gradients, dtype, incoming=True)
    neutral = backend.neutral_ctrl()
    block = backend.empty_ctrl()                         # written whole by the finalize
    backend.grad_prepass(plan, None, neutral.data_ptr())
    mirror = runtime.take_mirror() if with_mirror else None
    backend.grad_finalize(plan, block.data_ptr(), order, maximum, 0, carry_ptr=neutral.data_ptr(), mirror=mirror)
    return backend, block, backend.ctrl_norm(block), mirror


def _clip_on_device(gradients, maximum: float, order: float) -> Tensor | None:
    """``clip_grad_norm_`` with the norm, the clip decision and the
    coefficient left on the device, so the host does not wait
    (``_norm_on_device``).  The gradients get a device-decided clip
    transform that the next kernel reading them applies (the AdamW pass, or
    the write-back when a gradient is read), and the result is the device's
    norm.  The reference's version bump happens only when the coefficient is
    below 1: it is taken optimistically and undone when the step is settled.

    None (the host path decides) unless no host decision of the reference
    can raise or differ: ``_norm_on_device``'s conditions.  (The rewrite
    itself cannot fail: every Tensor here is writable.)
    """
    launched = _norm_on_device(gradients, order, maximum, with_mirror=True)
    if launched is None:
        return None
    backend, block, norm, mirror = launched
    from ..amp import DeviceStep                         # the amp module imports this one
    from ..tensor import _unsettled_steps
    clip_bumps: list = []
    device_step = DeviceStep(backend, block, unscale=False, honor_skip=False, clip_bumps=clip_bumps, mirror=mirror)
    device_step.clip_requested = True
    device_step.capture()
    transform = GradTransform(device=device_step)
    counters = tuple(map(_COUNTER, gradients))
    kept = tuple(map(eq, map(_FINITE_VERSION, gradients), map(_VALUE, counters)))
    for gradient, counter, keep in zip(gradients, counters, kept):
        gradient._pending = transform
        counter.value += 1
        if keep:
            gradient._finite_version = counter.value
    clip_bumps.extend(zip(gradients, map(_VALUE, counters)))
    if len(_unsettled_steps) >= _UNSETTLED_LIMIT:
        _settle_oldest(_unsettled_steps)
    _unsettled_steps.append(device_step)                 # version reads settle it first
    return Tensor._from_storage(norm, False)


def clip_grad_norm_(parameters, max_norm: float, norm_type: float = 2, error_if_nonfinite: bool = False) -> Tensor:
    maximum = _nonnegative(max_norm, "max_norm")
    order = _norm_type(norm_type)
    if type(error_if_nonfinite) is not bool:
        raise TypeError("error_if_nonfinite must be a Python bool.")
    gradients = _gradients(parameters)
    if not error_if_nonfinite:
        result = _clip_on_device(gradients, maximum, order)
        if result is not None:
            return result
    norm = _total_norm(gradients, order)
    if error_if_nonfinite and not math.isfinite(norm):
        raise RuntimeError(f"Cannot clip gradients with nonfinite total norm {np.asarray(norm, dtype=np.float64)}.")
    with np.errstate(invalid="ignore", divide="ignore"):
        coefficient = float(np.divide(np.float64(maximum), np.add(np.float64(norm), _NORM_EPS)))
    if coefficient < 1:
        # One shared clip transform per prior pending transform object (usually
        # the single unscale transform of unscale_, or none), found by
        # identity; the dict keeps each base alive, so identities stay unique.
        clipped: dict = {}
        unscaled_none = GradTransform()
        reject_during_capture("In-place Tensor updates")
        pendings = tuple(map(_PENDING, gradients))
        if pendings and all(map(is_, pendings, repeat(pendings[0]))) and (
                pendings[0] is None or (pendings[0].clip is None and pendings[0].device is None)):
            # Common case, one shared prior transform (or none): the loop below
            # with C-level passes.  Inside no_grad the in-place check cannot
            # fail (only writability could, and every Tensor is writable).
            base = unscaled_none if pendings[0] is None else pendings[0]
            transform = base.then_clip(coefficient)
            keep = tuple(map(eq, map(_FINITE_VERSION, gradients), map(_VERSION_VALUE, gradients)))
            for gradient, counter, kept in zip(gradients, map(_COUNTER, gradients), keep):
                gradient._pending = transform
                counter.value += 1
                if kept:
                    gradient._finite_version = counter.value
            return _norm_tensor(norm, gradients)
        with no_grad():
            for gradient in gradients:
                gradient._check_inplace()
                pending = gradient._pending
                if pending is not None and (pending.clip is not None or pending.device is not None):
                    gradient._materialize()
                    pending = None
                keep_finite = gradient._finite_version is not None and gradient._finite_version == gradient._version_counter.value
                base = unscaled_none if pending is None else pending
                shared = clipped.get(id(base))
                if shared is None:
                    shared = clipped[id(base)] = (base, base.then_clip(coefficient))
                gradient._pending = shared[1]
                gradient._version_counter.increment()
                if keep_finite:
                    gradient._finite_version = gradient._version_counter.value
    return _norm_tensor(norm, gradients)


def clip_grad_value_(parameters, clip_value: float) -> None:
    bound = _nonnegative(clip_value, "clip_value")
    _gradients(parameters)
    raise NotImplementedError(
        f"clip_grad_value_ (bound {bound}) is outside the optimizer-step path this package accelerates."
    )


__all__ = ["get_grad_norm", "clip_grad_norm_", "clip_grad_value_", "grad_stats", "GradStats"]
