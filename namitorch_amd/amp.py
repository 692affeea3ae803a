"""GradScaler (namitorch/amp.py:78-259) on the MI355X.

The state machine — scale range and rounding to float32 (``_scale_value``,
amp.py:114-119), the call-order checks and messages (127-234) and the
growth/backoff update (219-234) — is the reference's.  The per-gradient
work is not: ``unscale_`` records ``g <- to_grad_dtype(f32(g) / scale)`` on
every gradient as a pending transform and runs one device pre-pass per
(device, dtype) group that checks finiteness of the unscaled values and
accumulates the float64 norm statistics ``clip_grad_norm_`` reuses.
``step`` re-checks finiteness on the device only when a gradient was
written by something other than ``unscale_`` and ``clip_grad_norm_`` since
(both preserve "all finite"); the AdamW pass then consumes the pending
unscale/clip in the same kernel that reads the gradients.
"""

from __future__ import annotations

import ctypes
import math
import operator
from collections import deque
from itertools import repeat
from operator import attrgetter, eq, is_, itemgetter
from numbers import Real

import numpy as np

from . import _native, runtime
from .backends import get_backend
from .backends._graph_capture import reject_during_capture
from .dtype import float32, float64, promote_with_scalar
from .optim import clip_grad
from .optim.adam import Adam, AdamW
from .optim.clip_grad import _device_groups, _nonnegative, _norm_type, clip_grad_norm_, grad_stats
from .tensor import (GradTransform, _requires_grad_changes, _settle_lock, _unsettled_steps, check_addends,
                     is_grad_enabled)

_REQUIRES = attrgetter("_requires_grad")
_PENDING = attrgetter("_pending")
_COUNTER = attrgetter("_version_counter")
_VALUE = attrgetter("value")
_DTYPE = attrgetter("_dtype")
_FLOATING = attrgetter("_floating")
_FIRST_OF = itemgetter(0)
_SECOND_OF = itemgetter(1)
_PARAMETER_AND_GRADIENT = itemgetter(1, 2)
_THIRD_OF = itemgetter(2)
_FINITE_VERSION = attrgetter("_finite_version")
_VERSION_VALUE = attrgetter("_version_counter.value")
_GRAD = attrgetter("_grad")


class DeviceStep:
    """One iteration whose unscale/finite/clip/skip/scale decisions were taken
    on the device: its control block, the page-locked host mirror that the
    block's last writer fills, and the host-side bookkeeping to undo if the
    step was skipped."""

    def __init__(self, backend, block, unscale: bool, honor_skip: bool, clip_bumps: list, mirror=None):
        self.backend = backend
        self.block = block
        self.unscale = unscale
        self.honor_skip = honor_skip
        self.records: list = []
        self.clip_bumps = clip_bumps          # (gradient, version after the optimistic clip bump)
        # runtime.take_mirror(), passed to the block's last writer (finalize or
        # combine); None: the block is read back with a copy after an event.
        self.mirror = mirror
        self.launched = False                 # a kernel that writes `mirror` was queued
        self._ctrl = None
        self._reconciled = False
        self.scheduler = None                 # advanced at reconciliation iff the step updated
        self.ready = None                     # event on `stream` after the block's last writer, once needed
        self.stream = None
        # fused_step(error_if_nonfinite=True) without a scaler: a non-finite
        # norm skipped the clip and the step on the device; the reference's
        # error is kept here once the outcome is known.
        self.error_if_nonfinite = False
        self.error: RuntimeError | None = None

    def block_for_current_stream(self):
        """The control block, safe to read from work queued next on the
        caller's current stream: a different stream first waits for this
        step's finalize, and the block is kept from reuse until that stream's
        work completes."""
        current = self.backend.stream()
        if self.stream is not None and current != self.stream:
            with self.backend.context():
                _native.call("nt_stream_wait_event", current, self._ready_event().handle)
                self.block.record_stream(current)
        return self.block

    def _ready_event(self):
        """An event on the step's stream after the block's last writer.  It is
        recorded when first needed (another stream reads the block, or the
        host needs the block before its mirror is written), later than the
        writer but never before it: an event on the launch stream is a
        marker that idles the device for several microseconds, so a step
        whose mirror arrives in time records none."""
        if self.ready is None:
            with self.backend.context():
                self.ready = runtime.Event().record(self.stream)
        return self.ready

    def capture(self) -> None:
        """Note the stream the block's last writer was queued on; that
        kernel also fills the host mirror.  Nothing writes the block after
        it.  Without a mirror the block is read back after an event recorded
        here."""
        self.stream = self.backend.stream()
        self.launched = True
        if self.mirror is None:
            self._ready_event()

    def __del__(self):
        # A step dropped before its mirror was read: the mirror returns to
        # the pool, which reuses it once its flag shows the write done.
        try:
            if self.mirror is not None and not _native.shutting_down():
                runtime.give_mirror(self.mirror, self.launched)
                self.mirror = None
        except Exception:
            pass

    def _forget(self) -> None:
        """Leave the list of unsettled steps (every entry of this step).  One
        removal at a time: an entry another thread appends meanwhile stays."""
        while True:
            try:
                _unsettled_steps.remove(self)
            except ValueError:
                return

    def ctrl(self) -> _native.AmpCtrl:
        with _settle_lock:                    # one reader takes the mirror and gives it back
            return self._read_ctrl()

    def _read_ctrl(self) -> _native.AmpCtrl:
        if self._ctrl is None:
            mirror = self.mirror
            if mirror is None:
                self._ready_event().synchronize()      # the block's last writer has completed
                self._ctrl = self.backend.read_ctrl(self.block)
            else:
                if not mirror.ready:
                    with self.backend.context():
                        _native.call("nt_mirror_wait", ctypes.addressof(mirror), self.stream)
                self._ctrl = _native.AmpCtrl.from_buffer_copy(mirror)
                runtime.give_mirror(mirror)
                self.mirror = None
        return self._ctrl

    def reconcile(self) -> None:
        with _settle_lock:                    # the rollback below runs once, on one thread
            self._reconcile()

    def _reconcile(self) -> None:
        if self._reconciled:
            self._forget()                    # settled: never left waiting in the unsettled list
            return
        ctrl = self.ctrl()
        if self.honor_skip and ctrl.skip:
            # The AdamW pass left everything untouched: undo the host bookkeeping.
            for parameter, state, first, second, master, step, bumped, moved in self.records:
                if state.get("step") == step:
                    state["step"] = step - 1
                if bumped:
                    for buffer in (first, second):
                        buffer._version_counter.value -= 1
                        buffer._clean_version = buffer._version_counter.value
                    if moved:
                        parameter._version_counter.value -= 1
                        if master is not None:
                            master._version_counter.value -= 1
        if not ctrl.clip and self.clip_bumps:
            # The clip's one bump is taken back whatever was written since
            # (the reference counts one write per clip actually applied).
            for gradient, _ in self.clip_bumps:
                counter = gradient._version_counter
                counter.value -= 1
                stamp = gradient._finite_version
                if stamp == counter.value + 1:
                    gradient._finite_version = counter.value       # the same contents, renumbered
                elif stamp is not None and stamp >= counter.value:
                    gradient._finite_version = None                # would name other contents later
            # A lowered counter reaches its old values again at the next
            # writes, with other contents: statistics cached under them must
            # not match then.
            clip_grad._last_stats.clear()
        self.records.clear()
        self._reconciled = True
        self._forget()
        scheduler, self.scheduler = self.scheduler, None    # no reference cycle through it once settled
        if scheduler is not None and not (self.honor_skip and ctrl.skip):
            scheduler._advance()              # training/runner.py:252-253: only after an update
        if self.error_if_nonfinite and not math.isfinite(ctrl.norm):
            # optim/clip_grad.py:104-105, with the norm printed as there (a 0-d float64 array)
            self.error = RuntimeError(
                f"Cannot clip gradients with nonfinite total norm {np.asarray(ctrl.norm, dtype=np.float64)}.")

    def raise_error(self) -> None:
        """Settle; raise the deferred ``error_if_nonfinite`` error, if any
        (raised here, it is not raised again by the next fused_step)."""
        if self.error_if_nonfinite:
            self.reconcile()
            if self.error is not None:
                while True:
                    try:
                        _error_watch.remove(self)
                    except ValueError:
                        break
                raise self.error


# Fused steps taken with error_if_nonfinite=True whose error (if any) has not
# been raised yet: the next fused_step raises it before doing anything.
_error_watch: list = []


def _raise_deferred_errors() -> None:
    while True:
        try:
            device_step = _error_watch.pop(0)
        except IndexError:                    # empty, or emptied by another thread
            return
        device_step.raise_error()


class StepResult:
    """Outcome of ``fused_step``; reading a field waits for that step's
    finalize kernel (not for the AdamW pass)."""

    def __init__(self, device_step: DeviceStep | None = None, *, finite=None, updated=None, norm=None, scale=None):
        self._device_step = device_step
        self._eager = (finite, updated, norm, scale)

    def _ctrl(self):
        """The step's control block; raises the deferred error_if_nonfinite
        error of a step whose clip found a non-finite norm."""
        self._device_step.raise_error()
        return self._device_step.ctrl()

    @property
    def finite(self) -> bool:
        if self._device_step is None:
            return self._eager[0]
        return not self._ctrl().found_inf

    @property
    def updated(self) -> bool:
        if self._device_step is None:
            return self._eager[1]
        return not (self._device_step.honor_skip and self._ctrl().skip)

    @property
    def norm(self):
        """Global grad norm (float), or None when no norm was requested."""
        if self._device_step is None:
            return self._eager[2]
        return self._ctrl().norm if self._device_step.clip_requested else None

    @property
    def scale(self) -> float:
        """Loss scale for the next iteration."""
        if self._device_step is None:
            return self._eager[3]
        return float(self._ctrl().scale)

    def synchronize(self) -> "StepResult":
        if self._device_step is not None:
            self._device_step.reconcile()
            self._device_step.raise_error()
        return self


class GradScaler:
    _MIN_SCALE = float(np.finfo(np.float32).tiny)
    _MAX_SCALE = float(np.finfo(np.float32).max)

    def __init__(self, init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5, growth_interval=2000, enabled=True):
        if type(enabled) is not bool:
            raise TypeError("GradScaler enabled must be a Python bool.")
        self._scale = self._scale_value(init_scale)
        self._growth_factor = self._real(growth_factor, "growth_factor")
        self._backoff_factor = self._real(backoff_factor, "backoff_factor")
        if self._growth_factor <= 1:
            raise ValueError("growth_factor must be greater than 1.")
        if not 0 < self._backoff_factor < 1:
            raise ValueError("backoff_factor must be between 0 and 1.")
        if isinstance(growth_interval, (bool, np.bool_)):
            raise TypeError("growth_interval must be a positive integer.")
        self._growth_interval = operator.index(growth_interval)
        if self._growth_interval <= 0:
            raise ValueError("growth_interval must be positive.")
        self._enabled = enabled
        self._growth_tracker = 0
        self._optimizer_states: dict = {}
        self._scale_used = False
        self._device_blocks: dict = {}       # backend -> latest DeviceStep (its block holds the scale)
        self._device_steps: list = []        # fused steps not yet reflected in the host mirror

    @staticmethod
    def _real(value, name):
        if isinstance(value, (bool, np.bool_)) or not isinstance(value, Real):
            raise TypeError(f"{name} must be a finite real number.")
        try:
            result = float(value)
        except OverflowError:
            raise ValueError(f"{name} must be finite.") from None
        if not math.isfinite(result):
            raise ValueError(f"{name} must be finite.")
        return result

    @classmethod
    def _scale_value(cls, value):
        scale = cls._real(value, "scale")
        if not cls._MIN_SCALE <= scale <= cls._MAX_SCALE:
            raise ValueError(f"scale must be between {cls._MIN_SCALE} and {cls._MAX_SCALE}.")
        return float(np.float32(scale))

    def is_enabled(self):
        return self._enabled

    def _reconcile(self) -> None:
        """Bring the host mirror (scale, growth tracker) up to date with the
        device after fused steps; waits for their finalize kernels only."""
        if not self._device_steps:
            return
        for device_step in self._device_steps:
            device_step.reconcile()
        last = self._device_steps[-1].ctrl()
        self._scale = float(last.scale)
        self._growth_tracker = int(last.growth_tracker)
        self._device_steps.clear()

    def get_scale(self):
        self._reconcile()
        return self._scale if self._enabled else 1.0

    def scale(self, loss):
        reject_during_capture("GradScaler")
        dtype = getattr(loss, "dtype", None)
        if not hasattr(dtype, "can_require_grad") or not dtype.can_require_grad or not hasattr(loss, "_storage"):
            raise TypeError("GradScaler.scale requires a floating NamiTorch Tensor.")
        get_backend(loss)
        if not self._enabled:
            return loss
        if self._optimizer_states:
            raise RuntimeError("Call update() before scaling another loss after unscale_ or step.")
        backend = get_backend(loss)
        latest = self._device_blocks.get(backend) if self._device_steps else None
        block = None if latest is None else latest.block_for_current_stream()
        if block is not None:
            # The current scale lives on the device after a fused step; the
            # result dtype is loss * <Python float>'s (amp.py:138), e.g.
            # float32 for a float16 loss.
            result = backend.scalar_arithmetic(loss, 1.0, _native.NT_OP_MUL,
                                               promote_with_scalar(loss.dtype, float32), ctrl=block)
        else:
            result = loss * self._scale
        self._scale_used = True
        return result

    @staticmethod
    def _gradients(optimizer):
        if not callable(getattr(optimizer, "_parameters_with_grad", None)) or not callable(getattr(optimizer, "step", None)):
            raise TypeError("GradScaler requires a NamiTorch optimizer.")
        entries = optimizer._grad_entries() if callable(getattr(optimizer, "_grad_entries", None)) \
            else tuple(optimizer._parameters_with_grad())
        gradients = tuple(map(_PARAMETER_AND_GRADIENT, entries))
        if any(map(_REQUIRES, map(_THIRD_OF, entries))):
            raise RuntimeError("GradScaler requires detached floating gradients.")
        # Parameter dtypes never change: the floating check is skipped while
        # the entries come from the memo (which fixes the parameters) that
        # passed it last.
        attributes = getattr(optimizer, "__dict__", None)
        served = attributes.get("_entries_served") if attributes is not None else None
        if served is None or attributes.get("_floating_checked") is not served:
            if not all(map(_FLOATING, map(_DTYPE, map(_SECOND_OF, entries)))):
                raise RuntimeError("GradScaler requires detached floating gradients.")
            if served is not None:
                attributes["_floating_checked"] = served
        return gradients

    @staticmethod
    def _entry_inputs(optimizer, known=None):
        """What an optimizer's gradient entries are a pure function of
        (``Optimizer._grad_entries``): its registered-parameter cache (a new
        object whenever the groups change), the parameters' requires_grad
        flags and their gradient objects; None for an optimizer without that
        cache.  Returned as (cache, requires_grad change count, flags,
        gradients).  With `known`, an earlier result, the flags are taken
        from it when the cache is the same object and no requires_grad flag
        has changed anywhere since (the count is unchanged)."""
        registered_of = getattr(optimizer, "_registered_parameters", None)
        if not callable(registered_of) or not callable(getattr(optimizer, "_grad_entries", None)):
            return None
        registered = registered_of()
        cache = getattr(optimizer, "__dict__", {}).get("_registered_cache")
        if cache is None:
            return None
        changes = _requires_grad_changes.value
        if known is not None and known[0] is cache and known[1] == changes:
            requires = known[2]
        else:
            requires = tuple(map(_REQUIRES, registered))
        return cache, changes, requires, tuple(map(_GRAD, registered))

    @staticmethod
    def _finite(gradients) -> bool:
        """All elements of all gradients finite (amp.py:152-167), on the device."""
        stats, _ = grad_stats([gradient for _, gradient in gradients])
        return stats.finite

    def unscale_(self, optimizer):
        reject_during_capture("GradScaler")
        if not self._enabled:
            return True
        self._reconcile()
        if not self._scale_used:
            raise RuntimeError("Call scale(loss) and backward before unscale_.")
        identity = id(optimizer)
        if identity in self._optimizer_states:
            raise RuntimeError("unscale_ may be called only once per optimizer between update() calls.")
        gradients = self._gradients(optimizer)
        if not gradients:
            raise RuntimeError("No gradients were found for this optimizer.")
        previous = {id(parameter) for state in self._optimizer_states.values() for parameter, _ in state["gradients"]}
        if previous and any(id(parameter) in previous for parameter, _ in gradients):
            raise RuntimeError("Optimizers cannot share gradients in the same GradScaler iteration.")
        state = {"optimizer": optimizer, "stage": "unscaling", "gradients": gradients, "finite": False,
                 "inputs": self._entry_inputs(optimizer)}
        self._optimizer_states[identity] = state
        transform = GradTransform(scale=self._scale)
        grads = tuple(map(_SECOND_OF, gradients))
        if any(map(_REQUIRES, grads)) and is_grad_enabled():
            for gradient in grads:
                gradient._ensure_inplace_allowed()            # raises the matching error
        if any(map(_PENDING, grads)):
            for gradient in grads:
                if gradient._pending is not None:
                    gradient._materialize()
        counters = tuple(map(_COUNTER, grads))
        for gradient, counter in zip(grads, counters):
            gradient._pending = transform
            counter.value += 1
        # The check below is of these versions; they are stamped before its
        # wait for the device (and restored if it raises).
        stamped = tuple(map(_FINITE_VERSION, grads))
        deque(map(setattr, grads, repeat("_finite_version"), map(_VALUE, counters)), 0)
        try:
            state["finite"] = self._finite(gradients)
        except BaseException:
            deque(map(setattr, grads, repeat("_finite_version"), stamped), 0)
            raise
        state["stage"] = "unscaled"
        return state["finite"]

    def step(self, optimizer):
        reject_during_capture("GradScaler")
        if not self._enabled:
            optimizer.step()
            return True
        identity = id(optimizer)
        if identity not in self._optimizer_states:
            stepped = self._step_on_device(optimizer)
            if stepped is not None:
                return stepped
            self.unscale_(optimizer)
        state = self._optimizer_states[identity]
        if state["stage"] != "unscaled":
            raise RuntimeError("step() may be called only once per optimizer before update().")
        previous = state["gradients"]
        inputs, current = state["inputs"], None
        if inputs is not None:
            # The entries are those of unscale_ when what they are a function
            # of is unchanged (three passes instead of collecting them again).
            now = self._entry_inputs(optimizer, inputs)
            if now is not None and now[0] is inputs[0] and now[2] == inputs[2] and all(map(is_, now[3], inputs[3])):
                current = previous
                grads = tuple(map(_SECOND_OF, current))
                # unscale_ refused gradients that required grad; these are
                # the same objects, so only a flag changed since can matter.
                if now[1] != inputs[1] and any(map(_REQUIRES, grads)):
                    raise RuntimeError("GradScaler requires detached floating gradients.")
        if current is None:
            current = self._gradients(optimizer)
            grads = tuple(map(_SECOND_OF, current))
            if len(current) != len(previous) or not (all(map(is_, map(_FIRST_OF, current), map(_FIRST_OF, previous)))
                                                     and all(map(is_, grads, map(_SECOND_OF, previous)))):
                raise RuntimeError("Optimizer gradients changed after unscale_; clipping must modify the existing gradients in-place.")
        # Finite as checked by unscale_ unless something else wrote a gradient since.
        unchanged = all(map(eq, map(_FINITE_VERSION, grads), map(_VERSION_VALUE, grads)))
        now_finite = state["finite"] if unchanged else self._finite(current)
        state["finite"] = now_finite and state["finite"]
        if state["finite"]:
            state["stage"] = "stepping"
            optimizer.step()
            state["stage"] = "stepped"
            return True
        state["stage"] = "stepped"
        return False

    def _step_on_device(self, optimizer):
        """``step`` without an earlier ``unscale_``, which the reference's
        ``step`` then calls itself (amp.py:194-196).  The unscale, the finite
        check and the AdamW pass are queued together, the pass skipping on
        the device when a gradient is non-finite, and the host waits once,
        for the finalize, after the pass is queued: the device does not idle
        while the host prepares the pass, as it does after ``unscale_``'s
        wait.  Returns the step's bool, or None before any change where the
        host path (``unscale_``, then ``step``) runs instead: an optimizer
        other than this package's Adam/AdamW (subclasses included),
        gradients on several devices or of several dtypes, float64
        gradients.

        The reference calls ``optimizer.step()`` only after a finite
        unscale.  Here it runs first; if it raises, the error is raised only
        when the gradients turn out finite, and otherwise dropped with the
        step reported skipped, as the reference would not have stepped."""
        self._reconcile()
        if not self._scale_used:
            raise RuntimeError("Call scale(loss) and backward before unscale_.")
        if type(optimizer) not in (Adam, AdamW):          # a subclass may read the gradients itself
            return None
        gradients = self._gradients(optimizer)
        if not gradients:
            raise RuntimeError("No gradients were found for this optimizer.")
        previous = {id(parameter) for state in self._optimizer_states.values() for parameter, _ in state["gradients"]}
        if previous and any(id(parameter) in previous for parameter, _ in gradients):
            raise RuntimeError("Optimizers cannot share gradients in the same GradScaler iteration.")
        grads = list(map(_SECOND_OF, gradients))
        groups = _device_groups(grads)
        if len(groups) != 1:
            return None
        (backend, dtype), _ = next(iter(groups.items()))
        if dtype is float64 or backend.adamw is None:
            return None
        state = {"optimizer": optimizer, "stage": "unscaling", "gradients": gradients, "finite": False,
                 "inputs": None}
        self._optimizer_states[id(optimizer)] = state
        # The block the finalize carries from holds the host's scale, which
        # the pre-pass unscales by and the pass reads back as scale_used; no
        # scaler update on the device (update() makes it on the host).
        carry = backend.new_ctrl(self._scale, self._growth_tracker)
        device_step = _queue_decisions(backend, dtype, grads, carry, amp=True, maximum=None, order=2.0, flags=0,
                                       growth=self._growth_factor, backoff=self._backoff_factor,
                                       interval=self._growth_interval, honor_skip=True)
        state["stage"] = "stepping"
        try:
            optimizer.step()                              # the AdamW pass reads the control block
        except Exception:
            _unsettled_steps.append(device_step)
            state["finite"] = not device_step.ctrl().found_inf
            device_step.reconcile()
            if state["finite"]:
                raise
            state["stage"] = "stepped"
            return False
        _unsettled_steps.append(device_step)              # version reads settle it first
        state["finite"] = not device_step.ctrl().found_inf     # waits for the finalize, not the pass
        device_step.reconcile()
        state["stage"] = "stepped"
        return state["finite"]

    def update(self):
        reject_during_capture("GradScaler")
        if not self._enabled:
            return
        self._reconcile()
        if not self._optimizer_states or any(state["stage"] != "stepped" for state in self._optimizer_states.values()):
            raise RuntimeError("Call step() for every unscaled optimizer before update().")
        if any(not state["finite"] for state in self._optimizer_states.values()):
            self._scale = self._scale_value(max(self._MIN_SCALE, self._scale * self._backoff_factor))
            self._growth_tracker = 0
        else:
            self._growth_tracker += 1
            if self._growth_tracker == self._growth_interval:
                self._scale = self._scale_value(min(self._MAX_SCALE, self._scale * self._growth_factor))
                self._growth_tracker = 0
        self._optimizer_states.clear()
        self._scale_used = False

    def fused_step(self, optimizer, max_norm=None, norm_type=2.0) -> StepResult:
        """``unscale_`` → ``clip_grad_norm_`` (only when finite) → ``step`` →
        ``update`` — the reference training loop's sequence
        (training/runner.py:248-251) — with every decision on the device."""
        return fused_step(optimizer, self, max_norm=max_norm, norm_type=norm_type)

    def _ensure_idle(self):
        self._reconcile()
        if self._optimizer_states or self._scale_used:
            raise RuntimeError("GradScaler state can be saved or loaded only between iterations, after update().")

    def state_dict(self):
        self._ensure_idle()
        return dict(version=1, scale=self._scale, growth_factor=self._growth_factor, backoff_factor=self._backoff_factor,
                    growth_interval=self._growth_interval, enabled=self._enabled, growth_tracker=self._growth_tracker)

    def _prepare_load_state_dict(self, state):
        self._ensure_idle()
        if type(state) is not dict or set(state) != {"version", "scale", "growth_factor", "backoff_factor", "growth_interval", "enabled", "growth_tracker"}:
            raise ValueError("Invalid GradScaler state fields.")
        if type(state["version"]) is not int or state["version"] != 1:
            raise ValueError("Unsupported GradScaler state version.")
        prepared = GradScaler(state["scale"], state["growth_factor"], state["backoff_factor"], state["growth_interval"], state["enabled"])
        tracker = state["growth_tracker"]
        if type(tracker) is not int or not 0 <= tracker < prepared._growth_interval:
            raise ValueError("Invalid GradScaler growth_tracker.")
        prepared._growth_tracker = tracker
        return prepared

    def load_state_dict(self, state):
        prepared = self._prepare_load_state_dict(state)
        self.__dict__.update(prepared.__dict__)


def fused_step(optimizer, scaler: GradScaler | None = None, *, max_norm=None, norm_type=2.0,
               scheduler=None, error_if_nonfinite: bool = False) -> StepResult:
    """One optimizer step with the reference training loop's AMP/clip
    semantics and no host synchronization.

    With an enabled ``scaler``: gradients are unscaled by the current loss
    scale; if every unscaled gradient is finite they are clipped to
    ``max_norm`` (when given) and the optimizer steps, otherwise the step is
    skipped; then the scale is updated — exactly ``unscale_``,
    ``clip_grad_norm_`` (if finite), ``step`` and ``update`` of
    training/runner.py:248-251.  Without a scaler: clip (when ``max_norm``
    is given) and step.  One pre-pass kernel, one single-workgroup finalize
    and the fused AdamW pass; the host learns the outcome from an
    asynchronous snapshot of the control block and reconciles its
    bookkeeping (``state['step']``, version counters, the scale mirror) at
    the next step, ``get_scale``/``state_dict`` or ``StepResult`` access.

    ``error_if_nonfinite`` is ``clip_grad_norm_``'s.  With a scaler the clip
    only runs after a finite unscale, whose norm is finite, so it never
    raises.  Without one, a non-finite norm leaves the gradients, parameters
    and state untouched on the device (the clip and the step are skipped, as
    the reference's raise prevents both), and the reference's RuntimeError
    is raised once the host learns the outcome: at the first access to the
    returned StepResult, or else at the start of the next ``fused_step``.

    ``optimizer`` may also be a list or tuple of optimizers that share the
    scaler's iteration (``_fused_step_many``): ``scheduler`` is then None or
    a sequence with one entry (None or a scheduler) per optimizer, and the
    result is a list with one StepResult per optimizer.

    ``scheduler`` (an ``optim.lr_scheduler.LRScheduler`` of ``optimizer``) is
    stepped when this step turns out to have updated, as the training loop
    does after ``scaler.step`` (runner.py:250-253).  The outcome is known on
    the device first, so the scheduler advances when the step is reconciled:
    before the next step computes its coefficients, or at the first read of
    the schedule.
    """
    reject_during_capture("Optimizer steps")
    if type(error_if_nonfinite) is not bool:
        raise TypeError("error_if_nonfinite must be a Python bool.")
    _raise_deferred_errors()
    if isinstance(optimizer, (list, tuple)):
        return _fused_step_many(list(optimizer), scaler, max_norm, norm_type, scheduler, error_if_nonfinite)
    _check_scheduler(scheduler, optimizer)
    amp, maximum, order = _fused_arguments(scaler, max_norm, norm_type)
    pairs = GradScaler._gradients(optimizer)
    gradients = list(map(_SECOND_OF, pairs))
    if not gradients:
        raise RuntimeError("No gradients were found for this optimizer.")
    groups = _device_groups(gradients)
    if len(groups) != 1 or type(optimizer) not in (Adam, AdamW):   # a subclass may read the gradients itself
        result = _fused_step_host(optimizer, scaler, amp, maximum, order, [p for p, _ in pairs],
                                  error_if_nonfinite)
        if scheduler is not None and result.updated:
            scheduler.step()
        return result
    (backend, dtype), _ = next(iter(groups.items()))
    if backend.adamw is None:
        backend._unsupported("Optimizer steps")
    # This step's block is written whole by the finalize, which starts from
    # the previous block's scaler state (or a neutral one without a scaler);
    # the pre-pass reads the loss scale from the previous block.
    if amp:
        latest = scaler._device_blocks.get(backend) if scaler._device_steps else None
        if latest is None:
            previous = backend.new_ctrl(scaler._scale, scaler._growth_tracker)
        else:
            previous = latest.block_for_current_stream()
    else:
        previous = backend.neutral_ctrl()
    # error_if_nonfinite without a scaler: a non-finite norm skips the clip and the step.
    refuse = error_if_nonfinite and not amp and maximum is not None
    flags = (_native.NT_FINALIZE_SCALER_UPDATE | _native.NT_FINALIZE_CLIP_IF_FINITE) if amp else 0
    if refuse:
        flags |= _native.NT_FINALIZE_CLIP_IF_FINITE
    growth, backoff, interval = (scaler._growth_factor, scaler._backoff_factor, scaler._growth_interval) if amp else (2.0, 0.5, 1)
    device_step = _queue_decisions(backend, dtype, gradients, previous, amp=amp, maximum=maximum, order=order,
                                   flags=flags, growth=growth, backoff=backoff, interval=interval,
                                   honor_skip=amp or refuse)
    device_step.scheduler = scheduler
    device_step.error_if_nonfinite = refuse
    if amp:
        scaler._reconcile()                               # earlier fused steps: their finalize already ran
        scaler._device_blocks[backend] = device_step
        scaler._device_steps.append(device_step)
        scaler._scale_used = False
    optimizer.step()                                      # the AdamW pass reads the control block
    optimizer._track_device_step(device_step)
    _unsettled_steps.append(device_step)                  # version reads settle it first
    if refuse:
        _error_watch.append(device_step)
    return StepResult(device_step)


def _queue_decisions(backend, dtype, gradients, previous, *, amp, maximum, order, flags, growth, backoff, interval,
                     honor_skip, combined=False) -> DeviceStep:
    """Queue the pre-pass and the finalize over one (backend, dtype) group of
    gradients, carrying the scaler state of the control block `previous`
    (whose scale the pre-pass unscales by when `amp`), and give the
    gradients the device-decided transform that the AdamW pass applies:
    the unscale, the clip to `maximum` (when given) and, with `honor_skip`,
    the skip.  Host bookkeeping is set as if the outcome were known: one
    version bump for the unscale and one for the clip, the latter undone at
    reconciliation when the device does not clip.  Returns the DeviceStep,
    captured on the current stream; nothing is launched if a check raises.

    `combined`: one of several optimizers of an iteration.  The finalize
    then only gathers this optimizer's statistics (no clip, flags or host
    copy); ``nt_amp_combine`` makes the decisions into every block, writes
    the mirrors, and the caller captures the steps after it."""
    block = backend.empty_ctrl()
    clip_bumps: list = []
    # float64 gradients may get a second norm pass after the finalize: that
    # block is read back with a copy instead of the finalize's mirror.
    mirror = None if dtype is float64 and order == 2.0 else runtime.take_mirror()
    device_step = DeviceStep(backend, block, unscale=amp, honor_skip=honor_skip, clip_bumps=clip_bumps,
                             mirror=mirror)
    device_step.clip_requested = maximum is not None
    transform = GradTransform(device=device_step)
    if any(map(_REQUIRES, gradients)) and is_grad_enabled():
        for gradient in gradients:
            gradient._ensure_inplace_allowed()            # raises the matching error
    check_addends(gradients)                              # before any bookkeeping changes
    if any(map(_PENDING, gradients)):
        for gradient in gradients:
            if gradient._pending is not None:
                gradient._materialize()
    # unscale_ rewrites every gradient (one version bump); the clip may (one
    # more, undone on reconcile if the device decides not to clip).
    bumps = int(amp) + int(maximum is not None)
    deque(map(setattr, gradients, repeat("_pending"), repeat(transform)), 0)
    counters = tuple(map(_COUNTER, gradients))
    for counter in counters:
        counter.value += bumps
    deque(map(setattr, gradients, repeat("_finite_version"), map(_VALUE, counters)), 0)
    if maximum is not None:
        clip_bumps.extend(zip(gradients, map(_VALUE, map(_COUNTER, gradients))))
    plan = backend.grad_plan(gradients, dtype, incoming=True)
    backend.grad_prepass(plan, None, previous.data_ptr(), unscale=amp)
    if combined:
        backend.grad_finalize(plan, block.data_ptr(), order, -1.0, 0, growth, backoff, interval,
                              carry_ptr=previous.data_ptr())
        return device_step
    backend.grad_finalize(plan, block.data_ptr(), order, -1.0 if maximum is None else maximum, flags,
                          growth, backoff, interval, carry_ptr=previous.data_ptr(), mirror=mirror)
    if dtype is float64 and order == 2.0:
        # fp64 squares can overflow or underflow: where max|g| says they may
        # have, the device redoes the norm with the reference's max-abs
        # prescale (clip_grad.py:73-78) and refreshes the clip decision.
        backend.grad_norm_pow(plan, block.data_ptr(), 2.0, -1.0 if maximum is None else maximum, None,
                              scale_from_ctrl=amp, flags=_native.NT_NORM_POW_GUARD)
    device_step.capture()
    return device_step


def _check_scheduler(scheduler, optimizer) -> None:
    if scheduler is not None:
        from .optim.lr_scheduler import LRScheduler
        if not isinstance(scheduler, LRScheduler):
            raise TypeError("scheduler must be a NamiTorch LRScheduler or None.")
        if scheduler.optimizer is not optimizer:
            raise ValueError("scheduler must belong to the supplied optimizer.")


def _fused_arguments(scaler, max_norm, norm_type) -> tuple:
    """(amp, max_norm, norm_type) after fused_step's checks of the scaler
    state and the clip arguments."""
    amp = scaler is not None and scaler._enabled
    if amp:
        if not scaler._scale_used:
            raise RuntimeError("Call scale(loss) and backward before unscale_.")
        if scaler._optimizer_states:
            raise RuntimeError("fused_step cannot follow unscale_ or step in the same iteration; call update() first.")
    maximum = None if max_norm is None else _nonnegative(max_norm, "max_norm")
    order = _norm_type(norm_type)
    if order != 2.0 and not math.isinf(order):
        raise ValueError("fused_step supports norm_type 2 and inf; use clip_grad_norm_ for other norms.")
    return amp, maximum, order


def _fused_step_many(optimizers: list, scaler, max_norm, norm_type, schedulers, error_if_nonfinite=False) -> list:
    """``fused_step`` over several optimizers in one scaler iteration: the
    reference loop's ``unscale_`` of every optimizer, ``clip_grad_norm_`` of
    all their parameters when every ``unscale_`` returned True (when
    ``max_norm`` is given), ``step`` of every optimizer and one ``update``
    (amp.py:169-233, training/runner.py:248-251).  As there, each optimizer
    steps unless its own gradients are non-finite (GradScaler.step checks
    only them), the scale backs off once if any optimizer's are, and
    optimizers may not share gradients (``unscale_``'s error).  Every check
    runs before anything changes.

    One pre-pass and finalize per optimizer, then one ``nt_amp_combine``
    that takes the global norm, clip and scaler decisions and gives each
    optimizer's control block its own skip flag; the AdamW passes read
    their blocks, so the host does not wait.  Returns one StepResult per
    optimizer (its own ``finite`` and ``updated``; the global ``norm`` and
    the next ``scale``)."""
    if not optimizers:
        raise ValueError("fused_step needs at least one optimizer.")
    if schedulers is None:
        schedulers = [None] * len(optimizers)
    elif not isinstance(schedulers, (list, tuple)) or len(schedulers) != len(optimizers):
        raise TypeError("With several optimizers, scheduler must be None or a sequence with one entry per optimizer.")
    for optimizer, scheduler in zip(optimizers, schedulers):
        _check_scheduler(scheduler, optimizer)
    amp, maximum, order = _fused_arguments(scaler, max_norm, norm_type)
    if amp:
        seen: set = set()
        for optimizer in optimizers:
            if id(optimizer) in seen:
                raise RuntimeError("unscale_ may be called only once per optimizer between update() calls.")
            seen.add(id(optimizer))
    gathered = []
    shared: set = set()
    for optimizer in optimizers:
        pairs = GradScaler._gradients(optimizer)
        if not pairs:
            raise RuntimeError("No gradients were found for this optimizer.")
        if amp:
            if any(id(parameter) in shared for parameter, _ in pairs):
                raise RuntimeError("Optimizers cannot share gradients in the same GradScaler iteration.")
            shared.update(id(parameter) for parameter, _ in pairs)
        gathered.append(list(map(_SECOND_OF, pairs)))
    groups = [_device_groups(gradients) for gradients in gathered]
    keys = [next(iter(g)) if len(g) == 1 else None for g in groups]
    distinct = len({id(optimizer) for optimizer in optimizers}) == len(optimizers)
    refuse = error_if_nonfinite and not amp and maximum is not None
    if (refuse or not distinct or len(optimizers) > _native.NT_MAX_COMBINE or any(key is None for key in keys)
            or len({id(key[0]) for key in keys}) != 1 or any(key[1] is float64 for key in keys)
            or keys[0][0].adamw is None or any(type(optimizer) not in (Adam, AdamW) for optimizer in optimizers)):
        # Several devices, mixed dtypes within an optimizer, float64 (its
        # guarded second norm pass), repeated optimizers, more optimizers
        # than one combine takes, a clip that may raise without a scaler, or
        # an optimizer subclass (which may read the gradients itself): the
        # synchronizing API gives the same results.
        return _fused_step_host_many(optimizers, scaler, amp, maximum, order, schedulers, error_if_nonfinite)
    backend = keys[0][0]
    for gradients in gathered:
        if any(map(_REQUIRES, gradients)) and is_grad_enabled():
            for gradient in gradients:
                gradient._ensure_inplace_allowed()        # raises the matching error
        check_addends(gradients)                          # before any bookkeeping changes
    if amp:
        latest = scaler._device_blocks.get(backend) if scaler._device_steps else None
        previous = backend.new_ctrl(scaler._scale, scaler._growth_tracker) if latest is None \
            else latest.block_for_current_stream()
    else:
        previous = backend.neutral_ctrl()
    flags = (_native.NT_FINALIZE_SCALER_UPDATE | _native.NT_FINALIZE_CLIP_IF_FINITE) if amp else 0
    growth, backoff, interval = (scaler._growth_factor, scaler._backoff_factor, scaler._growth_interval) if amp \
        else (2.0, 0.5, 1)
    device_steps = []
    for gradients, (_, dtype), scheduler in zip(gathered, keys, schedulers):
        device_step = _queue_decisions(backend, dtype, gradients, previous, amp=amp, maximum=maximum, order=order,
                                       flags=flags, growth=growth, backoff=backoff, interval=interval,
                                       honor_skip=amp, combined=True)
        device_step.scheduler = scheduler
        device_steps.append(device_step)
    backend.grad_combine([device_step.block for device_step in device_steps], previous, order,
                         -1.0 if maximum is None else maximum, flags, growth, backoff, interval,
                         mirrors=[device_step.mirror for device_step in device_steps])
    for device_step in device_steps:
        device_step.capture()
    if amp:
        scaler._reconcile()                               # earlier fused steps: their finalize already ran
        scaler._device_blocks[backend] = device_steps[0]  # every block holds the same scaler state
        scaler._device_steps.append(device_steps[0])
        scaler._scale_used = False
    for optimizer, device_step in zip(optimizers, device_steps):
        optimizer.step()                                  # each AdamW pass reads its own control block
        optimizer._track_device_step(device_step)
        _unsettled_steps.append(device_step)
    return [StepResult(device_step) for device_step in device_steps]


def _fused_step_host_many(optimizers, scaler, amp, maximum, order, schedulers, error_if_nonfinite=False) -> list:
    """``_fused_step_many`` through the host-synchronizing API."""
    parameters = [parameter for optimizer in optimizers for parameter, _ in GradScaler._gradients(optimizer)]
    norm = None
    if amp:
        finite = [scaler.unscale_(optimizer) for optimizer in optimizers]
        if all(finite) and maximum is not None:
            norm = clip_grad_norm_(parameters, maximum, norm_type=order, error_if_nonfinite=error_if_nonfinite).item()
        updated = [scaler.step(optimizer) for optimizer in optimizers]
        scaler.update()
        scale = scaler.get_scale()
        results = [StepResult(finite=f, updated=u, norm=norm, scale=scale) for f, u in zip(finite, updated)]
    else:
        if maximum is not None:
            norm = clip_grad_norm_(parameters, maximum, norm_type=order, error_if_nonfinite=error_if_nonfinite).item()
        for optimizer in optimizers:
            optimizer.step()
        finite = None if norm is None else math.isfinite(norm)
        results = [StepResult(finite=finite, updated=True, norm=norm, scale=1.0) for _ in optimizers]
    for scheduler, result in zip(schedulers, results):
        if scheduler is not None and result.updated:
            scheduler.step()
    return results


def _fused_step_host(optimizer, scaler, amp, maximum, order, parameters, error_if_nonfinite=False) -> StepResult:
    """Several devices or gradient dtypes: the same sequence through the
    host-synchronizing API (identical results)."""
    norm = None
    if amp:
        finite = scaler.unscale_(optimizer)
        if finite and maximum is not None:
            norm = clip_grad_norm_(parameters, maximum, norm_type=order, error_if_nonfinite=error_if_nonfinite).item()
        updated = scaler.step(optimizer)
        scaler.update()
        return StepResult(finite=finite, updated=updated, norm=norm, scale=scaler.get_scale())
    if maximum is not None:
        norm = clip_grad_norm_(parameters, maximum, norm_type=order, error_if_nonfinite=error_if_nonfinite).item()
    optimizer.step()
    return StepResult(finite=None if norm is None else math.isfinite(norm), updated=True, norm=norm, scale=1.0)


__all__ = ["GradScaler", "fused_step", "StepResult"]
