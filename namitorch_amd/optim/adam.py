"""Adam and AdamW (namitorch/optim/adam.py:8-94) on the MI355X.

Public signatures, option validation and state layout follow the
reference.  The update of every parameter of a step runs in one
multi-tensor kernel launch per (device, storage layout) instead of one
Python-level update per parameter (adam.py:69-94 → optim/_common.py:165-166).

Element arithmetic is the reference's (adam.py:35-42 + _common.py:67-73 ==
backends/cuda/adamw.py:15-25): coefficients are rounded to the parameter
dtype on the host exactly as ``_scalar`` does, and the kernel performs the
same fp32 operations in the same order without FMA contraction, so float32
results are bit-identical to the NumPy path.

Extension (no reference counterpart): ``AdamW(..., master_weights=True,
state_dtype=None|bfloat16)`` keeps a float32 master copy of each
float16/bfloat16/float32 parameter in ``state['master']``; the update is the
reference float32 update computed on the master with the gradient widened
exactly to float32, and the parameter receives the master rounded to its
own dtype (RNE) in the same pass.  Gradients may then be float16, bfloat16
or float32 whatever the parameter dtype; ``state_dtype=bfloat16`` stores
``exp_avg``/``exp_avg_sq`` rounded to bfloat16 (the update uses the
unrounded float32 values).
"""

from __future__ import annotations

import math
import weakref
from collections import deque
from itertools import repeat
from operator import add, attrgetter, eq, is_, itemgetter, setitem

import numpy as np

from .. import _native
from ..backends import get_backend
from ..backends._settings import fused_kernels_enabled
from ..backends.hip import INCOMING, incoming_pointers, make_xform
from ..dtype import DType, bfloat16, float16, float32, float64, normalize_dtype
from ..tensor import Tensor, _assign_host, _requires_grad_changes
from ._common import _FirstOrderOptimizer, _real_option, _round_scalar, _zeros_views

_LOW_PRECISION = (float16, bfloat16, float32)


def _zeros_like(parameter: Tensor, dtype: DType) -> Tensor:
    return _zeros_views([parameter.shape], dtype, parameter.device)[0]


class Adam(_FirstOrderOptimizer):
    _state_buffers = ("exp_avg", "exp_avg_sq")
    _required_buffers = ("exp_avg", "exp_avg_sq")
    _nonnegative_buffers = ("exp_avg_sq",)
    _has_step = True
    _master_weights = False
    _moment_dtype = None

    def __init__(self, params, lr: float = 1e-3, betas: tuple[float, float] = (0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 0.0, *, maximize: bool = False):
        super().__init__(params, {"lr": lr, "betas": betas, "eps": eps, "weight_decay": weight_decay, "maximize": maximize})

    def _prepare_options(self, options: dict, path: str) -> dict:
        prepared = super()._prepare_options(options, path)
        _real_option(prepared, "eps", positive=True)
        betas = prepared.get("betas")
        if not isinstance(betas, (tuple, list)) or len(betas) != 2:
            raise TypeError("Adam betas must contain exactly two real scalars.")
        normalized = {"beta1": betas[0], "beta2": betas[1]}
        prepared["betas"] = tuple(_real_option(normalized, name, unit_interval=True) for name in ("beta1", "beta2"))
        return prepared

    # ---- dtypes --------------------------------------------------------------------------
    def _compute_dtype(self, parameter: Tensor) -> DType:
        return float32 if self._master_weights else parameter.dtype

    def _state_dtype(self, parameter: Tensor, name: str) -> DType:
        if not self._master_weights:
            return parameter.dtype
        if name == "master":
            return float32
        return self._moment_dtype or float32

    def _use_fused(self, parameter: Tensor, gradient: Tensor, options: dict) -> bool:
        return False

    # ---- the update ------------------------------------------------------------------------
    def _update_parameter(self, parameter: Tensor, gradient: Tensor, options: dict) -> None:
        self._update_many([(parameter, gradient, options)])

    def _coefficients(self, dtype: DType, options: dict, step: int, fused: bool):
        beta1, beta2 = options["betas"]
        lr, wd = options["lr"], options["weight_decay"]
        values = (lr, beta1, beta2, 1 - beta1, 1 - beta2, options["eps"], wd, 1 - lr * wd,
                  1 - beta1 ** step, 1 - beta2 ** step)
        coefficients = tuple(_round_scalar(dtype, value) for value in values)
        if fused and (coefficients[5] <= 0 or coefficients[8] <= 0 or coefficients[9] <= 0):
            raise ValueError("Fused AdamW eps and bias corrections must be positive.")
        record_type = _native.AdamWCoefs64 if dtype is float64 else _native.AdamWCoefs
        return record_type(*coefficients, int(options["maximize"]), int(lr != 0),
                           int(not self._decoupled_weight_decay), 0)

    @staticmethod
    def _next_coefficients(dtype: DType, options: dict, step: int, fused: bool, previous):
        """``_coefficients`` for `step` from the record of an earlier step with
        the same options: only the two bias corrections depend on the step."""
        beta1, beta2 = options["betas"]
        first = _round_scalar(dtype, 1 - beta1 ** step)
        second = _round_scalar(dtype, 1 - beta2 ** step)
        if fused and (first <= 0 or second <= 0):
            raise ValueError("Fused AdamW eps and bias corrections must be positive.")
        record = type(previous).from_buffer_copy(previous)
        record.correction1 = first
        record.correction2 = second
        return record

    def _create_buffers(self, parameters) -> None:
        """The missing buffers of `parameters`, created together: zero moments
        and the fp32 master copy as views of one flat allocation per (buffer,
        device, dtype).  Values are those ``_buffers`` gives one at a time."""
        names = ("exp_avg", "exp_avg_sq") + (("master",) if self._master_weights else ())
        states = self.state
        for name in names:
            groups: dict = {}
            for parameter in parameters:
                if states[id(parameter)].get(name) is None:
                    key = (parameter._device, self._state_dtype(parameter, name))
                    groups.setdefault(key, []).append(parameter)
            for (device, dtype), members in groups.items():
                views = _zeros_views([parameter.shape for parameter in members], dtype, device)
                for parameter, view in zip(members, views):
                    if name == "master":
                        if view._device.type == "cpu":
                            _assign_host(view._storage, parameter._data, view._dtype, parameter._dtype)
                        else:
                            view._storage.copy_from(parameter._data)     # exact: widening to float32
                    states[id(parameter)][name] = view

    def _buffers(self, parameter: Tensor, state: dict):
        first = state.get("exp_avg")
        if first is None:
            first = state["exp_avg"] = _zeros_like(parameter, self._state_dtype(parameter, "exp_avg"))
        second = state.get("exp_avg_sq")
        if second is None:
            second = state["exp_avg_sq"] = _zeros_like(parameter, self._state_dtype(parameter, "exp_avg_sq"))
        master = None
        if self._master_weights:
            master = state.get("master")
            if master is None:
                master = state["master"] = Tensor(parameter, dtype=float32, device=parameter.device)
        return first, second, master

    def _update_many(self, items) -> None:
        self._batches = []
        if not items:
            return
        layouts: dict = {}
        groups: dict = {}
        for member in items:
            parameter, gradient = member[0], member[1]
            key = (parameter._dtype, gradient._dtype)
            layout = layouts.get(key)
            if layout is None:
                compute = self._compute_dtype(parameter)
                if compute is bfloat16:
                    raise TypeError("bfloat16 parameters require AdamW(master_weights=True).")
                state_dtype = self._state_dtype(parameter, "exp_avg")
                copy = parameter._dtype.code if self._master_weights else _native.NT_DTYPE_NONE
                layout = layouts[key] = (compute.code, gradient._dtype.code, state_dtype.code, copy)
            groups.setdefault((parameter._device, layout), []).append(member)
        for (device, layout), members in groups.items():
            backend = get_backend(device)
            if backend.adamw is None:
                backend._unsupported("Optimizer steps")
            self._launch_group(backend, layout, members)

    def _launch_group(self, backend, layout, members) -> None:
        # A launch carries at most NT_MAX_SLOTS coefficient sets; split if the
        # (param group, step) combinations of this step exceed it.
        states = self.state
        keys = {(id(options), states[id(parameter)].get("step", 0) + 1) for parameter, _, options in members}
        if len(keys) <= _native.NT_MAX_SLOTS:
            self._launch_batch(backend, layout, members)
            return
        batch: list = []
        slot_keys: set = set()
        for member in members:
            parameter, _, options = member
            key = (id(options), states[id(parameter)].get("step", 0) + 1)
            if key not in slot_keys and len(slot_keys) == _native.NT_MAX_SLOTS:
                self._launch_batch(backend, layout, batch)
                batch, slot_keys = [], set()
            slot_keys.add(key)
            batch.append(member)
        if batch:
            self._launch_batch(backend, layout, batch)

    def _fused_decision(self, parameter: Tensor, gradient: Tensor, options: dict, first, second) -> bool:
        """``_use_fused``, memoized on the objects it depends on."""
        fused_option = options.get("fused")
        if self._master_weights:
            # Master-weight updates are always supported by the device pass:
            # the decision depends only on the option and the global switch.
            return self._use_fused(parameter, gradient, options)
        cache = self.__dict__.setdefault("_fused_checked", {})
        seen = cache.get(id(parameter))
        if (seen is not None and seen[0] is parameter and seen[1]() is gradient and seen[2] is first
                and seen[3] is second and seen[4] is fused_option and seen[5] == fused_kernels_enabled()):
            return seen[6]
        decision = self._use_fused(parameter, gradient, options)
        cache[id(parameter)] = (parameter, weakref.ref(gradient), first, second, fused_option,
                                fused_kernels_enabled(), decision)
        return decision

    def _launch_batch(self, backend, layout, members) -> None:
        compute = {_native.NT_F32: float32, _native.NT_F16: float16, _native.NT_F64: float64}[layout[0]]
        slot_of: dict = {}
        records: list = []
        rows: list = []
        bookkeeping: list = []
        slot_specs: list = []        # (id(options), step, fused) per coefficient slot
        grad_pointers: list = []
        member_slots: list = []
        transform = members[0][1]._pending
        for _, gradient, _ in members:
            if gradient._pending != transform:
                for _, other, _ in members:
                    other._materialize()
                transform = None
                break
        states = self.state
        master_mode = self._master_weights
        fused_cache = self.__dict__.setdefault("_fused_checked", {})
        enabled = fused_kernels_enabled()
        fresh = [parameter for parameter, _, _ in members
                 if states[id(parameter)].get("exp_avg") is None or states[id(parameter)].get("exp_avg_sq") is None
                 or (master_mode and states[id(parameter)].get("master") is None)]
        if len(fresh) > 1:
            self._create_buffers(fresh)
        for parameter, gradient, options in members:
            state = states[id(parameter)]
            first = state.get("exp_avg")
            second = state.get("exp_avg_sq")
            master = state.get("master") if master_mode else None
            if first is None or second is None or (master_mode and master is None):
                first, second, master = self._buffers(parameter, state)
            step = state.get("step", 0) + 1
            seen = fused_cache.get(id(parameter))
            if (seen is not None and seen[0] is parameter and seen[1]() is gradient and seen[2] is first
                    and seen[3] is second and seen[4] is options.get("fused") and seen[5] is enabled):
                fused = seen[6]
            else:
                fused = self._fused_decision(parameter, gradient, options, first, second)
            key = (id(options), step)
            slot = slot_of.get(key)
            if slot is None:
                slot = slot_of[key] = len(records)
                records.append(self._coefficients(compute, options, step, fused))
                slot_specs.append((id(options), step, fused))
            member_slots.append(slot)
            if master is not None:
                rows.append((master._ptr, 0, first._ptr, second._ptr, parameter._ptr, parameter._numel, slot))
            else:
                rows.append((parameter._ptr, 0, first._ptr, second._ptr, 0, parameter._numel, slot))
            grad_pointers.append(gradient._ptr)
            bookkeeping.append((parameter, state, first, second, master, step, fused, options["lr"] != 0))
        slots = ((_native.AdamWCoefs64 if compute is float64 else _native.AdamWCoefs) * len(records))(*records)
        pointers = {1: grad_pointers}
        # Deferred accumulations (accumulate_grads(..., defer=True)) are added
        # by the pass as it reads each gradient.
        addends = incoming_pointers([gradient for _, gradient, _ in members])
        if addends is not None:
            pointers[INCOMING] = addends
        plan = backend.plan(rows, layout, chunk=_pass_chunk(layout), pointers=pointers)
        backend.adamw_multi(plan, slots, None if transform is None else make_xform(transform))
        # A plan with an incoming column is not memoized: a replay could
        # otherwise add the same addends again.
        self._batches.append((backend, plan, compute, slot_specs, member_slots, bookkeeping) if addends is None
                             else None)
        device_step = None if transform is None else transform.device
        for parameter, state, first, second, master, step, fused, moves in bookkeeping:
            bumped = not fused or parameter._numel
            if bumped:
                first._version_counter.value += 1
                second._version_counter.value += 1
                first._clean_version = first._version_counter.value
                second._clean_version = second._version_counter.value
                if moves:
                    parameter._version_counter.value += 1
                    if master is not None:
                        master._version_counter.value += 1
            state["step"] = step
            if device_step is not None:
                # The device decides whether this step is skipped; remember
                # what to undo on the host if it was.
                device_step.records.append((parameter, state, first, second, master, step, bumped, moves))
        if device_step is not None:
            self._consume_device_step(device_step)

    def _memoize_step(self, options: dict) -> None:
        batches = self.__dict__.pop("_batches", None)
        self._replay = None
        if batches is None or len(batches) != 1 or batches[0] is None:
            return
        cached = self.__dict__.get("_registered_cache")
        if cached is None:
            return
        group_index = {id(options[id(group)]): index for index, group in enumerate(self.param_groups)}
        self._replay = _Replay(self, cached, group_index, *batches[0])


_GRAD = attrgetter("_grad")
_REQUIRES = attrgetter("_requires_grad")
_PENDING = attrgetter("_pending")
_INCOMING = attrgetter("_incoming")
_CLEAN = attrgetter("_clean_version")
_VALUE = attrgetter("value")
_COUNTER = attrgetter("_version_counter")
_FIRST = itemgetter("exp_avg")
_SECOND = itemgetter("exp_avg_sq")
_MASTER = itemgetter("master")
_STEP = itemgetter("step")
_DTYPE = attrgetter("_dtype")
_PTR = attrgetter("_ptr")
_SECOND_OF = itemgetter(1)
_THIRD_OF = itemgetter(2)


def _IS_NONE(value) -> bool:
    return value is None


def _exact_float(value: float):
    """A finite float as a key item that compares equal only to the same
    value with the same sign: float equality is exact except that +0.0 and
    -0.0 compare equal, so zeros carry their sign."""
    return (value, math.copysign(1.0, value)) if value == 0.0 else value


def _options_key(groups) -> tuple | None:
    """The option values of every parameter group, exactly: names, types,
    and values (floats by value and, for zeros, sign).  Two steps with equal
    keys prepare equal options and pass the same checks.  None (do not
    memoize) for values whose checks must run every step: non-finite floats,
    or anything other than scalars and tuples/lists of scalars."""
    key: list = []
    for group in groups:
        for name, value in group.items():
            if name == "params":
                continue
            kind = type(value)
            if kind is float:
                if not math.isfinite(value):
                    return None
                value = _exact_float(value)
            elif kind is tuple or kind is list:
                items = []
                for item in value:
                    if type(item) is float and math.isfinite(item):
                        items.append((float, _exact_float(item)))
                    elif type(item) in (int, bool):
                        items.append((type(item), item))
                    else:
                        return None
                value = tuple(items)
            elif kind not in (int, bool, str, type(None)):
                return None
            key.append((name, kind, value))
        key.append(None)
    return tuple(key)


_SIXTEEN_BIT = (_native.NT_F16, _native.NT_BF16)


def _pass_chunk(layout: tuple) -> int:
    """Elements per workgroup task of the AdamW pass for a plan layout
    (param, grad, state, copy dtype codes): 2048 when the gradient or the
    moments are 16-bit, else the library default of 4096.  Timed alternately
    in one process on the same buffers (bench.py --configs chunks), 2048 is
    2-3.5 % faster for the GPT-2 AMP, GPT-1.3B and Llama-7B layouts and
    2-3 % slower for all-fp32 ones."""
    return 2048 if layout[1] in _SIXTEEN_BIT or layout[2] in _SIXTEEN_BIT else 0


class _Replay:
    """Memo of the last step's single multi-tensor launch.

    The full step re-validates every parameter, gradient and state entry, at
    about a microsecond of Python per tensor.  Those checks depend only on
    which objects are involved (a Tensor's dtype, shape, device and storage
    never change) and on a few mutable fields.  A later step replays the
    launch when all of these are unchanged:
    - the registered parameters, their gradients and ``requires_grad`` flags;
    - the state dictionaries, their buffers and step counts;
    - the buffers' flags and the nonnegative buffer's versions.

    Each is verified with a C-level pass over the tuples kept here.  The
    replay prepares and validates the options again, recomputes the
    coefficients for the next step counts, relaunches the cached plan and
    applies the same bookkeeping.  Anything else makes ``run`` return False,
    and the caller runs the full step, which builds a new memo.
    """

    __slots__ = ("registered_cache", "registered", "requires", "requires_checked", "grads", "state", "ids", "dicts",
                 "lens", "firsts", "seconds", "masters", "master_mode", "steps", "buffers", "members", "member_grads",
                 "second_counters", "fused_options", "enabled", "validate", "slots", "backend", "plan", "compute",
                 "record_type", "moment_buffers", "moment_counters", "move_counters", "member_groups", "bumped", "stream", "options_key",
                 "prepared", "adoptable", "spans", "sizes", "records")

    def __init__(self, optimizer, cached, group_index, backend, plan, compute, slot_specs, member_slots, bookkeeping):
        self.registered_cache = cached
        self.registered = cached[1]
        self.requires = tuple(map(_REQUIRES, self.registered))
        self.requires_checked = _requires_grad_changes.value     # the flags above hold at this count
        self.grads = tuple(map(_GRAD, self.registered))
        self.state = optimizer.state
        self.members = tuple(entry[0] for entry in bookkeeping)
        self.member_grads = tuple(map(_GRAD, self.members))
        self.ids = tuple(map(id, self.members))
        self.dicts = tuple(entry[1] for entry in bookkeeping)
        self.lens = tuple(map(len, self.dicts))
        self.firsts = tuple(entry[2] for entry in bookkeeping)
        self.seconds = tuple(entry[3] for entry in bookkeeping)
        self.masters = tuple(entry[4] for entry in bookkeeping)
        self.master_mode = optimizer._master_weights
        self.steps = tuple(entry[5] for entry in bookkeeping)
        self.buffers = self.firsts + self.seconds + (self.masters if self.master_mode else ())
        self.second_counters = tuple(map(_COUNTER, self.seconds))
        groups = optimizer.param_groups
        self.fused_options = tuple(group.get("fused") for group in groups)
        self.enabled = fused_kernels_enabled()
        # Coefficient slots in launch order: (group index, step count used last, fused flag).
        self.slots = [(group_index[options_id], step, fused) for options_id, step, fused in slot_specs]
        self.member_groups = tuple(self.slots[slot][0] for slot in member_slots)
        representatives: dict = {}
        for parameter, group in zip(self.members, self.member_groups):
            representatives.setdefault((parameter._dtype, group), parameter)
        self.validate = tuple((group, parameter) for (_, group), parameter in representatives.items())
        self.backend = backend
        self.plan = plan
        self.stream = backend.stream()      # the plan's pointer columns are ordered on this stream
        self.compute = compute
        self.record_type = _native.AdamWCoefs64 if compute is float64 else _native.AdamWCoefs
        self.bumped = tuple(bool(not entry[6] or entry[0]._numel) for entry in bookkeeping)
        self.moment_buffers = tuple(buffer for entry, bumped in zip(bookkeeping, self.bumped) if bumped
                                    for buffer in (entry[2], entry[3]))
        self.moment_counters = tuple(map(_COUNTER, self.moment_buffers))
        moving: list = [[] for _ in groups]
        for entry, bumped, group in zip(bookkeeping, self.bumped, self.member_groups):
            if bumped:
                moving[group].append(entry[0]._version_counter)
                if entry[4] is not None:
                    moving[group].append(entry[4]._version_counter)
        self.move_counters = tuple(tuple(counters) for counters in moving)
        self.options_key = None
        self.prepared = None
        self.records = None                  # the last launch's coefficient records, one per slot
        # Adopting new gradient objects without master weights: the fused
        # decision of a member depends on its gradient only through overlap
        # with the parameter and moments (device, dtype, shape and layout are
        # what validation already checks), so a memo whose every
        # grad-dependent decision was "fused" keeps the byte ranges to test
        # new gradients against.
        self.adoptable = self.master_mode
        self.spans = self.sizes = None
        if not self.master_mode:
            depends = [self.fused_options[group] is not False and self.enabled for group in self.member_groups]
            fused = [entry[6] for entry in bookkeeping]
            pointers = [(entry[0]._ptr, entry[2]._ptr, entry[3]._ptr) for entry in bookkeeping]
            self.adoptable = (all(f or not d for f, d in zip(fused, depends)) and any(depends)
                              and None not in (value for row in pointers for value in row))
            if self.adoptable:
                self.sizes = np.array([entry[0]._numel * entry[0]._dtype.itemsize if d else 0
                                       for entry, d in zip(bookkeeping, depends)], dtype=np.int64)
                lows = np.array(pointers, dtype=np.int64).reshape(len(bookkeeping), 3)
                self.spans = (lows, lows + self.sizes[:, None])

    def _unchanged(self, optimizer) -> bool:
        optimizer._registered_parameters()
        if optimizer.__dict__.get("_registered_cache") is not self.registered_cache:
            return False
        registered = self.registered
        # requires_grad flags are re-read only when one changed somewhere
        # since they were last seen to hold (parameters as memoized, state
        # buffers all False).
        changes = _requires_grad_changes.value
        flags_seen = changes == self.requires_checked
        if not flags_seen and tuple(map(_REQUIRES, registered)) != self.requires:
            return False
        current = tuple(map(_GRAD, registered))
        if not all(map(is_, current, self.grads)) and not self._adopt(optimizer, current):
            return False
        if any(map(_INCOMING, self.member_grads)):
            return False                                        # the full step adds deferred accumulations
        state = optimizer.state
        if state is not self.state:
            return False
        dicts = tuple(map(state.get, self.ids))
        if not all(map(is_, dicts, self.dicts)) or tuple(map(len, dicts)) != self.lens:
            return False
        try:
            if not (all(map(is_, map(_FIRST, dicts), self.firsts)) and all(map(is_, map(_SECOND, dicts), self.seconds))
                    and (not self.master_mode or all(map(is_, map(_MASTER, dicts), self.masters)))):
                return False
            # The step counts are the int objects the last step stored (an
            # equal value of another type or object takes the full step).
            if not all(map(is_, map(_STEP, dicts), self.steps)):
                return False
        except KeyError:
            return False
        if not flags_seen and any(map(_REQUIRES, self.buffers)):
            return False
        self.requires_checked = changes
        if not all(map(eq, map(_CLEAN, self.seconds), map(_VALUE, self.second_counters))):
            return False
        # Equal transforms, as the full step compares; usually one shared object.
        pending = tuple(map(_PENDING, self.member_grads))
        if not pending or (not all(map(is_, pending, repeat(pending[0]))) and len(set(pending)) != 1):
            return False
        return fused_kernels_enabled() is self.enabled and self.backend.stream() == self.stream

    def _adopt(self, optimizer, current) -> bool:
        """New gradient objects for the same parameters (gradients reallocated
        every step): validate them as the full step does, then re-point the
        cached plan's gradient column.  Without master weights the fused
        decision must also come out the same: no new gradient may overlap its
        parameter or moments (otherwise the full step decides)."""
        if not self.adoptable or not all(map(is_, map(_IS_NONE, current), map(_IS_NONE, self.grads))):
            return False
        entries = optimizer._grad_entries()                      # raises the full step's errors
        if len(entries) != len(self.members) or not all(map(is_, map(_SECOND_OF, entries), self.members)):
            return False
        grads = tuple(map(_THIRD_OF, entries))
        if not all(map(is_, map(_DTYPE, grads), map(_DTYPE, self.member_grads))):
            return False                                        # another storage layout
        if self.spans is not None:
            lows, highs = self.spans
            start = np.fromiter(map(_PTR, grads), dtype=np.int64, count=len(grads))
            end = start + self.sizes
            if bool(np.any((start[:, None] < highs) & (lows < end[:, None]) & (self.sizes[:, None] > 0))):
                return False                                    # the full step decides "not fused"
        if not self.backend._refresh(self.plan, {1: tuple(map(_PTR, grads))}, self.stream):
            return False
        self.grads = current
        self.member_grads = grads
        return True

    def run(self, optimizer) -> bool:
        if not self._unchanged(optimizer):
            return False
        key = _options_key(optimizer.param_groups)
        previous = None
        if key is not None and key == self.options_key:
            prepared = self.prepared                 # same option values: same preparation and checks
            previous = self.records
        else:
            prepared = [optimizer._prepare_options({name: value for name, value in group.items() if name != "params"},
                                                   "param_group") for group in optimizer.param_groups]
            if tuple(options.get("fused") for options in prepared) != self.fused_options:
                return False
            checked: set = set()
            for group, parameter in self.validate:
                optimizer._validate_entry(parameter, prepared[group], checked)
            self.options_key, self.prepared = key, prepared
        if previous is not None:
            records = [optimizer._next_coefficients(self.compute, prepared[group], step + 1, fused, record)
                       for (group, step, fused), record in zip(self.slots, previous)]
        else:
            records = [optimizer._coefficients(self.compute, prepared[group], step + 1, fused)
                       for group, step, fused in self.slots]
        self.records = records
        transform = self.member_grads[0]._pending
        self.backend.adamw_multi(self.plan, (self.record_type * len(records))(*records),
                                 None if transform is None else make_xform(transform))
        # Bookkeeping of the full step: moments always, parameter (and master)
        # only for groups whose lr is nonzero, then the step counts.
        for counter in self.moment_counters:
            counter.value += 1
        deque(map(setattr, self.moment_buffers, repeat("_clean_version"), map(_VALUE, self.moment_counters)), 0)
        moves = [options["lr"] != 0 for options in prepared]
        for group, counters in enumerate(self.move_counters):
            if moves[group]:
                for counter in counters:
                    counter.value += 1
        steps = tuple(map(add, self.steps, repeat(1)))
        deque(map(setitem, self.dicts, repeat("step"), steps), 0)
        self.steps = steps
        self.slots = [(group, step + 1, fused) for group, step, fused in self.slots]
        device_step = None if transform is None else transform.device
        if device_step is not None:
            device_step.records.extend(zip(self.members, self.dicts, self.firsts, self.seconds, self.masters, steps,
                                           self.bumped, map(moves.__getitem__, self.member_groups)))
            optimizer._consume_device_step(device_step)
        return True


class AdamW(Adam):
    _decoupled_weight_decay = True

    def __init__(self, params, lr: float = 1e-3, betas: tuple[float, float] = (0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 1e-2, *, maximize: bool = False, fused=None,
                 master_weights: bool = False, state_dtype=None):
        if type(master_weights) is not bool:
            raise TypeError("AdamW master_weights must be a Python bool.")
        moment = None if state_dtype is None else normalize_dtype(state_dtype)
        if moment is not None and moment not in (float32, bfloat16):
            raise TypeError("AdamW state_dtype must be None, float32 or bfloat16.")
        if moment is not None and not master_weights:
            raise ValueError("AdamW state_dtype requires master_weights=True.")
        self._master_weights = master_weights
        self._moment_dtype = moment
        if master_weights:
            self._state_buffers = ("exp_avg", "exp_avg_sq", "master")
            self._required_buffers = ("exp_avg", "exp_avg_sq", "master")
        _FirstOrderOptimizer.__init__(self, params, {"lr": lr, "betas": betas, "eps": eps, "weight_decay": weight_decay,
                                                     "maximize": maximize, "fused": fused})

    def _prepare_options(self, options: dict, path: str) -> dict:
        prepared = super()._prepare_options(options, path)
        fused = prepared.setdefault("fused", None)
        if fused is not None and type(fused) is not bool:
            raise TypeError("AdamW fused must be None, True or False.")
        return prepared

    def _gradient_dtype_ok(self, parameter: Tensor, gradient: Tensor) -> bool:
        if self._master_weights:
            return gradient.dtype in _LOW_PRECISION and parameter.dtype in _LOW_PRECISION
        return gradient.dtype is parameter.dtype

    def _gradient_dtypes_ok(self, parameters: tuple, gradients: tuple) -> bool:
        if self._master_weights:
            allowed = _LOW_PRECISION.__contains__
            return all(map(allowed, map(_DTYPE, gradients))) and all(map(allowed, map(_DTYPE, parameters)))
        return super()._gradient_dtypes_ok(parameters, gradients)

    def _fused_supported(self, parameter: Tensor, gradient: Tensor) -> bool:
        """What the reference's ``supports`` checks (backends/cuda/adamw.py:33-46)."""
        backend = get_backend(parameter)
        if backend.adamw is None:
            return False
        if self._master_weights:
            return True
        state = self.state.get(id(parameter), {})
        arrays = [parameter._storage, gradient._storage] + [
            state[name]._storage for name in ("exp_avg", "exp_avg_sq") if isinstance(state.get(name), Tensor)
        ]
        return backend.adamw.supports(*arrays)

    def _validate_update(self, parameter, gradient, options):
        if options["fused"] is True and not self._fused_decision_supported(parameter, gradient):
            raise RuntimeError("fused=True requires non-overlapping contiguous float32 CUDA parameters, gradients and states on the same device.")

    def _fused_decision_supported(self, parameter: Tensor, gradient: Tensor) -> bool:
        """``_fused_supported`` memoized on the parameter/gradient/state objects."""
        state = self.state.get(id(parameter), {})
        first, second = state.get("exp_avg"), state.get("exp_avg_sq")
        cache = self.__dict__.setdefault("_support_checked", {})
        seen = cache.get(id(parameter))
        if seen is not None and seen[0] is parameter and seen[1]() is gradient and seen[2] is first and seen[3] is second:
            return seen[4]
        supported = self._fused_supported(parameter, gradient)
        cache[id(parameter)] = (parameter, weakref.ref(gradient), first, second, supported)
        return supported

    def _use_fused(self, parameter: Tensor, gradient: Tensor, options: dict) -> bool:
        fused = options["fused"]
        if fused is False or (fused is None and not fused_kernels_enabled()):
            return False
        if self._master_weights:
            return get_backend(parameter).adamw is not None
        supported = self._fused_decision_supported(parameter, gradient)
        if fused is True and not supported:
            raise RuntimeError("The parameter, gradient or optimizer state does not support fused AdamW.")
        return supported


__all__ = ["Adam", "AdamW"]
