"""First-order optimizer machinery (namitorch/optim/_common.py).

Option validation (``_real_option``/``_bool_option``, _common.py:16-36), the
rounding of host scalars to the parameter dtype (``_scalar``, 39-47) and the
step orchestration of ``_FirstOrderOptimizer.step`` (133-167) keep the
reference's checks, order and messages.  What changes is the update: the
reference loops over parameters in Python and launches one kernel each
(165-166); here every parameter of a step is handed to
``_update_many``, which groups them by device and storage layout and
launches one multi-tensor kernel per group.

Per-step validation is memoized where its inputs cannot have changed:
``_scalar`` checks depend only on (dtype, option values), and the
"exp_avg_sq is nonnegative" state check (a full read of the buffer in the
reference) is skipped for buffers whose version counter shows that only this
optimizer's kernels wrote them since the last check — those kernels cannot
produce a negative value.
"""

from __future__ import annotations

import math
import struct
from numbers import Real

import numpy as np

from ..array import DeviceArray, is_device_array
from ..backends import ensure_same_device, get_backend
from ..backends._graph_capture import reject_during_capture
from ..dtype import DType, bfloat16, from_numpy_dtype
from ..tensor import Tensor, enable_grad, no_grad
from .optimizer import Optimizer


def _real_option(options: dict, name: str, positive: bool = False, unit_interval: bool = False) -> float:
    if name not in options:
        raise ValueError(f"Missing optimizer option {name!r}.")
    value = options[name]
    if isinstance(value, (bool, np.bool_)) or not isinstance(value, Real):
        raise TypeError(f"Optimizer {name} must be a real scalar.")
    try:
        value = float(value)
    except OverflowError:
        raise ValueError(f"Optimizer {name} must be finite.") from None
    if not math.isfinite(value) or value < 0 or (positive and value == 0) or (unit_interval and value >= 1):
        constraint = "in [0, 1)" if unit_interval else "positive" if positive else "nonnegative"
        raise ValueError(f"Optimizer {name} must be finite and {constraint}.")
    options[name] = value
    return value


def _bool_option(options: dict, name: str) -> bool:
    if name not in options or type(options[name]) is not bool:
        raise TypeError(f"Optimizer {name} must be a Python bool.")
    return options[name]


_PACK = {DType.float32: struct.Struct("<f"), DType.float16: struct.Struct("<e")}
_FINFO_MAX = {dtype: dtype.finfo_max for dtype in (DType.float16, DType.float32, DType.float64, DType.bfloat16)}


def _round_scalar(dtype: DType, value: float, name: str = "coefficient") -> float:
    """Round a host float to `dtype` once (RNE), as ``dtype.type(value)``.

    float32/float16 use the C conversion of ``struct`` packing, the same
    single IEEE rounding NumPy's scalar constructors perform.
    """
    if not math.isfinite(value) or abs(value) > _FINFO_MAX[dtype]:
        raise ValueError(f"Optimizer {name} must be representable in {dtype.name}.")
    packer = _PACK.get(dtype)
    if packer is not None:
        try:
            result = packer.unpack(packer.pack(value))[0]
        except OverflowError:
            # |value| within finfo.max but rounding up past it: NumPy gives inf.
            result = math.copysign(math.inf, value)
    elif dtype is DType.float64:
        result = float(value)
    else:
        from ..tensor import _bf16_bits_from_f64
        bits = int(_bf16_bits_from_f64(np.asarray([value]))[0])
        result = float(np.array([bits << 16], dtype=np.uint32).view(np.float32)[0])
    if name == "eps" and result == 0:
        raise ValueError(f"Optimizer eps must remain positive in {dtype.name}.")
    return result


def _scalar(parameter: Tensor, value: float, name: str = "coefficient"):
    """The reference's ``_scalar``: `value` rounded to the parameter dtype."""
    return _round_scalar(parameter.dtype, value, name)


# ---- contiguous state buffers -------------------------------------------------------------
# The update pass streams optimizer-owned buffers (moments, master weights)
# faster when all buffers of one kind are ranges of a single allocation than
# when each is an allocation of its own: on MI355X the GPT-2-AMP and sharded
# Llama-7B passes ran 2 % and 10 % faster that way.  Each range starts on a
# multiple of _ARENA_ALIGN elements, which keeps every buffer 16-byte aligned
# and on the pass's 256-element slices.
_ARENA_ALIGN = 256


def _zeros_views(shapes, dtype: DType, device) -> list:
    """Zero-filled Tensors of `shapes` that are views of one flat buffer."""
    counts = [math.prod(shape) for shape in shapes]
    offsets, total = [], 0
    for count in counts:
        offsets.append(total)
        total += -(-count // _ARENA_ALIGN) * _ARENA_ALIGN
    if device.type == "cpu":
        flat = np.zeros(max(total, 1), dtype=np.uint16 if dtype is bfloat16 else dtype.numpy_dtype)
        return [Tensor._from_storage(flat[offset:offset + count].reshape(tuple(shape)), dtype=dtype)
                for offset, count, shape in zip(offsets, counts, shapes)]
    flat = DeviceArray.zeros((max(total, 1),), dtype, device)
    return [Tensor._from_storage(flat.narrow(offset, count, tuple(shape)))
            for offset, count, shape in zip(offsets, counts, shapes)]


def _pack_state_buffers(states, names, keep=frozenset()) -> None:
    """Move the buffers `names` of every state dictionary into one flat
    allocation per (name, device, dtype), values unchanged; buffers whose id
    is in `keep` stay where they are.  A buffer object held under several
    names or states stays one object."""
    for name in names:
        groups: dict = {}
        for values in states:
            buffer = values.get(name)
            if isinstance(buffer, Tensor) and not buffer._requires_grad and id(buffer) not in keep:
                groups.setdefault((buffer._device, buffer._dtype), {})[id(buffer)] = buffer
        for (device, dtype), unique in groups.items():
            if len(unique) < 2:
                continue
            buffers = list(unique.values())
            views = _zeros_views([buffer.shape for buffer in buffers], dtype, device)
            moved = {}
            for buffer, view in zip(buffers, views):
                if isinstance(view._storage, DeviceArray):
                    view._storage.copy_from(buffer._storage)
                else:
                    np.copyto(view._storage, buffer._storage)
                moved[id(buffer)] = view
            for values in states:
                for key, buffer in values.items():
                    replacement = moved.get(id(buffer)) if isinstance(buffer, Tensor) else None
                    if replacement is not None:
                        values[key] = replacement


class _FirstOrderOptimizer(Optimizer):
    _state_buffers = ()
    _required_buffers = ()
    _has_step = False
    _nonnegative_buffers = ()
    _decoupled_weight_decay = False

    def _prepare_options(self, options: dict, path: str) -> dict:
        prepared = super()._prepare_options(options, path)
        _real_option(prepared, "lr")
        _real_option(prepared, "weight_decay")
        _bool_option(prepared, "maximize")
        return prepared

    # ---- state ------------------------------------------------------------------------
    def _install_loaded_state(self, defaults: dict, param_groups: list, state) -> None:
        # Loaded buffers are fresh copies; give them the contiguous layout the
        # step creates.
        _pack_state_buffers(list(state.values()), self._state_buffers)
        super()._install_loaded_state(defaults, param_groups, state)

    def to(self, device):
        # Buffers already on `device` are kept as they are (Tensor.to returns
        # them); only the moved copies are packed.
        before = [value for values in self.state.values() if isinstance(values, dict)
                  for value in values.values() if isinstance(value, Tensor)]
        moved = super().to(device)
        _pack_state_buffers(list(self.state.values()), self._state_buffers, keep={id(value) for value in before})
        return moved

    def _state_dtype(self, parameter: Tensor, name: str) -> DType:
        """dtype every state buffer must have (the parameter's by default)."""
        return parameter.dtype

    def _allowed_state(self) -> tuple[set, set]:
        allowed = set(self._state_buffers) | ({"step"} if self._has_step else set())
        required = set(self._required_buffers) | ({"step"} if self._has_step else set())
        return allowed, required

    def _check_state_cached(self, values: dict, parameter: Tensor) -> None:
        """``_check_state(..., runtime=True)`` for the step loop.

        Passing the check depends on which buffer objects the state holds
        (their dtype/shape/device never change), on ``step`` being a
        nonnegative int and on the nonnegative buffers having no negative
        element; the last is re-checked whenever a buffer's version shows a
        write by something other than this optimizer's kernels.
        """
        if not values:
            return
        cache = self.__dict__.setdefault("_state_checked", {})
        seen = cache.get(id(parameter))
        if seen is not None and seen[0] is values and len(values) == seen[1]:
            step = values.get("step", 0)
            unchanged = type(step) is int and step >= 0
            if unchanged:
                for name, buffer, nonnegative in seen[2]:
                    if (values.get(name) is not buffer or buffer._requires_grad or not buffer._writable
                            or (nonnegative and buffer._clean_version != buffer._version_counter.value)):
                        unchanged = False
                        break
            if unchanged:
                return
        self._check_state(values, parameter, "parameter state", runtime=True)
        cache[id(parameter)] = (values, len(values), tuple(
            (name, values[name], name in self._nonnegative_buffers) for name in self._state_buffers if name in values))

    def _check_state(self, values: dict, parameter: Tensor, path: str, runtime: bool = False) -> None:
        if not isinstance(values, dict):
            raise TypeError(f"{path} must be a dictionary.")
        if not values:
            return
        allowed, required = self._allowed_state()
        if not set(values) <= allowed or not required <= values.keys():
            raise ValueError(f"{path} has invalid state fields for {type(self).__name__}.")
        if self._has_step and (type(values["step"]) is not int or values["step"] < 0):
            raise ValueError(f"{path} step must be a nonnegative Python integer.")
        for name in self._state_buffers:
            if name not in values:
                continue
            value = values[name]
            if isinstance(value, Tensor):
                dtype = value.dtype
            elif isinstance(value, np.ndarray):
                dtype = from_numpy_dtype(value.dtype)
            elif is_device_array(value):
                dtype = DeviceArray.wrap(value).dtype
            else:
                raise TypeError(f"{path}[{name!r}] must be a floating Tensor or NumPy array.")
            if not dtype.is_floating_point:
                raise TypeError(f"{path}[{name!r}] must have a floating dtype.")
            if tuple(value.shape) != parameter.shape:
                raise ValueError(f"{path}[{name!r}] shape {tuple(value.shape)} must equal parameter shape {parameter.shape}.")
            if name in self._nonnegative_buffers and self._has_negative(value):
                raise ValueError(f"{path}[{name!r}] must be nonnegative.")
            if runtime:
                ensure_same_device(parameter, value)
                expected = self._state_dtype(parameter, name)
                if not isinstance(value, Tensor) or dtype is not expected:
                    raise TypeError(f"{path}[{name!r}] must be a Tensor with parameter dtype {expected.name}.")
                if value.requires_grad or not value._writable:
                    raise RuntimeError(f"{path}[{name!r}] must be writable and detached from autograd.")

    @staticmethod
    def _has_negative(value) -> bool:
        if isinstance(value, Tensor):
            if value._clean_version is not None and value._clean_version == value._version_counter.value:
                return False      # written only by this optimizer's kernels since the last check
            if value.device.type == "cpu":
                result = bool(np.any(np.less(value.numpy(), 0)))
            else:
                result = get_backend(value).any_negative(value._data, value.dtype.code)
            if not result:
                value._clean_version = value._version_counter.value
            return result
        if not isinstance(value, np.ndarray):
            array = DeviceArray.wrap(value)
            if array.dtype.code != -1:
                return get_backend(array).any_negative(array, array.dtype.code)
            value = array.download()
        return bool(np.any(np.less(value, 0)))

    def _prepare_state(self, values: dict, parameter: Tensor, path: str) -> dict:
        copied = super()._prepare_state(values, parameter, path)
        self._check_state(copied, parameter, path)
        if copied and not parameter.dtype.is_floating_point:
            raise TypeError("Nonfloating parameters cannot have optimizer accumulation buffers.")
        for name in self._state_buffers:
            if name in copied:
                copied[name] = Tensor(copied[name], dtype=self._state_dtype(parameter, name), device=parameter.device)
        return copied

    # ---- step ----------------------------------------------------------------------------
    def _compute_dtype(self, parameter: Tensor) -> DType:
        """dtype the update arithmetic (and its scalars) uses: the parameter's."""
        return parameter.dtype

    def _validate_entry(self, parameter: Tensor, prepared: dict, checked: set) -> None:
        key = (parameter.dtype, id(prepared))
        if key in checked:
            return
        dtype = self._compute_dtype(parameter)
        for name, value in prepared.items():
            if type(value) is float:
                _round_scalar(dtype, value, name)
        if self._decoupled_weight_decay:
            _round_scalar(dtype, 1 - prepared["lr"] * prepared["weight_decay"], "decay factor")
        checked.add(key)

    def step(self, closure=None):
        reject_during_capture("Optimizer steps")
        if closure is not None and not callable(closure):
            raise TypeError("Optimizer closure must be callable or None.")
        self._reconcile_device_steps()
        loss = None
        if closure is not None:
            with enable_grad():
                loss = closure()
        replay = self.__dict__.get("_replay")
        if replay is not None:
            with no_grad():
                if replay.run(self):
                    self._track_consumed_device_steps()
                    return loss
            self._replay = None
        entries = list(self._grad_entries())
        options = {
            id(group): self._prepare_options({key: value for key, value in group.items() if key != "params"}, "param_group")
            for group in self.param_groups
        }
        checked: set = set()
        validate_update = getattr(self, "_validate_update", None)
        states = self.state
        state_cache = self.__dict__.setdefault("_state_checked", {})
        items = []
        for group, parameter, gradient in entries:
            dtype = parameter._dtype
            if not dtype._floating:
                raise TypeError("Optimizer updates require floating parameters.")
            if not parameter._writable:
                raise RuntimeError("Optimizer cannot update read-only parameter storage.")
            prepared = options[id(group)]
            if (dtype, id(prepared)) not in checked:
                self._validate_entry(parameter, prepared, checked)
            values = states.get(id(parameter))
            if values:
                # Inline fast path of _check_state_cached (per tensor, per step).
                seen = state_cache.get(id(parameter))
                unchanged = seen is not None and seen[0] is values and len(values) == seen[1]
                if unchanged:
                    step = values.get("step", 0)
                    unchanged = type(step) is int and step >= 0
                    if unchanged:
                        for name, buffer, nonnegative in seen[2]:
                            if (values.get(name) is not buffer or buffer._requires_grad or not buffer._writable
                                    or (nonnegative and buffer._clean_version != buffer._version_counter.value)):
                                unchanged = False
                                break
                if not unchanged:
                    self._check_state_cached(values, parameter)
            if validate_update is not None:
                validate_update(parameter, gradient, prepared)
            items.append((parameter, gradient, prepared))
        with no_grad():
            self._update_many(items)
        self._memoize_step(options)
        self._track_consumed_device_steps()
        return loss

    def _memoize_step(self, options: dict) -> None:
        """Record what a later step may replay without the per-tensor checks
        (subclasses that launch multi-tensor kernels); `options` maps id(group)
        to the prepared options of this step."""

    def _update_many(self, items) -> None:
        """Apply the update to every (parameter, gradient, options) of a step."""
        update = getattr(self, "_update_parameter", None)
        if not callable(update):
            raise RuntimeError("Optimizer subclass must implement parameter updates.")
        for parameter, gradient, prepared in items:
            update(parameter, gradient, prepared)


__all__ = ["_FirstOrderOptimizer", "_real_option", "_bool_option", "_scalar", "_round_scalar"]
