"""Optimizer base class.

The public contract is ``namitorch/optim/optimizer.py:120-315``: parameter
groups and their validation, the gradient iterator with its device, shape
and dtype checks (181-195), ``zero_grad`` (197-206), the versioned
``state_dict`` (211-233), ``load_state_dict`` (235-312) and ``to``
(288-309), raising the same exception classes with the same messages in the
same order, so callers that catch them or persist these dictionaries work
unchanged.

How it is built here:

* one walker (:class:`_StateTree`) validates and rebuilds nested optimizer
  state for all three consumers — copying into and out of a state dict, and
  moving state to another device — with the array leaf handled by a
  per-use function;
* the registered-parameter list and the ``(group, parameter, gradient)``
  entries are memoized on object identity (a Tensor's device, shape and
  dtype never change), with the per-item iterator as the path that raises;
* ``state`` is a property: a step whose skip decision was taken on the device
  (``namitorch_amd.amp.fused_step``) leaves the host's step counts
  optimistic until its outcome is read back, and reading ``state`` settles
  that first, so ``optimizer.state[id(p)]["step"]`` is always the
  reference's value.
"""

from __future__ import annotations

import weakref
from collections import defaultdict
from itertools import chain, compress, repeat
from operator import and_, attrgetter, eq, is_, is_not, itemgetter

import numpy as np

from ..array import DeviceArray, is_device_array
from ..backends import ensure_same_device
from ..backends._graph_capture import reject_during_capture
from ..device import Device
from ..dtype import from_numpy_dtype
from ..tensor import Parameter, Tensor, no_grad


_REQUIRES = attrgetter("_requires_grad")
_GRAD = attrgetter("_grad")
_DTYPE = attrgetter("_dtype")
_DEVICE = attrgetter("_device")
_SHAPE = attrgetter("_shape")
_PARAMS = itemgetter("params")
_FIRST_OF = itemgetter(0)
_SECOND_OF = itemgetter(1)
_CALL_REF = weakref.ReferenceType.__call__

_ARRAY_TYPES = (Tensor, np.ndarray, DeviceArray)


def _is_array(value) -> bool:
    """A Tensor, a NumPy array or a device array (ours or another framework's)."""
    return isinstance(value, _ARRAY_TYPES) or is_device_array(value)

_PASS_THROUGH = (bool, int, float, str, bytes)
_KEY_TYPES = (str, int)


class _StateTree:
    """Validating rebuild of one optimizer-state value.

    Array leaves (Tensors and storage arrays) go to ``leaf(value, path)``;
    NumPy scalars become Python scalars after their dtype is checked; None
    and plain Python scalars are kept; dicts, lists and tuples are rebuilt
    (keys must be strings or integers, cycles are rejected); anything else
    is a TypeError.  ``keys_first`` checks all keys of a dictionary before
    any of its values (the migration order), otherwise each key just before
    its value (the copy order)."""

    __slots__ = ("leaf", "keys_first", "open")

    def __init__(self, leaf, keys_first: bool):
        self.leaf = leaf
        self.keys_first = keys_first
        self.open: set = set()

    def rebuild(self, value, path: str):
        if _is_array(value):
            return self.leaf(value, path)
        if isinstance(value, np.generic):
            from_numpy_dtype(value.dtype)
            return value.item()
        if value is None or type(value) in _PASS_THROUGH:
            return value
        if not isinstance(value, (dict, list, tuple)):
            raise TypeError(f"{path} contains unsupported optimizer state type {type(value).__name__}.")
        marker = id(value)
        if marker in self.open:
            raise ValueError(f"{path} contains a cyclic optimizer state container.")
        self.open.add(marker)
        try:
            if isinstance(value, dict):
                return self._mapping(value, path)
            rebuilt = [self.rebuild(item, f"{path}[{position}]") for position, item in enumerate(value)]
            return tuple(rebuilt) if isinstance(value, tuple) else rebuilt
        finally:
            self.open.discard(marker)

    def _mapping(self, value: dict, path: str) -> dict:
        if self.keys_first and not all(type(key) in _KEY_TYPES for key in value):
            raise TypeError(f"{path} dictionary keys must be strings or integers.")
        rebuilt = {}
        for key, item in value.items():
            if type(key) not in _KEY_TYPES:
                raise TypeError(f"{path} dictionary keys must be strings or integers.")
            rebuilt[key] = self.rebuild(item, f"{path}[{key!r}]")
        return rebuilt


def _copy_leaf(parameter_shape):
    """Leaf function of a state copy: an independent copy of every array,
    optionally checked to be a scalar or of the parameter's shape."""
    expected = None if parameter_shape is None else tuple(parameter_shape)

    def copy(value, path):
        shape = tuple(value.shape)
        if expected is not None and shape != () and shape != expected:
            raise ValueError(f"{path} has shape {shape}; expected scalar state or parameter shape {expected}.")
        if isinstance(value, Tensor):
            return Tensor(value, device=value.device)
        if isinstance(value, np.ndarray):
            from_numpy_dtype(value.dtype)
            return value.copy()
        return DeviceArray.wrap(value).clone()

    return copy


def _copy_state(value, path: str, parameter_shape=None):
    return _StateTree(_copy_leaf(parameter_shape), keys_first=False).rebuild(value, path)


def _move_leaf(device: Device, shape, memo: dict):
    """Leaf function of a migration: each array object moves once (``memo``
    by identity, so buffers shared between entries stay shared)."""
    expected = tuple(shape)

    def move(value, path):
        found = tuple(value.shape)
        if found != () and found != expected:
            raise ValueError(f"{path} has incompatible optimizer state shape {found}; expected {expected}.")
        key = id(value)
        if key not in memo:
            if isinstance(value, Tensor):
                if value.requires_grad:
                    raise RuntimeError(f"{path} must be detached from autograd before migration.")
                memo[key] = value.to(device)
            else:
                memo[key] = Tensor(value, device=device)
        return memo[key]

    return move


def _checked_options(options, path: str) -> dict:
    """A validated copy of a group's (or the defaults') options."""
    if not isinstance(options, dict):
        raise TypeError(f"{path} must be a dictionary.")
    for name in options:
        if not isinstance(name, str) or not name:
            raise TypeError(f"{path} option names must be nonempty strings.")
    if "params" in options:
        raise ValueError(f"{path} cannot contain the reserved option 'params'.")
    return _copy_state(options, path)


def _collect_parameters(params, path: str, allow_single: bool = False) -> list:
    """The Parameters of one group, in order: leaves, each object once."""
    if allow_single and isinstance(params, Parameter):
        collected = [params]
    elif isinstance(params, (Tensor, dict, str, bytes, set, frozenset)):
        raise TypeError(f"{path} must be an ordered iterable of Parameters.")
    else:
        try:
            collected = list(params)
        except TypeError:
            raise TypeError(f"{path} must be an ordered iterable of Parameters.") from None
    if not collected:
        raise ValueError(f"{path} cannot be empty.")
    seen: set = set()
    for parameter in collected:
        if not isinstance(parameter, Parameter):
            raise TypeError(f"{path} must contain only NamiTorch Parameters, got {type(parameter).__name__}.")
        if not parameter.is_leaf:
            raise ValueError(f"{path} must contain only leaf Parameters.")
        if id(parameter) in seen:
            raise ValueError(f"{path} contains a duplicate Parameter object.")
        seen.add(id(parameter))
    return collected


def _valid_shape(shape) -> bool:
    return isinstance(shape, (list, tuple)) and all(type(size) is int and size >= 0 for size in shape)


class Optimizer:
    def __init__(self, params, defaults: dict | None = None):
        self.defaults = self._prepare_options({} if defaults is None else defaults, "defaults")
        self.state = defaultdict(dict)
        self.param_groups: list[dict] = []
        for group in self._initial_groups(params):
            self.add_param_group(group)

    @staticmethod
    def _initial_groups(params) -> list:
        described = "Optimizer params must be an ordered iterable of Parameters or parameter-group dictionaries."
        if isinstance(params, (Tensor, dict, str, bytes, set, frozenset)):
            raise TypeError(described)
        try:
            entries = list(params)
        except TypeError:
            raise TypeError(described) from None
        if not entries:
            raise ValueError("Optimizer cannot receive an empty parameter list.")
        dictionaries = sum(isinstance(entry, dict) for entry in entries)
        if dictionaries == len(entries):
            return entries
        if dictionaries:
            raise TypeError("Optimizer params cannot mix Parameters and parameter-group dictionaries.")
        return [{"params": entries}]

    # ---- per-parameter state ------------------------------------------------------------
    @property
    def state(self):
        """Per-parameter state keyed by ``id(parameter)``; steps decided on the
        device are settled before it is handed out."""
        if self.__dict__.get("_device_steps"):
            self._reconcile_device_steps()
        return self.__dict__["_state"]

    @state.setter
    def state(self, value) -> None:
        self.__dict__["_state"] = value

    def _reconcile_device_steps(self) -> None:
        """Settle host state (step counts, version counters) of steps whose
        skip decision was taken on the device (``namitorch_amd.amp.fused_step``)."""
        pending = self.__dict__.get("_device_steps")
        if pending:
            for device_step in pending:
                device_step.reconcile()
            pending.clear()

    def _track_device_step(self, device_step) -> None:
        """Settle `device_step` (a device-decided step or clip whose gradient
        transform a finished step of this optimizer consumed) before this
        optimizer's next step or state read."""
        pending = self.__dict__.setdefault("_device_steps", [])
        if not any(map(is_, pending, repeat(device_step))):
            pending.append(device_step)

    def _consume_device_step(self, device_step) -> None:
        """Note, during a step, that its pass reads `device_step`'s decisions.
        It is tracked only once the step has finished
        (``_track_consumed_device_steps``): the step's own state reads would
        otherwise settle it before its bookkeeping is complete."""
        self.__dict__.setdefault("_consumed_device_steps", []).append(device_step)

    def _track_consumed_device_steps(self) -> None:
        consumed = self.__dict__.pop("_consumed_device_steps", None)
        if consumed:
            for device_step in consumed:
                self._track_device_step(device_step)

    # ---- hooks for subclasses ------------------------------------------------------------
    def _prepare_options(self, options: dict, path: str) -> dict:
        return _checked_options(options, path)

    def _prepare_state(self, values: dict, parameter: Parameter, path: str) -> dict:
        return _copy_state(values, path, parameter.shape)

    # ---- parameter groups --------------------------------------------------------------------
    def _group_fingerprint(self):
        """Which objects the groups hold (None when a group is not a plain
        dict with a list of params: the full check then runs)."""
        try:
            return tuple(
                (id(group), id(group["params"]), tuple(map(id, group["params"])))
                if type(group) is dict and type(group.get("params")) is list else None
                for group in self.param_groups
            )
        except TypeError:
            return None

    def _groups_unchanged(self, cached) -> bool:
        """The groups hold what they held when `cached` was built: the same
        dict objects with the same params list objects, each of the same
        length and with the same items (by identity).  Equivalent to an equal
        fingerprint, without building one."""
        groups, lists, lengths = cached[2], cached[3], cached[4]
        current = self.param_groups
        if type(current) is not list or len(current) != len(groups) or not all(map(is_, current, groups)):
            return False
        try:
            if not all(map(is_, map(_PARAMS, groups), lists)):
                return False
        except KeyError:
            return False
        return tuple(map(len, lists)) == lengths and all(map(is_, chain.from_iterable(lists), cached[1]))

    def _registered_parameters(self) -> list:
        if not self.param_groups:
            raise ValueError("Optimizer must contain at least one parameter group.")
        # The structure check is a pure function of which objects the groups
        # hold; it is skipped while that is unchanged since the last call.
        cached = self.__dict__.get("_registered_cache")
        if cached is not None and self._groups_unchanged(cached):
            return list(cached[1])
        fingerprint = self._group_fingerprint()
        if fingerprint is not None and cached is not None and cached[0] == fingerprint:
            return list(cached[1])
        registered: list = []
        owners: set = set()
        for position, group in enumerate(self.param_groups):
            if not isinstance(group, dict) or "params" not in group:
                raise TypeError(f"Parameter group {position} must be a dictionary containing 'params'.")
            if not isinstance(group["params"], list):
                raise TypeError(f"Parameter group {position} params must remain a materialized list.")
            for parameter in _collect_parameters(group["params"], f"param_groups[{position}]['params']"):
                if id(parameter) in owners:
                    raise ValueError("A Parameter object cannot belong to more than one parameter group.")
                owners.add(id(parameter))
                registered.append(parameter)
        if fingerprint is not None and None not in fingerprint:
            groups = tuple(self.param_groups)
            lists = tuple(map(_PARAMS, groups))
            self._registered_cache = (fingerprint, tuple(registered), groups, lists, tuple(map(len, lists)))
        return registered

    def add_param_group(self, param_group: dict) -> None:
        if not isinstance(param_group, dict):
            raise TypeError("add_param_group requires a dictionary.")
        if "params" not in param_group:
            raise ValueError("A parameter group must contain 'params'.")
        members = _collect_parameters(param_group["params"], "param_group['params']", allow_single=True)
        if self.param_groups:
            taken = set(map(id, self._registered_parameters()))
            if not taken.isdisjoint(map(id, members)):
                raise ValueError("A Parameter object cannot belong to more than one parameter group.")
        merged = _checked_options(self.defaults, "defaults")
        merged.update(_checked_options({name: value for name, value in param_group.items() if name != "params"},
                                       "param_group"))
        group = self._prepare_options(merged, "param_group")
        group["params"] = members
        self.param_groups.append(group)

    # ---- gradients ----------------------------------------------------------------------------
    def _gradient_dtype_ok(self, parameter: Tensor, gradient: Tensor) -> bool:
        """Gradients must have the parameter's dtype (optimizer.py:193-194)."""
        return gradient.dtype is parameter.dtype

    def _gradient_dtypes_ok(self, parameters: tuple, gradients: tuple) -> bool:
        """``_gradient_dtype_ok`` for every pair, in C-level passes."""
        return all(map(is_, map(_DTYPE, gradients), map(_DTYPE, parameters)))

    def _bulk_entries(self, registered, requires: tuple, grads: tuple) -> tuple | None:
        """The entries of ``_parameters_with_grad`` with its checks done as
        C-level passes over all gradients at once; None when any check fails,
        and the iterator then raises the first failure in its own order."""
        mask = tuple(map(and_, requires, map(is_not, grads, repeat(None))))
        parameters = tuple(compress(registered, mask))
        gradients = tuple(compress(grads, mask))
        if not all(map(isinstance, gradients, repeat(Tensor))):
            return None
        devices = tuple(map(_DEVICE, gradients)), tuple(map(_DEVICE, parameters))
        if not (all(map(is_, *devices)) or all(map(eq, *devices))):
            return None
        if not (all(map(eq, map(_SHAPE, gradients), map(_SHAPE, parameters)))
                and self._gradient_dtypes_ok(parameters, gradients)):
            return None
        groups = self.param_groups
        owners = chain.from_iterable(map(repeat, groups, map(len, map(_PARAMS, groups))))
        return tuple(zip(compress(owners, mask), parameters, gradients))

    def _parameters_with_grad(self):
        self._registered_parameters()
        # A (parameter, gradient) pair that passed the checks once passes them
        # again: device, shape and dtype of a Tensor never change.  Gradients
        # are held weakly so the cache keeps no old gradient alive.
        checked = self.__dict__.setdefault("_checked_grads", {})
        for group in self.param_groups:
            for parameter in group["params"]:
                if not parameter._requires_grad or parameter._grad is None:
                    continue
                gradient = parameter._grad
                known = checked.get(id(parameter))
                if known is None or known[0] is not parameter or known[1]() is not gradient:
                    self._check_gradient(parameter, gradient)
                    checked[id(parameter)] = (parameter, weakref.ref(gradient))
                yield group, parameter, gradient

    def _check_gradient(self, parameter: Tensor, gradient) -> None:
        if not isinstance(gradient, Tensor):
            raise TypeError("Parameter gradients must be NamiTorch Tensors.")
        if gradient._device is not parameter._device and gradient._device != parameter._device:
            ensure_same_device(parameter, gradient)       # raises the device mismatch
        if gradient._shape != parameter._shape:
            raise ValueError(f"Gradient shape {gradient.shape} does not match parameter shape {parameter.shape}.")
        if not self._gradient_dtype_ok(parameter, gradient):
            raise TypeError(f"Gradient dtype {gradient.dtype} does not match parameter dtype {parameter.dtype}.")

    def _grad_entries(self) -> tuple:
        """``tuple(self._parameters_with_grad())``, memoized.

        The entries are a pure function of the registered parameters, their
        ``requires_grad`` flags and the gradient objects they hold (a
        Tensor's device, shape and dtype never change).  When all three are
        unchanged since the last call the entries are rebuilt from the memo
        with C-level passes; anything else runs the iterator, which raises
        its errors.  Gradients are held through weak references, so the memo
        keeps no old gradient alive."""
        registered = self._registered_parameters()
        cache = self.__dict__.get("_registered_cache")
        requires = tuple(map(_REQUIRES, registered))
        grads = tuple(map(_GRAD, registered))
        # Which parameters have a gradient is part of the key; the memo
        # holds references to those gradients only.
        present = tuple(map(is_not, grads, repeat(None)))
        memo = self.__dict__.get("_entries_memo")
        if (memo is not None and memo[0] is cache and memo[1] == requires and memo[2] == present
                and all(map(is_, compress(grads, present), map(_CALL_REF, memo[3])))):
            self.__dict__["_entries_served"] = memo    # these entries follow this memo
            return tuple(zip(memo[4], memo[5], compress(grads, memo[6])))
        self.__dict__["_entries_served"] = None
        entries = self._bulk_entries(registered, requires, grads)
        if entries is None:
            entries = tuple(self._parameters_with_grad())
        if cache is not None and self.__dict__.get("_registered_cache") is cache:
            refs = tuple(map(weakref.ref, compress(grads, present)))
            mask = tuple(map(and_, requires, present))
            memo = (cache, requires, present, refs, tuple(map(_FIRST_OF, entries)),
                    tuple(map(_SECOND_OF, entries)), mask)
            self.__dict__["_entries_memo"] = self.__dict__["_entries_served"] = memo
        return entries

    def zero_grad(self, set_to_none: bool = True) -> None:
        if type(set_to_none) is not bool:
            raise TypeError("set_to_none must be a Python bool.")
        parameters = self._registered_parameters()
        if set_to_none:
            for parameter in parameters:
                parameter._grad = None
            return
        from ..grads import zero_grads
        with no_grad():
            zero_grads([parameter.grad for parameter in parameters if parameter.grad is not None])

    def step(self, closure=None):
        raise RuntimeError("Optimizer subclass must implement step.")

    # ---- state dictionaries ---------------------------------------------------------------------
    def state_dict(self) -> dict:
        parameters = self._registered_parameters()
        position = {id(parameter): index for index, parameter in enumerate(parameters)}
        saved_state = {}
        for key, values in self.state.items():
            index = position.get(key) if type(key) is int else None
            if index is None:
                raise ValueError("Optimizer state keys must be identities of registered Parameters.")
            if not isinstance(values, dict):
                raise TypeError("Each parameter's optimizer state must be a dictionary.")
            saved_state[index] = self._prepare_state(values, parameters[index], f"state[{index}]")
        saved_groups = []
        for number, group in enumerate(self.param_groups):
            options = self._prepare_options({name: value for name, value in group.items() if name != "params"},
                                            f"param_groups[{number}]")
            options["params"] = [position[id(parameter)] for parameter in group["params"]]
            saved_groups.append(options)
        return {
            "version": 1,
            "defaults": self._prepare_options(self.defaults, "defaults"),
            "param_groups": saved_groups,
            "param_shapes": [list(parameter.shape) for parameter in parameters],
            "state": saved_state,
        }

    def _prepare_load_state_dict(self, state_dict: dict):
        """Validate a saved state against this optimizer and build the
        replacement (defaults, groups, state) without changing anything."""
        self._check_saved_layout(state_dict)
        parameters = self._registered_parameters()
        groups, shapes = state_dict["param_groups"], state_dict["param_shapes"]
        if not isinstance(groups, list) or len(groups) != len(self.param_groups):
            raise ValueError("Loaded optimizer must have the same number of parameter groups.")
        if not isinstance(shapes, list) or len(shapes) != len(parameters):
            raise ValueError("Loaded optimizer must contain one shape for each parameter.")
        defaults = self._prepare_options(state_dict["defaults"], "defaults")
        owner_of: dict = {}
        restored_groups = [self._restore_group(number, saved, current, defaults, shapes, len(parameters), owner_of)
                           for number, (saved, current) in enumerate(zip(groups, self.param_groups))]
        return defaults, restored_groups, self._restore_state(state_dict["state"], owner_of)

    @staticmethod
    def _check_saved_layout(state_dict) -> None:
        if not isinstance(state_dict, dict):
            raise TypeError("Optimizer state_dict must be a dictionary.")
        if set(state_dict) != {"version", "defaults", "param_groups", "param_shapes", "state"}:
            raise ValueError("Optimizer state_dict must contain version, defaults, param_groups, param_shapes and state.")
        if type(state_dict["version"]) is not int or state_dict["version"] != 1:
            raise ValueError("Unsupported optimizer state_dict version.")

    def _restore_group(self, number: int, saved, current: dict, defaults: dict, shapes: list, count: int,
                       owner_of: dict) -> dict:
        """One saved group matched to the current one; records which current
        parameter each saved index now names in `owner_of`."""
        if not isinstance(saved, dict) or "params" not in saved:
            raise ValueError(f"Loaded parameter group {number} must contain 'params'.")
        indices = saved["params"]
        if not isinstance(indices, list) or len(indices) != len(current["params"]):
            raise ValueError(f"Loaded parameter group {number} has a different number of parameters.")
        options = self._prepare_options({name: value for name, value in saved.items() if name != "params"},
                                        f"param_groups[{number}]")
        if not defaults.keys() <= options.keys():
            raise ValueError(f"Loaded parameter group {number} is missing default options.")
        for index, parameter in zip(indices, current["params"]):
            if type(index) is not int or not 0 <= index < count:
                raise ValueError("Loaded parameter indices must be integers in the registered parameter range.")
            if index in owner_of:
                raise ValueError("Loaded parameter groups contain duplicate parameter indices.")
            shape = shapes[index]
            if not _valid_shape(shape):
                raise ValueError(f"Invalid saved parameter shape for index {index}.")
            if tuple(shape) != parameter.shape:
                raise ValueError(f"Saved parameter {index} shape {tuple(shape)} does not match current shape {parameter.shape}.")
            owner_of[index] = parameter
        options["params"] = list(current["params"])
        return options

    def _restore_state(self, saved_state, owner_of: dict):
        if not isinstance(saved_state, dict):
            raise TypeError("Loaded optimizer state must be a dictionary keyed by parameter indices.")
        restored = defaultdict(dict)
        for index, values in saved_state.items():
            parameter = owner_of.get(index) if type(index) is int else None
            if parameter is None:
                raise ValueError("Loaded state keys must be registered parameter indices.")
            if not isinstance(values, dict):
                raise TypeError(f"Loaded state[{index}] must be a dictionary.")
            restored[id(parameter)] = self._prepare_state(values, parameter, f"state[{index}]")
        return restored

    def _install_loaded_state(self, defaults: dict, param_groups: list, state) -> None:
        """Replace options and state with a prepared load; device-side steps
        still in flight settle against the state they updated first."""
        self._reconcile_device_steps()
        self.defaults, self.param_groups, self.state = defaults, param_groups, state

    def load_state_dict(self, state_dict: dict) -> None:
        self._install_loaded_state(*self._prepare_load_state_dict(state_dict))

    # ---- migration --------------------------------------------------------------------------------
    def to(self, device):
        reject_during_capture("Moving optimizer state")
        target = Device(device)
        by_identity = {id(parameter): parameter for parameter in self._registered_parameters()}
        if any(parameter.device != target for parameter in by_identity.values()):
            raise RuntimeError(f"Move all optimizer parameters to {target} first with model.to(device); optimizer.to(device) moves only optimizer state.")
        moved_state = defaultdict(dict)
        moved_arrays: dict = {}
        validate = getattr(self, "_check_state", None)
        with no_grad():
            for key, values in self.state.items():
                parameter = by_identity.get(key) if type(key) is int else None
                if parameter is None:
                    raise ValueError("Optimizer state keys must identify registered Parameters.")
                if not isinstance(values, dict):
                    raise TypeError("Each parameter's optimizer state must be a dictionary.")
                tree = _StateTree(_move_leaf(target, parameter.shape, moved_arrays), keys_first=True)
                moved = tree.rebuild(values, "optimizer state")
                if validate is not None:
                    validate(moved, parameter, "optimizer state", runtime=True)
                moved_state[key] = moved
        self.state = moved_state
        return self

    def __repr__(self) -> str:
        return f"{type(self).__name__}(param_groups={len(self.param_groups)})"


__all__ = ["Optimizer"]
