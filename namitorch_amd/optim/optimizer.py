"""Optimizer base class.

Same public behaviour as ``namitorch/optim/optimizer.py:120-315``: parameter
groups, the gradient iterator and its checks (181-195), ``zero_grad``
(197-206), the versioned ``state_dict`` (211-233), ``load_state_dict``
(235-312) and ``to`` (288-309), with the same exception classes and messages.
"""

from __future__ import annotations

import weakref
from collections import defaultdict
from itertools import chain, compress, repeat
from operator import and_, attrgetter, eq, is_, is_not, itemgetter

import numpy as np
import torch

from ..backends import ensure_same_device
from ..backends._graph_capture import reject_during_capture
from ..device import Device
from ..dtype import from_numpy_dtype
from ..tensor import Parameter, Tensor, no_grad


_REQUIRES = attrgetter("_requires_grad")
_GRAD = attrgetter("_grad")
_DTYPE = attrgetter("_dtype")
_DEVICE = attrgetter("_device")
_STORAGE_SHAPE = attrgetter("_storage.shape")
_PARAMS = itemgetter("params")
_FIRST_OF = itemgetter(0)
_SECOND_OF = itemgetter(1)
_CALL_REF = weakref.ReferenceType.__call__


def _copy_value(value, path: str, parameter_shape=None, active=None):
    if isinstance(value, (Tensor, np.ndarray, torch.Tensor)):
        shape = tuple(value.shape)
        if parameter_shape is not None and shape not in ((), tuple(parameter_shape)):
            raise ValueError(f"{path} has shape {shape}; expected scalar state or parameter shape {tuple(parameter_shape)}.")
        if isinstance(value, Tensor):
            return Tensor(value, device=value.device)
        if isinstance(value, np.ndarray):
            from_numpy_dtype(value.dtype)
            return value.copy()
        return value.clone()
    if isinstance(value, np.generic):
        from_numpy_dtype(value.dtype)
        return value.item()
    if value is None or type(value) in (bool, int, float, str, bytes):
        return value
    if not isinstance(value, (dict, list, tuple)):
        raise TypeError(f"{path} contains unsupported optimizer state type {type(value).__name__}.")
    active = set() if active is None else active
    identity = id(value)
    if identity in active:
        raise ValueError(f"{path} contains a cyclic optimizer state container.")
    active.add(identity)
    try:
        if isinstance(value, dict):
            copied = {}
            for key, item in value.items():
                if type(key) not in (str, int):
                    raise TypeError(f"{path} dictionary keys must be strings or integers.")
                copied[key] = _copy_value(item, f"{path}[{key!r}]", parameter_shape, active)
            return copied
        copied = [_copy_value(item, f"{path}[{index}]", parameter_shape, active) for index, item in enumerate(value)]
        return tuple(copied) if isinstance(value, tuple) else copied
    finally:
        active.remove(identity)


def _move_state(value, device: Device, shape, path, memo, active):
    identity = id(value)
    if isinstance(value, (Tensor, np.ndarray, torch.Tensor)):
        if tuple(value.shape) not in ((), tuple(shape)):
            raise ValueError(f"{path} has incompatible optimizer state shape {tuple(value.shape)}; expected {tuple(shape)}.")
        if identity not in memo:
            if isinstance(value, Tensor):
                if value.requires_grad:
                    raise RuntimeError(f"{path} must be detached from autograd before migration.")
                memo[identity] = value.to(device)
            else:
                memo[identity] = Tensor(value, device=device)
        return memo[identity]
    if isinstance(value, np.generic):
        from_numpy_dtype(value.dtype)
        return value.item()
    if value is None or type(value) in (bool, int, float, str, bytes):
        return value
    if not isinstance(value, (dict, list, tuple)):
        raise TypeError(f"{path} contains unsupported optimizer state type {type(value).__name__}.")
    if identity in active:
        raise ValueError(f"{path} contains a cyclic optimizer state container.")
    active.add(identity)
    try:
        if isinstance(value, dict):
            if any(type(key) not in (str, int) for key in value):
                raise TypeError(f"{path} dictionary keys must be strings or integers.")
            return {key: _move_state(item, device, shape, f"{path}[{key!r}]", memo, active) for key, item in value.items()}
        result = [_move_state(item, device, shape, f"{path}[{index}]", memo, active) for index, item in enumerate(value)]
        return tuple(result) if isinstance(value, tuple) else result
    finally:
        active.remove(identity)


def _copy_options(options: dict, path: str) -> dict:
    if not isinstance(options, dict):
        raise TypeError(f"{path} must be a dictionary.")
    if any(not isinstance(key, str) or not key for key in options):
        raise TypeError(f"{path} option names must be nonempty strings.")
    if "params" in options:
        raise ValueError(f"{path} cannot contain the reserved option 'params'.")
    return _copy_value(options, path)


def _parameter_list(params, path: str, allow_single: bool = False) -> list:
    if allow_single and isinstance(params, Parameter):
        values = [params]
    else:
        if isinstance(params, (Tensor, dict, str, bytes, set, frozenset)):
            raise TypeError(f"{path} must be an ordered iterable of Parameters.")
        try:
            values = list(params)
        except TypeError:
            raise TypeError(f"{path} must be an ordered iterable of Parameters.") from None
    if not values:
        raise ValueError(f"{path} cannot be empty.")
    identities = set()
    for parameter in values:
        if not isinstance(parameter, Parameter):
            raise TypeError(f"{path} must contain only NamiTorch Parameters, got {type(parameter).__name__}.")
        if not parameter.is_leaf:
            raise ValueError(f"{path} must contain only leaf Parameters.")
        if id(parameter) in identities:
            raise ValueError(f"{path} contains a duplicate Parameter object.")
        identities.add(id(parameter))
    return values


class Optimizer:
    def __init__(self, params, defaults: dict | None = None):
        self.defaults = self._prepare_options({} if defaults is None else defaults, "defaults")
        self.state: dict[int, dict] = defaultdict(dict)
        self.param_groups: list[dict] = []
        if isinstance(params, (Tensor, dict, str, bytes, set, frozenset)):
            raise TypeError("Optimizer params must be an ordered iterable of Parameters or parameter-group dictionaries.")
        try:
            entries = list(params)
        except TypeError:
            raise TypeError("Optimizer params must be an ordered iterable of Parameters or parameter-group dictionaries.") from None
        if not entries:
            raise ValueError("Optimizer cannot receive an empty parameter list.")
        if all(isinstance(entry, dict) for entry in entries):
            groups = entries
        elif any(isinstance(entry, dict) for entry in entries):
            raise TypeError("Optimizer params cannot mix Parameters and parameter-group dictionaries.")
        else:
            groups = [{"params": entries}]
        for group in groups:
            self.add_param_group(group)

    def _prepare_options(self, options: dict, path: str) -> dict:
        return _copy_options(options, path)

    def _prepare_state(self, values: dict, parameter: Parameter, path: str) -> dict:
        return _copy_value(values, path, parameter.shape)

    def _registered_parameters(self) -> list:
        if not self.param_groups:
            raise ValueError("Optimizer must contain at least one parameter group.")
        # The structure check below is a pure function of which objects the
        # groups hold; skip it when that is unchanged since the last call.
        try:
            fingerprint = tuple(
                (id(group), id(group["params"]), tuple(map(id, group["params"])))
                if type(group) is dict and type(group.get("params")) is list else None
                for group in self.param_groups
            )
        except TypeError:
            fingerprint = None
        cached = self.__dict__.get("_registered_cache")
        if fingerprint is not None and cached is not None and cached[0] == fingerprint:
            return list(cached[1])
        parameters = []
        identities = set()
        for index, group in enumerate(self.param_groups):
            if not isinstance(group, dict) or "params" not in group:
                raise TypeError(f"Parameter group {index} must be a dictionary containing 'params'.")
            if not isinstance(group["params"], list):
                raise TypeError(f"Parameter group {index} params must remain a materialized list.")
            current = _parameter_list(group["params"], f"param_groups[{index}]['params']")
            for parameter in current:
                if id(parameter) in identities:
                    raise ValueError("A Parameter object cannot belong to more than one parameter group.")
                identities.add(id(parameter))
            parameters.extend(current)
        if fingerprint is not None and None not in fingerprint:
            self._registered_cache = (fingerprint, tuple(parameters))
        return parameters

    def add_param_group(self, param_group: dict) -> None:
        if not isinstance(param_group, dict):
            raise TypeError("add_param_group requires a dictionary.")
        if "params" not in param_group:
            raise ValueError("A parameter group must contain 'params'.")
        parameters = _parameter_list(param_group["params"], "param_group['params']", allow_single=True)
        existing = {id(parameter) for parameter in self._registered_parameters()} if self.param_groups else set()
        if any(id(parameter) in existing for parameter in parameters):
            raise ValueError("A Parameter object cannot belong to more than one parameter group.")
        options = _copy_options(self.defaults, "defaults")
        options.update(_copy_options({key: value for key, value in param_group.items() if key != "params"}, "param_group"))
        options = self._prepare_options(options, "param_group")
        options["params"] = parameters
        self.param_groups.append(options)

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
        if not (all(map(eq, map(_STORAGE_SHAPE, gradients), map(_STORAGE_SHAPE, parameters)))
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
                if not parameter._requires_grad:
                    continue
                gradient = parameter._grad
                if gradient is None:
                    continue
                seen = checked.get(id(parameter))
                if seen is not None and seen[0] is parameter and seen[1]() is gradient:
                    yield group, parameter, gradient
                    continue
                if not isinstance(gradient, Tensor):
                    raise TypeError("Parameter gradients must be NamiTorch Tensors.")
                if gradient._device is not parameter._device and gradient._device != parameter._device:
                    ensure_same_device(parameter, gradient)       # raises the device mismatch
                if gradient._storage.shape != parameter._storage.shape:
                    raise ValueError(f"Gradient shape {gradient.shape} does not match parameter shape {parameter.shape}.")
                if not self._gradient_dtype_ok(parameter, gradient):
                    raise TypeError(f"Gradient dtype {gradient.dtype} does not match parameter dtype {parameter.dtype}.")
                checked[id(parameter)] = (parameter, weakref.ref(gradient))
                yield group, parameter, gradient

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

    def _reconcile_device_steps(self) -> None:
        """Settle host state (step counts, version counters) of steps whose
        skip decision was taken on the device (``namitorch_amd.amp.fused_step``)."""
        pending = self.__dict__.get("_device_steps")
        if pending:
            for device_step in pending:
                device_step.reconcile()
            pending.clear()

    def state_dict(self) -> dict:
        self._reconcile_device_steps()
        parameters = self._registered_parameters()
        indices = {id(parameter): index for index, parameter in enumerate(parameters)}
        state = {}
        for identity, values in self.state.items():
            if type(identity) is not int or identity not in indices:
                raise ValueError("Optimizer state keys must be identities of registered Parameters.")
            if not isinstance(values, dict):
                raise TypeError("Each parameter's optimizer state must be a dictionary.")
            index = indices[identity]
            state[index] = self._prepare_state(values, parameters[index], f"state[{index}]")
        groups = []
        for index, group in enumerate(self.param_groups):
            copied = self._prepare_options({key: value for key, value in group.items() if key != "params"}, f"param_groups[{index}]")
            copied["params"] = [indices[id(parameter)] for parameter in group["params"]]
            groups.append(copied)
        return {
            "version": 1,
            "defaults": self._prepare_options(self.defaults, "defaults"),
            "param_groups": groups,
            "param_shapes": [list(parameter.shape) for parameter in parameters],
            "state": state,
        }

    def _prepare_load_state_dict(self, state_dict: dict):
        if not isinstance(state_dict, dict):
            raise TypeError("Optimizer state_dict must be a dictionary.")
        expected_keys = {"version", "defaults", "param_groups", "param_shapes", "state"}
        if set(state_dict) != expected_keys:
            raise ValueError("Optimizer state_dict must contain version, defaults, param_groups, param_shapes and state.")
        if type(state_dict["version"]) is not int or state_dict["version"] != 1:
            raise ValueError("Unsupported optimizer state_dict version.")
        parameters = self._registered_parameters()
        groups = state_dict["param_groups"]
        if not isinstance(groups, list) or len(groups) != len(self.param_groups):
            raise ValueError("Loaded optimizer must have the same number of parameter groups.")
        shapes = state_dict["param_shapes"]
        if not isinstance(shapes, list) or len(shapes) != len(parameters):
            raise ValueError("Loaded optimizer must contain one shape for each parameter.")
        defaults = self._prepare_options(state_dict["defaults"], "defaults")
        restored_groups = []
        index_to_parameter = {}
        for group_index, (saved, current) in enumerate(zip(groups, self.param_groups)):
            if not isinstance(saved, dict) or "params" not in saved:
                raise ValueError(f"Loaded parameter group {group_index} must contain 'params'.")
            saved_indices = saved["params"]
            if not isinstance(saved_indices, list) or len(saved_indices) != len(current["params"]):
                raise ValueError(f"Loaded parameter group {group_index} has a different number of parameters.")
            options = self._prepare_options({key: value for key, value in saved.items() if key != "params"}, f"param_groups[{group_index}]")
            if not defaults.keys() <= options.keys():
                raise ValueError(f"Loaded parameter group {group_index} is missing default options.")
            for index, parameter in zip(saved_indices, current["params"]):
                if type(index) is not int or not 0 <= index < len(parameters):
                    raise ValueError("Loaded parameter indices must be integers in the registered parameter range.")
                if index in index_to_parameter:
                    raise ValueError("Loaded parameter groups contain duplicate parameter indices.")
                shape = shapes[index]
                if not isinstance(shape, (list, tuple)) or any(type(dimension) is not int or dimension < 0 for dimension in shape):
                    raise ValueError(f"Invalid saved parameter shape for index {index}.")
                if tuple(shape) != parameter.shape:
                    raise ValueError(f"Saved parameter {index} shape {tuple(shape)} does not match current shape {parameter.shape}.")
                index_to_parameter[index] = parameter
            options["params"] = list(current["params"])
            restored_groups.append(options)
        saved_state = state_dict["state"]
        if not isinstance(saved_state, dict):
            raise TypeError("Loaded optimizer state must be a dictionary keyed by parameter indices.")
        restored_state = defaultdict(dict)
        for index, values in saved_state.items():
            if type(index) is not int or index not in index_to_parameter:
                raise ValueError("Loaded state keys must be registered parameter indices.")
            if not isinstance(values, dict):
                raise TypeError(f"Loaded state[{index}] must be a dictionary.")
            parameter = index_to_parameter[index]
            restored_state[id(parameter)] = self._prepare_state(values, parameter, f"state[{index}]")
        return defaults, restored_groups, restored_state

    def _install_loaded_state(self, defaults: dict, param_groups: list, state) -> None:
        """Replace options and state with a prepared load; device-side steps
        still in flight settle against the state they updated first."""
        self._reconcile_device_steps()
        self.defaults, self.param_groups, self.state = defaults, param_groups, state

    def load_state_dict(self, state_dict: dict) -> None:
        self._install_loaded_state(*self._prepare_load_state_dict(state_dict))

    def to(self, device):
        reject_during_capture("Moving optimizer state")
        target = Device(device)
        parameters = {id(parameter): parameter for parameter in self._registered_parameters()}
        if any(parameter.device != target for parameter in parameters.values()):
            raise RuntimeError(f"Move all optimizer parameters to {target} first with model.to(device); optimizer.to(device) moves only optimizer state.")
        staged = defaultdict(dict)
        memo = {}
        with no_grad():
            for identity, values in self.state.items():
                if type(identity) is not int or identity not in parameters:
                    raise ValueError("Optimizer state keys must identify registered Parameters.")
                if not isinstance(values, dict):
                    raise TypeError("Each parameter's optimizer state must be a dictionary.")
                parameter = parameters[identity]
                moved = _move_state(values, target, parameter.shape, "optimizer state", memo, set())
                validate = getattr(self, "_check_state", None)
                if validate is not None:
                    validate(moved, parameter, "optimizer state", runtime=True)
                staged[identity] = moved
        self.state = staged
        return self

    def __repr__(self) -> str:
        return f"{type(self).__name__}(param_groups={len(self.param_groups)})"


__all__ = ["Optimizer"]
