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

import weakref

from .. import _native
from ..backends import get_backend
from ..backends._settings import fused_kernels_enabled
from ..backends.hip import make_xform
from ..dtype import DType, bfloat16, float16, float32, float64, normalize_dtype
from ..tensor import GradTransform, Tensor
from ._common import _FirstOrderOptimizer, _real_option, _round_scalar

_LOW_PRECISION = (float16, bfloat16, float32)


def _zeros_like(parameter: Tensor, dtype: DType) -> Tensor:
    import torch
    return Tensor._from_storage(torch.zeros(parameter.shape, dtype=dtype.torch_dtype, device=parameter.device.torch))


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
            if master is not None:
                rows.append((master._ptr, gradient._ptr, first._ptr, second._ptr, parameter._ptr, parameter._numel, slot))
            else:
                rows.append((parameter._ptr, gradient._ptr, first._ptr, second._ptr, 0, parameter._numel, slot))
            bookkeeping.append((parameter, state, first, second, master, step, fused, options["lr"] != 0))
        slots = ((_native.AdamWCoefs64 if compute is float64 else _native.AdamWCoefs) * len(records))(*records)
        plan = backend.plan(rows, layout)
        backend.adamw_multi(plan, slots, None if transform is None else make_xform(transform))
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
            device_step.optimizers.add(self)


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
        supported = self._fused_decision_supported(parameter, gradient)
        if fused is True and not supported:
            raise RuntimeError("The parameter, gradient or optimizer state does not support fused AdamW.")
        return supported


__all__ = ["Adam", "AdamW"]
