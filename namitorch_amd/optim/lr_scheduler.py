"""Learning-rate schedules over optimizer parameter groups.

Contract: the classes, arguments, rates, state dictionaries and messages of
``namitorch/optim/lr_scheduler.py:37-272`` (LRScheduler, StepLR,
MultiStepLR, ExponentialLR, CosineAnnealingLR, LinearLR, WarmupCosine).
Each rate is a Python float computed on the host with the reference's
expression, operation for operation, because AdamW rounds ``lr`` and
``1 - lr * weight_decay`` to the parameter dtype from exactly that float.

Structure: each schedule declares its configuration as an ordered list of
field rules (``_FIELDS``: a name and its validator, or a check across the
fields validated so far) and a rate rule — a factor applied to every base
rate, or a fraction of the way from a floor to each base rate.  The base
class does the rest: validation in rule order, the rate checks, applying
rates to the groups, and the state dictionary.

Device-side skips: after ``amp.fused_step`` the host does not yet know
whether the step updated (the skip is decided on the GPU).  A scheduler
passed to ``fused_step`` is advanced when that step is reconciled — at the
start of the next optimizer step, or at the first read of the schedule
(``get_lr``, ``get_last_lr``, ``step``, ``state_dict``) — and only if the
step updated, which is the training loop's ``if updated:
scheduler.step()`` (training/runner.py:250-254) without a host
synchronisation.  Rates are never computed on the device: the cosine and
power functions would have to match the host C library bit for bit.
"""

from __future__ import annotations

import math
from bisect import bisect_right
from copy import deepcopy
from numbers import Integral, Real

from .optimizer import Optimizer


# ---- value rules -------------------------------------------------------------------------
def _integer(value, name: str, minimum: int = 0) -> int:
    if isinstance(value, bool) or not isinstance(value, Integral):
        raise TypeError(f"{name} must be an integer.")
    value = int(value)
    if value < minimum:
        raise ValueError(f"{name} must be at least {minimum}.")
    return value


def _rate(value, name: str) -> float:
    if isinstance(value, bool) or not isinstance(value, Real):
        raise TypeError(f"{name} must be a finite nonnegative real scalar.")
    try:
        value = float(value)
    except OverflowError:
        raise ValueError(f"{name} must be finite.") from None
    if not math.isfinite(value) or value < 0:
        raise ValueError(f"{name} must be finite and nonnegative.")
    return value


def _count(minimum: int):
    return lambda value, name: _integer(value, name, minimum)


def _milestones(value, name):
    if not isinstance(value, (list, tuple)):
        raise TypeError("milestones must be a list or tuple of integers.")
    return sorted(_integer(item, "milestone") for item in value)


def _toward(base_lrs, floor: float, fraction: float) -> list:
    """floor + (base - floor) * fraction for every group (cosine families)."""
    if any(floor > base for base in base_lrs):
        raise ValueError("Minimum learning rate cannot exceed a group's base learning rate.")
    return [floor + (base - floor) * fraction for base in base_lrs]


def _half_cosine(progress: float) -> float:
    return (1 + math.cos(math.pi * progress)) / 2


class LRScheduler:
    """Constant schedule; subclasses add field rules and a rate rule."""

    # (name, validator(value, name)) in validation order; a rule whose name
    # is None is a check over the fields validated before it.
    _FIELDS: tuple = ()

    def __init_subclass__(cls, **kwargs):
        super().__init_subclass__(**kwargs)
        cls._config_keys = tuple(name for name, _ in cls._FIELDS if name is not None)

    _config_keys: tuple = ()

    def __init__(self, optimizer: Optimizer, last_step: int = 0, **configuration):
        if not isinstance(optimizer, Optimizer):
            raise TypeError("Scheduler optimizer must be a NamiTorch Optimizer.")
        optimizer._registered_parameters()
        step = _integer(last_step, "last_step")
        config = self._normalize_config(configuration)
        bases = [self._group_base(group) for group in optimizer.param_groups]
        rates = self._checked_lrs(step, bases, config)
        self.optimizer = optimizer
        self.base_lrs = bases
        self.last_step = step
        self._group_signature = self._signature()
        self.__dict__.update(config)
        self._apply(rates)

    @staticmethod
    def _group_base(group: dict) -> float:
        if "lr" not in group:
            raise ValueError("Every optimizer parameter group must define lr.")
        _rate(group["lr"], "lr")
        return _rate(group.get("initial_lr", group["lr"]), "initial_lr")

    # ---- configuration ------------------------------------------------------------------
    @classmethod
    def _normalize_config(cls, config: dict) -> dict:
        if not isinstance(config, dict) or set(config) != set(cls._config_keys):
            raise ValueError(f"{cls.__name__} configuration must contain {cls._config_keys}.")
        checked = deepcopy(config)
        for name, rule in cls._FIELDS:
            if name is None:
                rule(checked)
            else:
                checked[name] = rule(checked[name], name)
        return checked

    def _configuration(self) -> dict:
        return self._normalize_config({name: getattr(self, name) for name in self._config_keys})

    def _signature(self):
        return tuple(tuple(map(id, group["params"])) for group in self.optimizer.param_groups)

    def _validate_groups(self) -> None:
        self.optimizer._registered_parameters()
        if self._signature() != self._group_signature or len(self.base_lrs) != len(self.optimizer.param_groups):
            raise RuntimeError("Optimizer parameter groups changed after scheduler construction; create a new scheduler.")

    # ---- rates ----------------------------------------------------------------------------
    def _compute_lrs(self, step: int, base_lrs: list, config: dict) -> list:
        return list(base_lrs)

    def _checked_lrs(self, step: int, base_lrs: list, config: dict) -> list:
        try:
            rates = self._compute_lrs(step, base_lrs, config)
        except OverflowError:
            raise ValueError("Scheduled learning rate exceeds the finite supported range.") from None
        return [_rate(value, "scheduled lr") for value in rates]

    def _bases(self) -> list:
        return [_rate(value, "base_lr") for value in self.base_lrs]

    def _apply(self, rates: list) -> None:
        for group, base, value in zip(self.optimizer.param_groups, self.base_lrs, rates):
            group["initial_lr"] = base
            group["lr"] = value
        self._last_lr = list(rates)

    def _settle(self) -> None:
        """Fold in fused steps whose update/skip outcome is still on the device."""
        self.optimizer._reconcile_device_steps()

    def get_lr(self) -> list:
        self._settle()
        self._validate_groups()
        return self._checked_lrs(_integer(self.last_step, "last_step"), self._bases(), self._configuration())

    def get_last_lr(self) -> list:
        self._settle()
        return list(self._last_lr)

    def step(self) -> None:
        self._settle()
        self._advance()

    def _advance(self) -> None:
        self._validate_groups()
        following = _integer(self.last_step, "last_step") + 1
        self._apply(self._checked_lrs(following, self._bases(), self._configuration()))
        self.last_step = following

    # ---- state ----------------------------------------------------------------------------
    def state_dict(self) -> dict:
        self.get_lr()
        return {
            "version": 1,
            "scheduler": type(self).__name__,
            "last_step": int(self.last_step),
            "base_lrs": self._bases(),
            "config": self._configuration(),
        }

    def _prepare_load_state_dict(self, state: dict):
        self._settle()
        self._validate_groups()
        if not isinstance(state, dict):
            raise TypeError("Scheduler state must be a dictionary.")
        if set(state) != {"version", "scheduler", "last_step", "base_lrs", "config"}:
            raise ValueError("Invalid scheduler state fields.")
        if type(state["version"]) is not int or state["version"] != 1:
            raise ValueError("Unsupported scheduler state version.")
        if state["scheduler"] != type(self).__name__:
            raise ValueError("Saved scheduler type does not match the current scheduler.")
        step = _integer(state["last_step"], "last_step")
        saved_bases = state["base_lrs"]
        if not isinstance(saved_bases, list) or len(saved_bases) != len(self.optimizer.param_groups):
            raise ValueError("Saved base_lrs must match the optimizer parameter group count.")
        bases = [_rate(value, "base_lr") for value in saved_bases]
        config = self._normalize_config(state["config"])
        return step, bases, config, self._checked_lrs(step, bases, config)

    def _apply_loaded_state(self, prepared) -> None:
        step, bases, config, rates = prepared
        self.base_lrs = bases
        self.last_step = step
        self.__dict__.update(config)
        self._apply(rates)

    def load_state_dict(self, state: dict) -> None:
        self._apply_loaded_state(self._prepare_load_state_dict(state))


class _ScaledSchedule(LRScheduler):
    """Rates are base * factor(step) for every group."""

    def _factor(self, step: int, config: dict) -> float:
        raise NotImplementedError

    def _compute_lrs(self, step, base_lrs, config):
        factor = self._factor(step, config)
        return [base * factor for base in base_lrs]


class StepLR(_ScaledSchedule):
    """base * gamma ** (step // step_size)."""

    _FIELDS = (("step_size", _count(1)), ("gamma", _rate))

    def __init__(self, optimizer: Optimizer, step_size: int, gamma: float = 0.1, last_step: int = 0):
        super().__init__(optimizer, last_step, step_size=step_size, gamma=gamma)

    def _factor(self, step, config):
        return config["gamma"] ** (step // config["step_size"])


class MultiStepLR(_ScaledSchedule):
    """base * gamma ** (number of milestones <= step)."""

    _FIELDS = (("milestones", _milestones), ("gamma", _rate))

    def __init__(self, optimizer: Optimizer, milestones, gamma: float = 0.1, last_step: int = 0):
        if isinstance(milestones, (str, bytes, dict, set, frozenset)):
            raise TypeError("milestones must be an ordered iterable of integers.")
        try:
            milestones = list(milestones)
        except TypeError:
            raise TypeError("milestones must be an ordered iterable of integers.") from None
        super().__init__(optimizer, last_step, milestones=milestones, gamma=gamma)

    def _factor(self, step, config):
        return config["gamma"] ** bisect_right(config["milestones"], step)


class ExponentialLR(_ScaledSchedule):
    """base * gamma ** step."""

    _FIELDS = (("gamma", _rate),)

    def __init__(self, optimizer: Optimizer, gamma: float, last_step: int = 0):
        super().__init__(optimizer, last_step, gamma=gamma)

    def _factor(self, step, config):
        return config["gamma"] ** step


class LinearLR(_ScaledSchedule):
    """base * (start * (1 - p) + end * p), p = min(step, total_iters) / total_iters."""

    _FIELDS = (("start_factor", _rate), ("end_factor", _rate), ("total_iters", _count(1)))

    def __init__(self, optimizer: Optimizer, start_factor: float = 1 / 3, end_factor: float = 1.0,
                 total_iters: int = 5, last_step: int = 0):
        super().__init__(optimizer, last_step, start_factor=start_factor, end_factor=end_factor, total_iters=total_iters)

    def _factor(self, step, config):
        progress = min(step, config["total_iters"]) / config["total_iters"]
        return config["start_factor"] * (1 - progress) + config["end_factor"] * progress


class CosineAnnealingLR(LRScheduler):
    """eta_min + (base - eta_min) * (1 + cos(pi * min(step, T_max) / T_max)) / 2."""

    _FIELDS = (("T_max", _count(1)), ("eta_min", _rate))

    def __init__(self, optimizer: Optimizer, T_max: int, eta_min: float = 0.0, last_step: int = 0):
        super().__init__(optimizer, last_step, T_max=T_max, eta_min=eta_min)

    def _compute_lrs(self, step, base_lrs, config):
        return _toward(base_lrs, config["eta_min"], _half_cosine(min(step, config["T_max"]) / config["T_max"]))


def _warmup_before_total(config: dict) -> None:
    if config["warmup_steps"] >= config["total_steps"]:
        raise ValueError("warmup_steps must be smaller than total_steps.")


class WarmupCosine(LRScheduler):
    """Linear warm-up to the base rate over warmup_steps, then cosine decay
    to min_lr at total_steps (the training runner's schedule)."""

    _FIELDS = (("warmup_steps", _count(0)), ("total_steps", _count(1)), (None, _warmup_before_total),
               ("min_lr", _rate))

    def __init__(self, optimizer: Optimizer, warmup_steps: int, total_steps: int, min_lr: float = 0.0,
                 last_step: int = 0):
        super().__init__(optimizer, last_step, warmup_steps=warmup_steps, total_steps=total_steps, min_lr=min_lr)

    def _compute_lrs(self, step, base_lrs, config):
        floor, warmup, total = config["min_lr"], config["warmup_steps"], config["total_steps"]
        _toward(base_lrs, floor, 1.0)                 # every base at least the floor
        if step < warmup:
            return [base * (step / warmup) for base in base_lrs]
        return _toward(base_lrs, floor, _half_cosine((min(step, total) - warmup) / (total - warmup)))


__all__ = ["LRScheduler", "StepLR", "MultiStepLR", "ExponentialLR", "CosineAnnealingLR", "LinearLR", "WarmupCosine"]
