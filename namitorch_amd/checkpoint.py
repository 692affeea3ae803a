"""Optimizer and GradScaler state in NamiTorch training checkpoints.

A training checkpoint (``namitorch/training/checkpoint.py:12-174``) is an
archive (``serialization``) holding one dictionary with the keys
``checkpoint_version`` (1), ``model``, ``optimizer``, ``optimizer_type``,
``optimizer_parameter_names``, ``scheduler``, ``rng``, ``step``, ``epoch``,
``config``, ``cumulative_tokens`` and, when AMP is on, ``scaler``.  The
optimizer entry is ``Optimizer.state_dict()`` with its per-parameter state
keyed by decimal strings (the archive's dictionaries take string keys only).

This module covers the optimizer-step side of that file:

* `pack_optimizer` / `unpack_optimizer` convert between ``state_dict()`` and
  the archived form (checkpoint.py:59-77);
* `optimizer_type` names the optimizer class as the reference does, so an
  AdamW of this package and the reference's AdamW read each other's
  checkpoints;
* `save_checkpoint` writes a complete checkpoint from named parameters, an
  optimizer, a learning-rate scheduler and a scaler (model entries are the
  named parameters);
* `load_checkpoint` reads one, checks it like checkpoint.py:113-174 does for
  the parts it restores, and restores parameters, optimizer and scaler state
  with nothing changed unless every check passes.

Everything device-resident round-trips exactly: fp32 masters and moments,
bfloat16 moments (stored as their exact float32 widening), integer step
counts and the scaler's scale (a Python float, stored as a hexadecimal
string) and growth tracker.  ``state_dict()`` first folds in the outcome of
any ``amp.fused_step`` still in flight.
"""

from __future__ import annotations

from numbers import Integral

import numpy as np

from .amp import GradScaler
from .optim.lr_scheduler import LRScheduler
from .optim.optimizer import Optimizer
from .serialization import SerializationError, load, save
from .tensor import Tensor, no_grad

CHECKPOINT_VERSION = 1
_KEYS = frozenset({"checkpoint_version", "model", "optimizer", "optimizer_type", "optimizer_parameter_names",
                   "scheduler", "rng", "step", "epoch", "config", "cumulative_tokens"})
# Classes of this package stand in for the reference classes of the same name.
_REFERENCE_TYPES = {"Adam": "namitorch.optim.adam.Adam", "AdamW": "namitorch.optim.adam.AdamW"}


def _counter(value, name: str) -> int:
    if isinstance(value, bool) or not isinstance(value, Integral) or value < 0:
        raise ValueError(f"{name} must be a nonnegative integer.")
    return int(value)


def optimizer_type(optimizer: Optimizer | None) -> str | None:
    """Qualified class name recorded in a checkpoint; this package's Adam and
    AdamW record the reference's names."""
    if optimizer is None:
        return None
    cls = type(optimizer)
    if cls.__module__.startswith("namitorch_amd.") and cls.__qualname__ in _REFERENCE_TYPES:
        return _REFERENCE_TYPES[cls.__qualname__]
    return f"{cls.__module__}.{cls.__qualname__}"


def pack_optimizer(optimizer: Optimizer | None) -> dict | None:
    """``optimizer.state_dict()`` with string state keys, as archived."""
    if optimizer is None:
        return None
    state = optimizer.state_dict()
    state["state"] = {str(index): values for index, values in state["state"].items()}
    return state


def unpack_optimizer(state) -> dict:
    """The archived optimizer entry back in ``load_state_dict`` form."""
    if not isinstance(state, dict) or not isinstance(state.get("state"), dict):
        raise SerializationError("Invalid checkpoint optimizer state.")
    restored = dict(state)
    values = {}
    for key, value in state["state"].items():
        if type(key) is not str or not key.isascii() or not key.isdecimal() or str(int(key)) != key:
            raise SerializationError("Optimizer state indices must be canonical nonnegative integer strings.")
        values[int(key)] = value
    restored["state"] = values
    return restored


def _named(named_parameters) -> dict:
    items = list(named_parameters.items() if isinstance(named_parameters, dict) else named_parameters)
    result = {}
    for name, parameter in items:
        if type(name) is not str or not name:
            raise TypeError("Parameter names must be nonempty strings.")
        if not isinstance(parameter, Tensor):
            raise TypeError(f"Parameter {name!r} must be a NamiTorch Tensor.")
        if name in result:
            raise ValueError(f"Duplicate parameter name {name!r}.")
        result[name] = parameter
    return result


def parameter_names(named: dict, optimizer: Optimizer | None):
    """Per group, the names of the optimizer's parameters (checkpoint.py:43-53)."""
    if optimizer is None:
        return None
    names = {id(parameter): name for name, parameter in named.items()}
    optimizer._registered_parameters()
    result = []
    for group in optimizer.param_groups:
        if any(id(parameter) not in names for parameter in group["params"]):
            raise ValueError("Checkpoint optimizer parameters must belong to the saved model.")
        result.append([names[id(parameter)] for parameter in group["params"]])
    return result


def _check_components(optimizer, scheduler, scaler) -> None:
    if scaler is not None and not isinstance(scaler, GradScaler):
        raise TypeError("scaler must be a NamiTorch GradScaler or None.")
    if optimizer is not None and not isinstance(optimizer, Optimizer):
        raise TypeError("optimizer must be a NamiTorch Optimizer or None.")
    if scheduler is not None:
        if not isinstance(scheduler, LRScheduler):
            raise TypeError("scheduler must be a NamiTorch LRScheduler or None.")
        if optimizer is None or scheduler.optimizer is not optimizer:
            raise ValueError("scheduler must belong to the supplied optimizer.")


def _fresh_rng_state(seed: int = 0) -> dict:
    """A PCG64 generator state in the reference's layout (the bit generator's
    state dictionary plus a version); RNG streams are not part of this path."""
    state = dict(np.random.PCG64(seed).state)
    state["version"] = 1
    return state


def save_checkpoint(path, named_parameters, optimizer: Optimizer | None = None, scheduler: LRScheduler | None = None,
                    *, scaler: GradScaler | None = None, step: int = 0, epoch: int = 0, config=None,
                    cumulative_tokens: int = 0) -> None:
    """Write a training checkpoint in the reference layout; ``model`` holds
    the named parameters (detached)."""
    _check_components(optimizer, scheduler, scaler)
    named = _named(named_parameters)
    if scheduler is not None and scheduler.get_lr() != [group["lr"] for group in optimizer.param_groups]:
        raise ValueError("Optimizer learning rates disagree with the scheduler state.")
    checkpoint = {
        "checkpoint_version": CHECKPOINT_VERSION,
        "model": {name: parameter.detach() for name, parameter in named.items()},
        "optimizer": pack_optimizer(optimizer),
        "optimizer_type": optimizer_type(optimizer),
        "optimizer_parameter_names": parameter_names(named, optimizer),
        "scheduler": None if scheduler is None else scheduler.state_dict(),
        "rng": {"default": _fresh_rng_state(), "generators": {}},
        "step": _counter(step, "step"),
        "epoch": _counter(epoch, "epoch"),
        "config": config,
        "cumulative_tokens": _counter(cumulative_tokens, "cumulative_tokens"),
    }
    if scaler is not None:
        checkpoint["scaler"] = scaler.state_dict()
    save(checkpoint, path)


def load_checkpoint(path, named_parameters, optimizer: Optimizer | None = None, scheduler: LRScheduler | None = None,
                    *, scaler: GradScaler | None = None, strict: bool = True, max_array_bytes=None) -> dict:
    """Restore parameters (copied in place, so optimizers keep their
    references), optimizer and scaler state from a checkpoint written here or
    by the reference.  Every check runs before anything is modified.  Returns
    ``{"step", "epoch", "cumulative_tokens", "config", "missing",
    "unexpected"}``."""
    _check_components(optimizer, scheduler, scaler)
    if type(strict) is not bool:
        raise TypeError("strict must be a Python bool.")
    named = _named(named_parameters)
    checkpoint = load(path, max_array_bytes=max_array_bytes)
    if type(checkpoint) is not dict or set(checkpoint) not in (_KEYS, _KEYS | {"scaler"}):
        raise SerializationError("Invalid checkpoint fields.")
    if type(checkpoint["checkpoint_version"]) is not int or checkpoint["checkpoint_version"] != CHECKPOINT_VERSION:
        raise SerializationError("Unsupported checkpoint_version.")
    info = {name: _counter(checkpoint[name], name) for name in ("step", "epoch", "cumulative_tokens")}
    info["config"] = checkpoint["config"]

    prepared_scaler = scaler._prepare_load_state_dict(checkpoint.get("scaler")) if scaler is not None else None
    saved = checkpoint["model"]
    if type(saved) is not dict:
        raise SerializationError("Invalid checkpoint model state.")
    missing = [name for name in named if name not in saved]
    unexpected = [name for name in saved if name not in named]
    if strict and (missing or unexpected):
        raise RuntimeError(f"Checkpoint parameters do not match: missing {missing}, unexpected {unexpected}.")
    copies = []
    for name, parameter in named.items():
        if name not in saved:
            continue
        value = saved[name]
        if not isinstance(value, Tensor) or value.shape != parameter.shape:
            raise ValueError(f"Checkpoint parameter {name!r} must be a Tensor of shape {parameter.shape}.")
        copies.append((parameter, value))
    optimizer_update = None
    if optimizer is not None:
        if checkpoint["optimizer_type"] != optimizer_type(optimizer):
            raise ValueError("Checkpoint optimizer type does not match the supplied optimizer.")
        if checkpoint["optimizer_parameter_names"] != parameter_names(named, optimizer):
            raise ValueError("Checkpoint optimizer parameter names or group order do not match the model.")
        optimizer_update = optimizer._prepare_load_state_dict(unpack_optimizer(checkpoint["optimizer"]))
    scheduler_update = None
    if scheduler is not None:
        scheduler_update = scheduler._prepare_load_state_dict(checkpoint["scheduler"])
        if [group["lr"] for group in optimizer_update[1]] != scheduler_update[3]:
            raise ValueError("Checkpoint optimizer learning rates disagree with the scheduler state.")

    with no_grad():
        for parameter, value in copies:
            parameter.copy_(value.to(parameter.device))
    if optimizer_update is not None:
        optimizer._install_loaded_state(*optimizer_update)
    if scheduler_update is not None:
        scheduler._apply_loaded_state(scheduler_update)
    if prepared_scaler is not None:
        scaler.load_state_dict(checkpoint["scaler"])
    info["missing"] = missing
    info["unexpected"] = unexpected
    return info


__all__ = ["CHECKPOINT_VERSION", "optimizer_type", "pack_optimizer", "unpack_optimizer", "parameter_names",
           "save_checkpoint", "load_checkpoint"]
