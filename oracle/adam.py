"""NumPy restatement of Adam/AdamW (test infrastructure).

Follows the reference's NumPy backend path operation for operation:

* coefficients — ``_scalar`` (optim/_common.py:39-47): each host float is
  rounded once to the parameter dtype with ``dtype.type(value)``; the ten
  values of adam.py:82-86 are ``lr, b1, b2, 1-b1, 1-b2, eps, wd, 1-lr*wd,
  1-b1**step, 1-b2**step`` computed in Python float64;
* gradient — ``_gradient`` (_common.py:57-64): copy, negate when maximizing,
  add ``wd*p`` for (coupled) Adam;
* moments — adam.py:35-36: ``m = b1*m + c1*g``, ``v = b2*v + c2*g*g``,
  stored in the state dtype (``Tensor.copy_``, tensor.py:1269-1287);
* update — adam.py:39-42 + ``_apply_update`` (_common.py:67-73): skipped
  when lr == 0; decoupled decay ``p*(1-lr*wd)`` when wd != 0;
  ``p - lr*((m/bc1)/(sqrt(v/bc2)+eps))``.

Pinned by: golden fixtures written by the reference's own AdamW/Adam
(tests/golden/make_golden.py, float32 and float16, maximize, lr=0, wd=0,
Adam), step-1 closed form (update = lr*g/(|g|+eps) to fp32 accuracy),
the g=0 invariant (update exactly 0, moments decay), and a float64
brute-force bound over 10 steps.

Extensions with no reference counterpart (pinned by composition: the
float32 master update equals the reference float32 update on the widened
gradient, checked against the same golden fixtures with bfloat16-valued
gradients; the copy-out and bfloat16 moments equal RNE of the float32
values, checked against torch's RNE conversion):

* master weights: float32 master ``p``, gradient widened exactly to float32,
  model copy = RNE(p) in the parameter dtype;
* bfloat16 moments: stored moments widened to float32 before the step; the
  update uses the unrounded float32 moments; the stored moments are
  RNE(m), RNE(v).

``reference_step`` is ``adam_step`` with the reference's staging copies and
state check added, for the CPU baseline's timing; it is pinned to
``adam_step`` bit for bit.
"""

from __future__ import annotations

import math

import numpy as np

from . import lowp


def scalar(dtype, value: float):
    """``_scalar`` (optim/_common.py:39-47) without its error checks."""
    with np.errstate(under="ignore"):
        return np.dtype(dtype).type(value)


def coefficients(dtype, lr: float, betas, eps: float, weight_decay: float, step: int):
    """The ten rounded coefficients of adam.py:82-86, in kernel order."""
    beta1, beta2 = betas
    values = (lr, beta1, beta2, 1 - beta1, 1 - beta2, eps, weight_decay, 1 - lr * weight_decay,
              1 - beta1 ** step, 1 - beta2 ** step)
    return tuple(scalar(dtype, value) for value in values)


def adam_step(param, grad, exp_avg, exp_avg_sq, step: int, *, lr, betas, eps, weight_decay,
              maximize=False, decoupled=True) -> None:
    """One in-place update of NumPy arrays; `step` is the new step count.

    Restates ``Adam._update_parameter`` (optim/adam.py:27-42) with
    ``_gradient``/``_apply_update`` (optim/_common.py:57-73).
    """
    dtype = param.dtype
    g = grad.copy()
    if maximize:
        np.negative(g, out=g)
    if weight_decay != 0 and not decoupled:
        g += scalar(dtype, weight_decay) * param
    beta1, beta2 = betas
    with np.errstate(over="ignore", under="ignore", invalid="ignore", divide="ignore"):
        exp_avg[...] = scalar(dtype, beta1) * exp_avg + scalar(dtype, 1 - beta1) * g
        exp_avg_sq[...] = scalar(dtype, beta2) * exp_avg_sq + scalar(dtype, 1 - beta2) * g * g
        first_corrected = exp_avg / scalar(dtype, 1 - beta1 ** step)
        second_corrected = exp_avg_sq / scalar(dtype, 1 - beta2 ** step)
        denominator = np.sqrt(second_corrected) + scalar(dtype, eps)
        update = first_corrected / denominator
        if lr == 0:
            return
        values = param
        if decoupled and weight_decay != 0:
            values = values * scalar(dtype, 1 - lr * weight_decay)
        param[...] = values - scalar(dtype, lr) * update


def _staged_write(target: np.ndarray, values: np.ndarray) -> None:
    """``Tensor.copy_`` of a host array (tensor.py:1269-1287): ``Tensor(value)``
    copies it (``_make_array(copy=True)``), ``__setitem__`` fills a staged
    array from that copy and assigns the staged array to the storage."""
    value = np.array(values, dtype=target.dtype, copy=True)
    staged = np.empty(target.shape, dtype=target.dtype)
    staged[...] = value
    target[...] = staged


def reference_step(param, grad, exp_avg, exp_avg_sq, step: int, *, lr, betas, eps, weight_decay,
                   maximize=False, decoupled=True) -> None:
    """``adam_step`` with the reference's memory traffic around the same
    arithmetic, for timing the reference's CPU path: the per-step check that
    ``exp_avg_sq`` holds no negative value (``_check_state`` with
    ``runtime=True``, optim/_common.py:114 via :157), and every write through
    ``Tensor.copy_``'s staging (``_staged_write``) for the two moments
    (adam.py:35-36) and the parameter (_common.py:73).  Same results as
    ``adam_step``."""
    if np.any(np.less(exp_avg_sq, 0)):
        raise ValueError("exp_avg_sq must be nonnegative.")
    dtype = param.dtype
    g = grad.copy()
    if maximize:
        np.negative(g, out=g)
    if weight_decay != 0 and not decoupled:
        g += scalar(dtype, weight_decay) * param
    beta1, beta2 = betas
    with np.errstate(over="ignore", under="ignore", invalid="ignore", divide="ignore"):
        _staged_write(exp_avg, scalar(dtype, beta1) * exp_avg + scalar(dtype, 1 - beta1) * g)
        _staged_write(exp_avg_sq, scalar(dtype, beta2) * exp_avg_sq + scalar(dtype, 1 - beta2) * g * g)
        first_corrected = exp_avg / scalar(dtype, 1 - beta1 ** step)
        second_corrected = exp_avg_sq / scalar(dtype, 1 - beta2 ** step)
        denominator = np.sqrt(second_corrected) + scalar(dtype, eps)
        update = first_corrected / denominator
        if lr == 0:
            return
        values = param
        if decoupled and weight_decay != 0:
            values = values * scalar(dtype, 1 - lr * weight_decay)
        _staged_write(param, values - scalar(dtype, lr) * update)


def master_step(master, grad32, exp_avg, exp_avg_sq, step: int, *, lr, betas, eps, weight_decay,
                maximize=False, state_bf16=False):
    """float32-master extension; moments as float32 arrays (bf16-valued when
    `state_bf16`).  Returns the unrounded float32 moments used by the update;
    the caller stores RNE(m), RNE(v) for bfloat16 moments."""
    m = exp_avg.astype(np.float32).copy()
    v = exp_avg_sq.astype(np.float32).copy()
    adam_step(master, grad32.astype(np.float32), m, v, step, lr=lr, betas=betas, eps=eps,
              weight_decay=weight_decay, maximize=maximize, decoupled=True)
    if state_bf16:
        exp_avg[...] = lowp.round_bf16(m)
        exp_avg_sq[...] = lowp.round_bf16(v)
    else:
        exp_avg[...] = m
        exp_avg_sq[...] = v
    return m, v


def copy_out(master: np.ndarray, dtype: str) -> np.ndarray:
    """Model copy written from the float32 master: RNE to `dtype`."""
    if dtype == "bfloat16":
        return lowp.round_bf16(master)
    if dtype == "float16":
        return master.astype(np.float16)
    return master.copy()


def adam_f64_reference(param, grads, *, lr, betas, eps, weight_decay, maximize=False, decoupled=True):
    """The same recurrence evaluated in float64 (brute-force bound for pins)."""
    p = param.astype(np.float64).copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    beta1, beta2 = betas
    for step, grad in enumerate(grads, start=1):
        g = grad.astype(np.float64)
        if maximize:
            g = -g
        if weight_decay != 0 and not decoupled:
            g = g + weight_decay * p
        m = beta1 * m + (1 - beta1) * g
        v = beta2 * v + (1 - beta2) * g * g
        if lr == 0:
            continue
        if decoupled and weight_decay != 0:
            p = p * (1 - lr * weight_decay)
        p = p - lr * (m / (1 - beta1 ** step)) / (np.sqrt(v / (1 - beta2 ** step)) + eps)
    return p, m, v


def bias_corrections_positive(dtype, betas, step: int) -> bool:
    beta1, beta2 = betas
    return float(scalar(dtype, 1 - beta1 ** step)) > 0 and float(scalar(dtype, 1 - beta2 ** step)) > 0 and math.isfinite(step)
