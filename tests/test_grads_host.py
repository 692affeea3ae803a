"""Gradient accumulation validation on the host (no device compute): the
checks and messages of autograd.validate_gradient/validate_accumulation
(autograd.py:176-195) run before anything is written."""

from __future__ import annotations

import numpy as np
import pytest

import namitorch_amd as nt


def test_accumulate_validation_messages():
    p = nt.Parameter(np.zeros(3, np.float32))
    with pytest.raises(RuntimeError, match="Gradient accumulation must be a registered backend gradient array."):
        nt.accumulate_grads([p], [np.zeros(3, np.float32)])
    with pytest.raises(RuntimeError, match=r"Gradient accumulation has invalid gradient shape \(4,\); expected \(3,\)."):
        nt.accumulate_grads([p], [nt.tensor(np.zeros(4, np.float32))])
    with pytest.raises(RuntimeError, match="requires supported floating gradients and a floating parent, got int32"):
        nt.accumulate_grads([p], [nt.tensor(np.zeros(3, np.int32))])
    p.grad = nt.tensor(np.zeros(3, np.float64))
    with pytest.raises(RuntimeError, match="Stored gradient has gradient dtype float64; expected namitorch.float32."):
        nt.accumulate_grads([p], [nt.tensor(np.zeros(3, np.float32))])
    with pytest.raises(ValueError, match="one gradient per parameter"):
        nt.accumulate_grads([p], [])


def test_accumulate_on_host_tensors_is_not_computed():
    p = nt.Parameter(np.zeros(3, np.float32))
    with pytest.raises(RuntimeError):
        nt.accumulate_grads([p], [nt.tensor(np.ones(3, np.float32))])
    assert p.grad is None


def test_zero_grad_on_host():
    p = nt.Parameter(np.zeros(3, np.float32))
    p.grad = nt.tensor(np.ones(3, np.float32))
    grad = p.grad
    optimizer = nt.optim.AdamW([p])
    optimizer.zero_grad(set_to_none=False)
    assert p.grad is grad and not grad.numpy().any()
    optimizer.zero_grad()
    assert p.grad is None
