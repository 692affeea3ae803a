"""Graph-capture guards (namitorch/backends/_graph_capture.py:12-14 and its
call sites: optim/_common.py:134, optim/optimizer.py:289, amp.py:128,170,
197,220, tensor.py:471-481,1253), on the host: with capture reported as
active, every guarded operation raises the reference's RuntimeError text
and changes nothing; with it inactive the same calls work."""

from __future__ import annotations

import re

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd.backends import _graph_capture

SUFFIX = " is not supported in CUDA graph preparation or capture; only deterministic FP32 inference is supported."


def _message(operation):
    return "^" + re.escape(operation + SUFFIX) + "$"


@pytest.fixture
def capture(monkeypatch):
    monkeypatch.setattr(_graph_capture, "capturing", lambda: True)


def _setup():
    p = nt.Parameter(np.ones(4, np.float32))
    p.grad = nt.Tensor(np.full(4, 0.5, np.float32))
    optimizer = nt.optim.AdamW([p])
    scaler = nt.GradScaler()
    return p, optimizer, scaler


def test_reference_message_text():
    with pytest.MonkeyPatch.context() as patch:
        patch.setattr(_graph_capture, "capturing", lambda: True)
        with pytest.raises(RuntimeError) as error:
            _graph_capture.reject_during_capture("Optimizer steps")
    assert str(error.value) == "Optimizer steps" + SUFFIX
    _graph_capture.reject_during_capture("Optimizer steps")          # no capture: no error


def test_optimizer_and_scaler_calls_are_rejected(capture):
    p, optimizer, scaler = _setup()
    loss = nt.Tensor(np.float32(1.0))
    with pytest.raises(RuntimeError, match=_message("Optimizer steps")):
        optimizer.step()
    with pytest.raises(RuntimeError, match=_message("Optimizer steps")):
        nt.amp.fused_step(optimizer, scaler)
    for call in (lambda: scaler.scale(loss), lambda: scaler.unscale_(optimizer), lambda: scaler.step(optimizer),
                 scaler.update):
        with pytest.raises(RuntimeError, match=_message("GradScaler")):
            call()
    with pytest.raises(RuntimeError, match=_message("Moving optimizer state")):
        optimizer.to("cpu")
    assert optimizer.state == {} or all(not state for state in optimizer.state.values())
    assert not scaler._scale_used and not scaler._optimizer_states
    assert p._version == 0 and p.grad._version == 0


def test_inplace_updates_and_host_reads_are_rejected(capture):
    p, optimizer, _ = _setup()
    t = nt.Tensor(np.zeros(3, np.float32))
    for call in (lambda: t.copy_(np.ones(3, np.float32)), lambda: t.fill_(2.0), t.zero_,
                 lambda: t.__setitem__(Ellipsis, 1.0), lambda: optimizer.zero_grad(set_to_none=False),
                 lambda: nt.accumulate_grads([p], [nt.Tensor(np.ones(4, np.float32))])):
        with pytest.raises(RuntimeError, match=_message("In-place Tensor updates")):
            call()
    for call in (t.numpy, t.bits, lambda: nt.Tensor(np.float32(1.0)).item(),
                 lambda: nt.optim.clip_grad_norm_([p], 1.0), lambda: nt.optim.get_grad_norm([p])):
        with pytest.raises(RuntimeError, match=_message("Host Tensor reads")):
            call()
    assert t._version == 0 and p.grad._version == 0
    optimizer.zero_grad(set_to_none=True)                      # not guarded in the reference either
    assert p.grad is None


def test_argument_errors_still_come_first(capture):
    """The guards sit where the reference's do: after argument checks in
    clip_grad_norm_ (which reaches the device only in _total_norm)."""
    p, _, _ = _setup()
    with pytest.raises(ValueError):
        nt.optim.clip_grad_norm_([p], -1.0)
    with pytest.raises(TypeError):
        nt.optim.clip_grad_norm_([p], 1.0, error_if_nonfinite=1)


def test_without_capture_everything_works():
    p, optimizer, _ = _setup()
    t = nt.Tensor(np.zeros(3, np.float32))
    t.fill_(2.0)
    assert t.numpy().tolist() == [2.0, 2.0, 2.0]
    assert nt.Tensor(np.float32(3.0)).item() == 3.0
    with pytest.raises(ValueError, match=r"item\(\) requires exactly one element, got 3\."):
        t.item()
    optimizer.zero_grad(set_to_none=False)
