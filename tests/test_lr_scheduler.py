"""Learning-rate schedules, host side: every scheduler's rates, state and
errors against the reference's own values (tests/golden/golden.json), and
schedule state in checkpoints."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd import checkpoint as ck
from namitorch_amd.optim import lr_scheduler as sched

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "golden.json").read_text())
NAMES = ["StepLR", "MultiStepLR", "ExponentialLR", "CosineAnnealingLR", "LinearLR", "WarmupCosine"]


def _two_groups():
    a = nt.Parameter(np.zeros(3, np.float32))
    b = nt.Parameter(np.zeros(2, np.float32))
    return nt.optim.AdamW([{"params": [a]}, {"params": [b], "lr": 3e-4}], lr=1e-3)


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("last_step", [0, 4])
def test_rates_and_state_match_reference(name, last_step):
    case = GOLDEN["schedulers"][name]
    want = case[f"last_step_{last_step}"]
    optimizer = _two_groups()
    scheduler = getattr(sched, name)(optimizer, last_step=last_step, **case["config"])
    rates = [[group["lr"] for group in optimizer.param_groups]]
    for _ in range(14):
        scheduler.step()
        rates.append([group["lr"] for group in optimizer.param_groups])
    assert rates == want["lrs"]                      # exact float equality
    assert scheduler.get_last_lr() == want["last_lr"]
    state = scheduler.state_dict()
    assert json.loads(json.dumps(state)) == want["state"]
    # A fresh scheduler continues identically from the saved state.
    other = getattr(sched, name)(_two_groups(), **case["config"])
    other.load_state_dict(state)
    scheduler.step()
    other.step()
    assert other.get_last_lr() == scheduler.get_last_lr()


def test_error_texts_match_reference():
    expected = GOLDEN["schedulers"]["errors"]
    a = nt.Parameter(np.zeros(3, np.float32))
    optimizer = nt.optim.AdamW([a], lr=1e-3)
    cases = {
        "warmup_ge_total": lambda: sched.WarmupCosine(optimizer, 5, 5),
        "min_lr_above_base": lambda: sched.WarmupCosine(optimizer, 1, 5, min_lr=1.0),
        "step_size_zero": lambda: sched.StepLR(optimizer, 0),
        "gamma_negative": lambda: sched.ExponentialLR(optimizer, -0.5),
        "milestones_set": lambda: sched.MultiStepLR(optimizer, {1, 2}),
        "last_step_bool": lambda: sched.StepLR(optimizer, 2, last_step=True),
        "load_wrong_type": lambda: sched.ExponentialLR(nt.optim.AdamW([a]), 0.5).load_state_dict(
            sched.StepLR(nt.optim.AdamW([a]), 2).state_dict()),
    }
    scheduler = sched.StepLR(optimizer, 2)
    optimizer.add_param_group({"params": [nt.Parameter(np.zeros(2, np.float32))]})
    cases["groups_changed"] = scheduler.step
    assert set(cases) == set(expected)
    for name, action in cases.items():
        with pytest.raises(Exception) as caught:
            action()
        assert [type(caught.value).__name__, str(caught.value)] == expected[name], name


def test_scheduler_must_belong_to_optimizer():
    optimizer = _two_groups()
    scheduler = sched.StepLR(_two_groups(), 2)
    with pytest.raises(ValueError, match="belong to the supplied optimizer"):
        nt.amp.fused_step(optimizer, None, scheduler=scheduler)
    with pytest.raises(TypeError, match="LRScheduler"):
        nt.amp.fused_step(optimizer, None, scheduler=object())


def test_checkpoint_carries_the_schedule(tmp_path):
    named = {"a": nt.Parameter(np.zeros(3, np.float32)), "b": nt.Parameter(np.ones(2, np.float32))}
    optimizer = nt.optim.AdamW([{"params": [named["a"]]}, {"params": [named["b"]], "lr": 3e-4}], lr=1e-3)
    scheduler = sched.WarmupCosine(optimizer, 3, 12, min_lr=2e-5)
    for _ in range(5):
        scheduler.step()
    path = tmp_path / "sched.nt"
    ck.save_checkpoint(path, named, optimizer, scheduler, step=5)
    assert nt.load(path)["scheduler"] == scheduler.state_dict()

    fresh = {"a": nt.Parameter(np.zeros(3, np.float32)), "b": nt.Parameter(np.zeros(2, np.float32))}
    fresh_optimizer = nt.optim.AdamW([{"params": [fresh["a"]]}, {"params": [fresh["b"]], "lr": 3e-4}], lr=1e-3)
    fresh_scheduler = sched.WarmupCosine(fresh_optimizer, 3, 12, min_lr=2e-5)
    ck.load_checkpoint(path, fresh, fresh_optimizer, fresh_scheduler)
    assert fresh_scheduler.state_dict() == scheduler.state_dict()
    assert [g["lr"] for g in fresh_optimizer.param_groups] == [g["lr"] for g in optimizer.param_groups]
    scheduler.step()
    fresh_scheduler.step()
    assert fresh_scheduler.get_last_lr() == scheduler.get_last_lr()

    optimizer.param_groups[0]["lr"] = 0.5                 # out of step with the schedule
    with pytest.raises(ValueError, match="disagree with the scheduler state"):
        ck.save_checkpoint(tmp_path / "bad.nt", named, optimizer, scheduler)
    with pytest.raises(ValueError, match="belong to the supplied optimizer"):
        ck.save_checkpoint(tmp_path / "bad.nt", named, optimizer, fresh_scheduler)
