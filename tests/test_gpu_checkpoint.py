"""Checkpoint resume on the device.

* A checkpoint written by the reference's own save_checkpoint after 3 AMP
  steps (tests/golden/checkpoint_reference.nt) is restored into this
  package's AdamW and GradScaler on the GPU; the next 2 steps must give the
  reference's parameters, moments, step counts and scaler state bit for bit
  (through the reference call sequence and through amp.fused_step).
* Device-resident state written here (fp32 masters, bfloat16 moments, the
  scale held on the device by fused steps) must survive save/load exactly:
  3 steps + checkpoint + 3 steps in fresh objects equals 6 uninterrupted
  steps, bit for bit.
* The training loop's learning-rate schedule, stepped only after updated
  steps, gives the reference's run bit for bit, also when the skip decision
  stays on the device (fused_step with a scheduler).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd import checkpoint as ck

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
GOLDEN = Path(__file__).resolve().parent / "golden"


def _bits(tensor):
    return tensor.bits().tobytes()


def _tiny(device=DEV):
    named = {"weight": nt.Parameter(np.zeros((40, 48), np.float32), device=device),
             "bias": nt.Parameter(np.zeros(40, np.float32), device=device)}
    optimizer = nt.optim.AdamW([{"params": [named["weight"]], "weight_decay": 0.1},
                                {"params": [named["bias"]], "weight_decay": 0.0}],
                               lr=1e-3, betas=(0.9, 0.95), eps=1e-8)
    scaler = nt.GradScaler(init_scale=1024.0, growth_interval=2)
    return named, optimizer, scaler


@pytest.mark.parametrize("mode", ["api", "fused"])
def test_resume_from_reference_checkpoint(mode):
    golden = json.loads((GOLDEN / "golden.json").read_text())["checkpoint"]
    data = np.load(GOLDEN / "checkpoint_resume.npz")
    named, optimizer, scaler = _tiny()
    info = ck.load_checkpoint(GOLDEN / "checkpoint_reference.nt", named, optimizer, scaler=scaler)
    assert info["step"] == golden["saved_at"]
    params = [named["weight"], named["bias"]]
    for k in range(golden["saved_at"], golden["steps"]):
        for i, p in enumerate(params):
            p.grad = nt.Tensor(data[f"grad{i}_{k}"], device=DEV)
        scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
        if mode == "api":
            finite = scaler.unscale_(optimizer)
            if finite:
                nt.optim.clip_grad_norm_(params, 1.0, error_if_nonfinite=True)
            scaler.step(optimizer)
            scaler.update()
        else:
            finite = nt.amp.fused_step(optimizer, scaler, max_norm=1.0).finite
        assert finite == golden["finite"][k], k
    for i, p in enumerate(params):
        state = optimizer.state[id(p)]
        assert p.numpy().tobytes() == data[f"p{i}"].tobytes(), i
        assert state["exp_avg"].numpy().tobytes() == data[f"m{i}"].tobytes(), i
        assert state["exp_avg_sq"].numpy().tobytes() == data[f"v{i}"].tobytes(), i
        assert state["step"] == int(data[f"step{i}"])
    assert scaler.state_dict() == golden["scaler"]


def _master_setup(seed):
    rng = np.random.default_rng(seed)
    shapes = {"embed": (1000, 64), "proj": (64, 64), "norm": (64,), "tail": (4099,)}
    named = {}
    for name, shape in shapes.items():
        host = (rng.standard_normal(shape) * 0.05).astype(np.float32)
        named[name] = nt.Parameter(host, dtype="bfloat16", device=DEV)
    decay = [p for n, p in named.items() if n != "norm"]
    optimizer = nt.optim.AdamW([{"params": decay, "weight_decay": 0.1},
                                {"params": [named["norm"]], "weight_decay": 0.0}],
                               lr=2e-3, master_weights=True, state_dtype="bfloat16")
    scaler = nt.GradScaler(init_scale=2.0 ** 14, growth_interval=2)
    return named, optimizer, scaler


def _grads(named, k, scale):
    rng = np.random.default_rng(1000 + k)
    grads = {}
    for name, p in named.items():
        g = (rng.standard_normal(p.shape) * 1e-3 * scale).astype(np.float32)
        if k == 1 and name == "tail":
            g[17] = np.inf
        grads[name] = g
    return grads


def _run(named, optimizer, scaler, steps):
    for k in steps:
        scale = scaler.get_scale()
        for name, g in _grads(named, k, scale).items():
            named[name].grad = nt.Tensor(g, dtype="bfloat16", device=DEV)
        scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
        nt.amp.fused_step(optimizer, scaler, max_norm=0.05)


def _snapshot(named, optimizer, scaler):
    out = {"scaler": scaler.state_dict()}
    for name, p in named.items():
        state = optimizer.state[id(p)]
        out[name] = (_bits(p), _bits(state["master"]), _bits(state["exp_avg"]), _bits(state["exp_avg_sq"]),
                     state["step"], state["exp_avg"].dtype)
    return out


def test_device_state_roundtrip_is_exact(tmp_path):
    named, optimizer, scaler = _master_setup(5)
    _run(named, optimizer, scaler, range(6))
    uninterrupted = _snapshot(named, optimizer, scaler)

    named, optimizer, scaler = _master_setup(5)
    _run(named, optimizer, scaler, range(3))
    path = tmp_path / "resume.nt"
    ck.save_checkpoint(path, named, optimizer, scaler=scaler, step=3)
    fresh_named, fresh_optimizer, fresh_scaler = _master_setup(99)      # different weights until loaded
    ck.load_checkpoint(path, fresh_named, fresh_optimizer, scaler=fresh_scaler)
    assert fresh_scaler.state_dict() == scaler.state_dict()
    _run(fresh_named, fresh_optimizer, fresh_scaler, range(3, 6))
    resumed = _snapshot(fresh_named, fresh_optimizer, fresh_scaler)
    assert resumed["scaler"] == uninterrupted["scaler"]
    for name in named:
        assert resumed[name] == uninterrupted[name], name
    assert uninterrupted["tail"][5] is nt.bfloat16


@pytest.mark.parametrize("mode", ["api", "fused", "fused_observed"])
def test_schedule_follows_updates_like_reference(mode):
    """The training loop's WarmupCosine steps only after updated steps
    (runner.py:250-253); with fused_step the skip is known on the device and
    the scheduler advances at reconciliation.  10 steps with non-finite
    gradients at steps 2 and 6 (lr 0 at step 0) must reproduce the
    reference's parameters, moments, scale and schedule bit for bit."""
    golden = json.loads((GOLDEN / "golden.json").read_text())["schedule_runner"]
    data = np.load(GOLDEN / "schedule_runner.npz")
    params = [nt.Parameter(data["p0_0"], device=DEV), nt.Parameter(data["p0_1"], device=DEV)]
    optimizer = nt.optim.AdamW([{"params": [params[0]], "weight_decay": 0.1},
                                {"params": [params[1]], "weight_decay": 0.0}], lr=2e-3, betas=(0.9, 0.95))
    scheduler = nt.optim.WarmupCosine(optimizer, 3, 12, min_lr=1e-4)
    scaler = nt.GradScaler(init_scale=4096.0, growth_interval=3)
    for k in range(golden["steps"]):
        if mode != "fused":
            assert scheduler.get_last_lr() == golden["lr_used"][k], k
        for i, p in enumerate(params):
            p.grad = nt.Tensor(data[f"grad{i}_{k}"], device=DEV)
        scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
        if mode == "api":
            finite = scaler.unscale_(optimizer)
            if finite:
                nt.optim.clip_grad_norm_(params, 1.0, error_if_nonfinite=True)
            updated = scaler.step(optimizer)
            scaler.update()
            if updated:
                scheduler.step()
        else:
            result = nt.amp.fused_step(optimizer, scaler, max_norm=1.0, scheduler=scheduler)
            if mode == "fused_observed":
                assert result.updated == golden["updated"][k], k
                assert scaler.get_scale() == golden["scale"][k], k
    assert scheduler.get_last_lr() == golden["last_lr"]
    assert scheduler.state_dict() == golden["scheduler_state"]
    assert scaler.get_scale() == golden["scale"][-1]
    for i, p in enumerate(params):
        state = optimizer.state[id(p)]
        assert p.numpy().tobytes() == data[f"p{i}"].tobytes(), i
        assert state["exp_avg"].numpy().tobytes() == data[f"m{i}"].tobytes(), i
        assert state["exp_avg_sq"].numpy().tobytes() == data[f"v{i}"].tobytes(), i
        assert state["step"] == int(data[f"step{i}"])


@pytest.mark.parametrize("first_read", ["state", "version"])
def test_reads_right_after_a_skipped_fused_step(first_read):
    """The last step of a fused run is skipped on the device (non-finite
    gradients) and read back at once, with no other synchronizing call:
    ``optimizer.state[...]["step"]`` and the version counters must be those
    of the reference call sequence at the same point, where the skipped step
    never happened (amp.py:211-217)."""
    golden = json.loads((GOLDEN / "golden.json").read_text())["schedule_runner"]
    data = np.load(GOLDEN / "schedule_runner.npz")
    last = golden["updated"].index(False)             # first skipped step of the reference run
    assert last > 0

    def run(mode):
        params = [nt.Parameter(data["p0_0"], device=DEV), nt.Parameter(data["p0_1"], device=DEV)]
        optimizer = nt.optim.AdamW([{"params": [params[0]], "weight_decay": 0.1},
                                    {"params": [params[1]], "weight_decay": 0.0}], lr=2e-3, betas=(0.9, 0.95))
        scaler = nt.GradScaler(init_scale=4096.0, growth_interval=3)
        for k in range(last + 1):
            for i, p in enumerate(params):
                p.grad = nt.Tensor(data[f"grad{i}_{k}"], device=DEV)
            scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
            if mode == "api":
                if scaler.unscale_(optimizer):
                    nt.optim.clip_grad_norm_(params, 1.0)
                scaler.step(optimizer)
                scaler.update()
            else:
                nt.amp.fused_step(optimizer, scaler, max_norm=1.0)
        if first_read == "version":
            versions = [(p._version, optimizer.state[id(p)]["exp_avg"]._version) for p in params]
            steps = [optimizer.state[id(p)]["step"] for p in params]
        else:
            steps = [optimizer.state[id(p)]["step"] for p in params]
            versions = [(p._version, optimizer.state[id(p)]["exp_avg"]._version) for p in params]
        return steps, versions, [p.grad._version for p in params], [p.numpy().tobytes() for p in params]

    api = run("api")
    fused = run("fused")
    assert fused[0] == api[0] == [sum(golden["updated"][:last + 1])] * 2
    assert fused[1] == api[1]
    assert fused[2] == api[2]
    assert fused[3] == api[3]
