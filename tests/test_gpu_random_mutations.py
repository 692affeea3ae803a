"""Seeded random edits between optimizer steps, against the oracle.

The step memo replays a step when nothing it depends on changed; these runs
change things between steps the way training code does and check every step
against the oracle (``adam.adam_step`` / ``adam.master_step`` applied to the
parameters the reference would update, optim/optimizer.py:181-195):

* a gradient set to None, ``requires_grad`` switched off and on again
  (the parameter is skipped, its state and step count unchanged);
* new gradient objects, gradients rewritten in place (``grad[...] = x``),
  ``zero_grad(set_to_none=True)`` followed by new gradients;
* option changes in a group (lr including 0, betas, eps, weight decay,
  maximize, the fused switch);
* a moment buffer rewritten in place by the caller (``exp_avg[...] = x``);
* ``load_state_dict(state_dict())`` and ``add_param_group`` with a new
  parameter in the middle of the run.

Bar: parameters, master weights, moments and step counts bit-exact after
every step.
"""

from __future__ import annotations

import numpy as np
import pytest

import namitorch_amd as nt
from oracle import adam as oadam
from oracle import lowp

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
CASES = 40
STEPS = 6
SIZES = (1, 255, 256, 257, 2047, 2049, 4096, 4097, 12289)


def _grad(rng, shape, dtype):
    values = rng.standard_normal(shape) * 1e-3
    return lowp.round_to("bfloat16", values) if dtype == "bfloat16" else values.astype(np.float32)


class _Reference:
    """Host mirror: values, moments and step counts per parameter, updated
    with the oracle for the parameters that have a gradient and require it."""

    def __init__(self, master: bool):
        self.master = master
        self.values, self.m, self.v, self.steps = {}, {}, {}, {}

    def add(self, key, host):
        self.values[key] = host.astype(np.float32).copy()
        self.steps[key] = 0

    def update(self, key, grad, options):
        if key not in self.m:
            self.m[key] = np.zeros_like(self.values[key])
            self.v[key] = np.zeros_like(self.values[key])
        self.steps[key] += 1
        kw = dict(lr=options["lr"], betas=options["betas"], eps=options["eps"],
                  weight_decay=options["weight_decay"], maximize=options["maximize"])
        if self.master:
            oadam.master_step(self.values[key], grad.astype(np.float32), self.m[key], self.v[key], self.steps[key], **kw)
        else:
            oadam.adam_step(self.values[key], grad, self.m[key], self.v[key], self.steps[key], **kw)


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32 if a.itemsize == 4 else np.uint16)


@pytest.mark.parametrize("seed", range(CASES))
def test_random_edits_between_steps(seed):
    rng = np.random.default_rng(7000 + seed)
    master = bool(rng.random() < 0.35)
    dtype = "bfloat16" if master else "float32"
    count = int(rng.integers(2, 6))
    shapes = [(int(rng.choice(SIZES)),) for _ in range(count + 1)]       # the last one joins later
    hosts = [(rng.standard_normal(s) * 0.02) for s in shapes]
    hosts = [lowp.round_to("bfloat16", h) if master else h.astype(np.float32) for h in hosts]
    params = [nt.Parameter(h, dtype=dtype, device=DEV) for h in hosts]
    ref = _Reference(master)
    for key, h in enumerate(hosts):
        ref.add(key, h)
    cut = int(rng.integers(1, count)) if count > 1 else count
    groups = [dict(params=params[:cut], lr=1e-3, weight_decay=0.1), dict(params=params[cut:count], lr=3e-4, weight_decay=0.0)]
    groups = [g for g in groups if g["params"]]
    optimizer = nt.optim.AdamW(groups, master_weights=master)
    member = {id(p): gi for gi, g in enumerate(optimizer.param_groups) for p in g["params"]}
    active = list(range(count))
    print(f"case {seed}: master={master} shapes={shapes} groups={[len(g['params']) for g in groups]}", flush=True)
    for step in range(STEPS):
        edits = []
        # Gradients: new objects, in place, or zero_grad(set_to_none=True) then new ones.
        mode = str(rng.choice(["new", "inplace", "none_then_new"]))
        grads = {k: _grad(rng, shapes[k], dtype) for k in active}
        if mode == "none_then_new" or step == 0:
            optimizer.zero_grad(set_to_none=True)
        for k in active:
            p = params[k]
            if mode == "inplace" and p.grad is not None:
                p.grad[...] = nt.Tensor(grads[k], dtype=dtype, device=DEV)
            else:
                p.grad = nt.Tensor(grads[k], dtype=dtype, device=DEV)
        skipped = set()
        if rng.random() < 0.3:
            k = int(rng.choice(active))
            params[k].grad = None
            skipped.add(k)
            edits.append(f"grad[{k}]=None")
        if rng.random() < 0.2:
            k = int(rng.choice(active))
            params[k].requires_grad = False
            skipped.add(k)
            edits.append(f"requires_grad[{k}]=False")
        if rng.random() < 0.4:
            g = optimizer.param_groups[int(rng.integers(len(optimizer.param_groups)))]
            name = str(rng.choice(["lr", "betas", "eps", "weight_decay", "maximize", "fused"]))
            value = {"lr": float(rng.choice([0.0, 1e-3, 2e-4])), "betas": (float(rng.choice([0.9, 0.0])), 0.99),
                     "eps": float(rng.choice([1e-8, 1e-6])), "weight_decay": float(rng.choice([0.0, 0.05])),
                     "maximize": bool(rng.random() < 0.5), "fused": [None, False][int(rng.integers(2))]}[name]
            g[name] = value
            edits.append(f"group.{name}={value}")
        if not master and rng.random() < 0.2:
            candidates = [k for k in active if k in ref.m and id(params[k]) in optimizer.state]
            if candidates:
                k = int(rng.choice(candidates))
                halved = (ref.m[k] * np.float32(0.5)).astype(np.float32)
                optimizer.state[id(params[k])]["exp_avg"][...] = nt.Tensor(halved, device=DEV)
                ref.m[k] = halved
                edits.append(f"exp_avg[{k}]*=0.5")
        if rng.random() < 0.15:
            optimizer.load_state_dict(optimizer.state_dict())
            edits.append("load_state_dict")
        if step == STEPS // 2 and count not in active:
            new = params[count]
            new.grad = nt.Tensor(_grad(rng, shapes[count], dtype), dtype=dtype, device=DEV)
            grads[count] = new.grad.numpy() if not master else lowp.round_to("bfloat16", new.grad.numpy())
            optimizer.add_param_group(dict(params=[new], lr=5e-4, weight_decay=0.01))
            member[id(new)] = len(optimizer.param_groups) - 1
            active.append(count)
            edits.append("add_param_group")
        optimizer.step()
        for k in active:
            if k in skipped:
                continue
            options = optimizer.param_groups[member[id(params[k])]]
            ref.update(k, grads[k], options)
        print(f"  step {step}: {mode} {edits}", flush=True)
        for k in active:
            if k in skipped and params[k].requires_grad is False:
                params[k].requires_grad = True
            state = optimizer.state.get(id(params[k]), {})
            assert state.get("step", 0) == ref.steps[k], (step, k)
            if master:
                if ref.steps[k]:
                    assert np.array_equal(_bits(state["master"].numpy()), _bits(ref.values[k])), (step, k)
                want = lowp.round_to("bfloat16", ref.values[k].astype(np.float64))
            else:
                want = ref.values[k]
            assert np.array_equal(_bits(params[k].numpy()), _bits(want)), (step, k, edits)
            if ref.steps[k]:
                assert np.array_equal(_bits(state["exp_avg"].numpy()), _bits(ref.m[k])), (step, k)
                assert np.array_equal(_bits(state["exp_avg_sq"].numpy()), _bits(ref.v[k])), (step, k)
