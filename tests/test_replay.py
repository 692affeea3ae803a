"""The step memo (adam._Replay) against the full step, on the host.

A recording backend stands in for the device: it keeps every launch's
rows, coefficient records and grad transform.  The same sequence of steps
and mutations (lr changes, new or missing gradients, requires_grad flips,
replaced or rewritten state buffers, edited step counts, pending grad
transforms, fused-flag changes, invalid state) runs once with the memo and
once with it disabled; launches, errors and every version counter and step
count must agree, and the memo must actually replay the unchanged steps.
Option changes (learning rates, betas, eps, a NaN learning rate) must reach
the coefficients or raise exactly as the full step does.
"""

from __future__ import annotations

from contextlib import nullcontext

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd.optim import adam as adam_mod
from namitorch_amd.tensor import GradTransform


class _Kernel:
    def supports(self, *arrays):
        return True


class _RecordingBackend:
    def __init__(self):
        self.device = nt.Device("cpu")
        self.adamw = _Kernel()
        self.launches = []
        self._plans = {}

    def context(self, *operands):
        return nullcontext()

    def stream(self):
        return 0

    def _refresh(self, plan, pointers, stream):
        # Re-point the volatile columns, as nt_plan_set_pointers does; the
        # launch records what the plan holds at launch time.
        layout, chunk, rows, _ = plan[1]
        plan[1] = (layout, chunk, rows, tuple((c, tuple(v)) for c, v in sorted(pointers.items())))
        return True

    def plan(self, rows, layout, chunk=0, pointers=None):
        volatile = tuple(sorted((pointers or {}).items()))
        key = (layout, chunk, tuple(rows), tuple((c, tuple(v)) for c, v in volatile))
        stable = (layout, chunk, tuple(rows), tuple(c for c, _ in volatile))
        plan = self._plans.setdefault(stable, ["plan", key])
        if plan[1] != key:
            self._refresh(plan, dict(pointers or {}), 0)
        return plan

    def adamw_multi(self, plan, slots, xform):
        records = [tuple(getattr(record, name) for name, _ in record._fields_) for record in slots]
        transform = None if xform is None else (xform.scale, xform.unscale, xform.clip, xform.clip_coef)
        self.launches.append((plan[1], records, transform))


def _run(monkeypatch, memo: bool, master: bool = False):
    backend = _RecordingBackend()
    monkeypatch.setattr(adam_mod, "get_backend", lambda value=None: backend)
    # Host tensors get addresses as device tensors have them, so the memo's
    # overlap test for adopted gradients runs: one synthetic address per
    # storage (aliases of a storage share it), numbered in creation order and
    # never reused, 2**32 bytes apart, so both runs see the same addresses.
    initialize = nt.Tensor._initialize
    addresses: dict = {}
    storages: list = []                                   # kept alive, so ids are not reused

    def with_pointer(self, storage, *args, **kwargs):
        initialize(self, storage, *args, **kwargs)
        if id(storage) not in addresses:
            storages.append(storage)
            addresses[id(storage)] = len(storages) << 32
        self._ptr = addresses[id(storage)]

    monkeypatch.setattr(nt.Tensor, "_initialize", with_pointer)
    replays = []
    original_run = adam_mod._Replay.run

    def counting_run(self, optimizer):
        done = original_run(self, optimizer)
        replays.append(done)
        return done

    monkeypatch.setattr(adam_mod._Replay, "run", counting_run)
    if not memo:
        monkeypatch.setattr(adam_mod.Adam, "_memoize_step", lambda self, options: setattr(self, "_replay", None))
    rng = np.random.default_rng(3)
    shapes = [(8, 4), (5,), (3, 3), (7,), (2, 6), (4,)]
    dtype = "bfloat16" if master else "float32"
    params = [nt.Parameter(rng.standard_normal(s).astype(np.float32), dtype=dtype) for s in shapes]
    for p in params:
        p.grad = nt.Tensor(rng.standard_normal(p.shape).astype(np.float32), dtype=dtype)
    optimizer = nt.optim.AdamW([{"params": params[:3], "weight_decay": 0.1},
                                {"params": params[3:], "weight_decay": 0.0}], lr=1e-3, master_weights=master)
    errors = []
    for k in range(26):
        if k == 3:
            optimizer.param_groups[0]["lr"] = 5e-4
        elif k == 4:
            params[2].grad = nt.Tensor(rng.standard_normal(params[2].shape).astype(np.float32), dtype=dtype)
        elif k == 12:
            for p in params:                                  # every gradient reallocated
                p.grad = nt.Tensor(rng.standard_normal(p.shape).astype(np.float32), dtype=dtype)
        elif k == 5:
            params[3].grad = None
        elif k == 6:
            params[3].grad = nt.Tensor(np.ones(params[3].shape, np.float32), dtype=dtype)
            params[1].requires_grad = False
        elif k == 7:
            params[1].requires_grad = True
            state = optimizer.state[id(params[0])]
            state["exp_avg"] = state["exp_avg"].clone()
        elif k == 8:
            optimizer.param_groups[1]["lr"] = 0.0
        elif k == 9:
            buffer = optimizer.state[id(params[4])]["exp_avg_sq"]
            buffer.copy_(nt.Tensor(np.full(buffer.shape, 0.25, np.float32), dtype=buffer.dtype))
        elif k == 10:
            optimizer.param_groups[1]["lr"] = 2e-3
            transform = GradTransform(scale=4.0)
            for p in params:
                p.grad._pending = transform
        elif k == 11:
            for p in params:
                p.grad._pending = None
            optimizer.state[id(params[5])]["step"] += 2
        elif k == 13:
            optimizer.param_groups[0]["fused"] = False
        elif k == 14:
            optimizer.state[id(params[1])]["step"] = 7.0
        elif k == 15:
            optimizer.state[id(params[1])]["step"] = 7
            buffer = optimizer.state[id(params[4])]["exp_avg_sq"]
            buffer.copy_(nt.Tensor(np.full(buffer.shape, -1.0, np.float32), dtype=buffer.dtype))
        elif k == 16:
            buffer = optimizer.state[id(params[4])]["exp_avg_sq"]
            buffer.copy_(nt.Tensor(np.full(buffer.shape, 1.0, np.float32), dtype=buffer.dtype))
        elif k == 18:
            optimizer.param_groups[0]["betas"] = (0.8, 0.99)
        elif k == 19:
            optimizer.param_groups[1]["eps"] = 1e-6
        elif k == 20:
            optimizer.param_groups[1]["lr"] = float("nan")
        elif k == 21:
            optimizer.param_groups[1]["lr"] = 2e-3
        elif k == 22:                                         # every gradient reallocated again
            for p in params:
                p.grad = nt.Tensor(rng.standard_normal(p.shape).astype(np.float32), dtype=dtype)
        elif k == 23:                                         # a gradient aliasing its parameter's storage
            params[2].grad = nt.Tensor._from_storage(params[2]._storage, dtype=params[2].dtype)
        elif k == 24:
            params[2].grad = nt.Tensor(rng.standard_normal(params[2].shape).astype(np.float32), dtype=dtype)
        try:
            optimizer.step()
        except (TypeError, ValueError) as error:
            errors.append((k, type(error).__name__, str(error)))
    versions = []
    for p in params:
        state = optimizer.state[id(p)]
        versions.append((p._version, state["step"], state["exp_avg"]._version, state["exp_avg_sq"]._version,
                         state["exp_avg_sq"]._clean_version, state["master"]._version if master else None))
    return backend.launches, errors, versions, replays


@pytest.mark.parametrize("master", [False, True])
def test_memo_replays_exactly_what_the_full_step_launches(monkeypatch, master):
    with monkeypatch.context() as patch:
        full = _run(patch, memo=False, master=master)
    with monkeypatch.context() as patch:
        memo = _run(patch, memo=True, master=master)
    assert memo[0] == full[0]                 # every launch: rows, coefficients, transform
    assert memo[1] == full[1] and len(full[1]) == 3   # invalid step counts, negative state, NaN lr
    assert memo[2] == full[2]
    assert full[3] == []
    replayed = sum(memo[3])
    # Unchanged steps replay, and so do steps whose gradients were
    # reallocated (k = 4, 12, 22, 24).  Other mutations fall back, the
    # aliasing gradient (k = 23) included.
    assert replayed >= 10, memo[3]
    assert len(memo[3]) - replayed >= 6, memo[3]


def test_memo_is_dropped_by_load_state_dict(monkeypatch):
    backend = _RecordingBackend()
    monkeypatch.setattr(adam_mod, "get_backend", lambda value=None: backend)
    p = nt.Parameter(np.ones(4, np.float32))
    p.grad = nt.Tensor(np.ones(4, np.float32))
    optimizer = nt.optim.AdamW([p])
    optimizer.step()
    optimizer.step()
    saved = optimizer.state_dict()
    optimizer.step()
    assert optimizer._replay is not None
    optimizer.load_state_dict(saved)
    optimizer.step()
    assert optimizer.state[id(p)]["step"] == 3
    assert backend.launches[-1][1] == backend.launches[-2][1]      # same coefficients as the third step


def test_comparison_detects_a_memo_that_ignores_option_changes(monkeypatch):
    """The comparison above is sensitive to the options key: with a key that
    never changes, the memo replays stale coefficients after the lr, betas
    and eps changes, and the launches no longer match the full step's."""
    with monkeypatch.context() as patch:
        full = _run(patch, memo=False)
    with monkeypatch.context() as patch:
        patch.setattr(adam_mod, "_options_key", lambda groups: ("unchanging",))
        stale = _run(patch, memo=True)
    assert stale[0] != full[0]


def test_next_coefficients_equal_a_full_computation():
    """The replay rebuilds each coefficient record from the previous step's by
    recomputing the two bias corrections; every field must equal what
    ``_coefficients`` computes from scratch, and the same errors must rise."""
    import ctypes
    import random

    from namitorch_amd import dtype as dtypes
    from namitorch_amd.optim.adam import AdamW

    optimizer = AdamW([nt.Parameter(np.zeros(4, np.float32))], lr=1e-3)
    rng = random.Random(5)
    for trial in range(300):
        dtype = rng.choice([dtypes.float32, dtypes.float16, dtypes.float64])
        options = {"lr": rng.choice([0.0, 1e-3, 3e-4, rng.random()]), "betas": (rng.random() * 0.999, rng.random() * 0.9999),
                   "eps": rng.choice([1e-8, 1e-6, 1e-3]), "weight_decay": rng.choice([0.0, 0.1, 0.01]),
                   "maximize": rng.random() < 0.2}
        fused = rng.random() < 0.5
        step = rng.choice([1, 2, 3, 10, 1000, 100000])
        try:
            previous = optimizer._coefficients(dtype, options, step, fused)
        except ValueError:
            continue
        for later in (step + 1, step + 7):
            try:
                want = optimizer._coefficients(dtype, options, later, fused)
            except ValueError as error:
                with pytest.raises(ValueError, match=str(error)):
                    optimizer._next_coefficients(dtype, options, later, fused, previous)
                continue
            got = optimizer._next_coefficients(dtype, options, later, fused, previous)
            assert type(got) is type(want)
            assert bytes(got) == bytes(want), (trial, dtype, options, later)
            assert ctypes.addressof(got) != ctypes.addressof(previous)


def test_options_key_is_exact():
    """Equal keys only for the same option values and types; zeros keep their sign."""
    from namitorch_amd.optim.adam import _options_key
    base = [{"params": [], "lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 0.0, "maximize": False}]
    same = [{"params": [1], "lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 0.0, "maximize": False}]
    assert _options_key(base) == _options_key(same)
    for name, value in (("weight_decay", -0.0), ("lr", float(np.nextafter(1e-3, 1.0))), ("betas", (0.9, 0.99)),
                        ("betas", [0.9, 0.999]), ("weight_decay", 0), ("maximize", 0), ("eps", 1e-8 + 1e-24)):
        changed = [dict(base[0], **{name: value})]
        assert _options_key(changed) != _options_key(base), (name, value)
    assert _options_key([dict(base[0], betas=(0.0, -0.0))]) != _options_key([dict(base[0], betas=(-0.0, 0.0))])
    assert _options_key([dict(base[0], lr=float("nan"))]) is None
    assert _options_key([dict(base[0], lr=np.float32(1e-3))]) is None
