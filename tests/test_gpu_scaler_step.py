"""``GradScaler.step`` without an earlier ``unscale_`` (amp.py:194-196: the
reference's ``step`` unscales itself) queues the unscale, the finite check
and a device-gated AdamW pass together and waits once, after the pass is
queued.  Checked bit for bit against the host path (``unscale_``, then
``step``) over sequences with inf and NaN iterations, growth and backoff:
return values, scales, parameters, master weights, moments, step counts,
version counters and the unscaled gradients; with two optimizers stepped
separately in one iteration; with a deferred last micro-batch; and for an
optimizer whose ``step`` raises, which the reference reaches only after a
finite unscale."""

from __future__ import annotations

import math

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd.amp import GradScaler
from oracle import scaler as oscaler

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SHAPES = [(257, 129), (4099,), (64, 33), (7,)]
KW = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
# (parameter dtype, gradient dtype, master weights, state dtype)
LAYOUTS = {
    "f32": ("float32", "float32", False, None),
    "f16": ("float16", "float16", False, None),
    "c3": ("bfloat16", "float16", True, None),
    "c4": ("bfloat16", "bfloat16", True, "bfloat16"),
}


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view({2: np.uint16, 4: np.uint32, 8: np.uint64}[a.itemsize])


def _same(label, got, want):
    got, want = np.asarray(got), np.asarray(want)
    assert got.dtype == want.dtype and got.shape == want.shape, label
    assert np.array_equal(_bits(got), _bits(want)), label


def _build(values, layout):
    param_dtype, _, master, state_dtype = LAYOUTS[layout]
    params = [nt.Parameter(v, dtype=param_dtype, device=DEV) for v in values]
    options = dict(KW, master_weights=True, state_dtype=state_dtype) if master else dict(KW)
    if param_dtype == "float16":
        options["eps"] = 1e-4                                    # 1e-8 is zero in float16
    return params, nt.optim.AdamW(params, **options)


class _CountFinite:
    """Counts the host path's finite checks (GradScaler._finite)."""

    def __init__(self, monkeypatch):
        self.calls = 0
        original = GradScaler._finite

        def counted(gradients):
            self.calls += 1
            return original(gradients)
        monkeypatch.setattr(GradScaler, "_finite", staticmethod(counted))


def _state_of(params, optimizer):
    out = []
    for p in params:
        state = optimizer.state[id(p)]
        out.append((p.numpy(), state["exp_avg"].numpy(), state["exp_avg_sq"].numpy(),
                    state["master"].numpy() if "master" in state else None, state["step"],
                    p._version, state["exp_avg"]._version, state["exp_avg_sq"]._version))
    return out


@pytest.mark.parametrize("layout", sorted(LAYOUTS))
def test_step_without_unscale_matches_the_host_path(layout, monkeypatch):
    rng = np.random.default_rng(61)
    _, grad_dtype, _, _ = LAYOUTS[layout]
    values = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES]
    device_params, device_opt = _build(values, layout)
    host_params, host_opt = _build(values, layout)
    device_scaler = nt.GradScaler(init_scale=1024.0, growth_interval=3)
    host_scaler = nt.GradScaler(init_scale=1024.0, growth_interval=3)
    oracle_scaler = oscaler.Scaler(1024.0, growth_interval=3)
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    counter = _CountFinite(monkeypatch)
    poisons = {3: math.inf, 6: math.nan, 7: -math.inf}
    for k in range(10):
        grads = [(rng.standard_normal(s) * 1e-3 * oracle_scaler.scale).astype(np.float32) for s in SHAPES]
        if k in poisons:
            grads[k % len(SHAPES)].reshape(-1)[5] = poisons[k]
        for params in (device_params, host_params):
            for p, g in zip(params, grads):
                p.grad = nt.Tensor(g, dtype=grad_dtype, device=DEV)
        device_scaler.scale(loss)
        before = counter.calls
        stepped = device_scaler.step(device_opt)
        assert counter.calls == before, k                        # no host finite check: the device path ran
        device_scaler.update()
        host_scaler.scale(loss)
        finite = host_scaler.unscale_(host_opt)
        assert host_scaler.step(host_opt) == finite
        host_scaler.update()
        oracle_scaler.update(k in poisons)
        assert stepped == finite == (k not in poisons), k
        assert device_scaler.get_scale() == host_scaler.get_scale() == oracle_scaler.scale, k
        for i, (p, q) in enumerate(zip(device_params, host_params)):
            _same(f"grad {k} {i}", p.grad.numpy(), q.grad.numpy())   # unscaled in place, also when skipped
            assert p.grad._version == q.grad._version, (k, i)
    for i, (got, want) in enumerate(zip(_state_of(device_params, device_opt), _state_of(host_params, host_opt))):
        for name, a, b in zip(("param", "exp_avg", "exp_avg_sq", "master"), got[:4], want[:4]):
            if b is not None:
                _same(f"{name} {i}", a, b)
        assert got[4:] == want[4:] == (7,) + got[5:], i                # steps and version counters
    assert device_scaler.state_dict() == host_scaler.state_dict()


def test_two_optimizers_stepped_separately():
    """step(a), step(b), update(): each optimizer skips only on its own
    non-finite gradients; the scale backs off once for the iteration."""
    rng = np.random.default_rng(62)
    values = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES]
    runs = []
    for explicit in (False, True):
        params = [nt.Parameter(v, device=DEV) for v in values]
        opts = [nt.optim.AdamW(params[:2], **KW), nt.optim.AdamW(params[2:], **KW)]
        scaler = nt.GradScaler(init_scale=256.0, growth_interval=2)
        loss = nt.Tensor(np.float32(1.0), device=DEV)
        draw = np.random.default_rng(63)
        results = []
        for k in range(6):
            grads = [(draw.standard_normal(s) * 1e-3 * scaler.get_scale()).astype(np.float32) for s in SHAPES]
            if k == 2:
                grads[3][1] = np.inf                              # only the second optimizer's
            for p, g in zip(params, grads):
                p.grad = nt.Tensor(g, device=DEV)
            scaler.scale(loss)
            if explicit:
                for opt in opts:
                    scaler.unscale_(opt)
            results.append([scaler.step(opt) for opt in opts])
            scaler.update()
            results.append(scaler.get_scale())
        runs.append((results, [p.numpy() for p in params], [p._version for p in params],
                     [opts[i // 2].state[id(p)]["step"] for i, p in enumerate(params)]))
    (device, device_values, device_versions, device_steps), (host, host_values, host_versions, host_steps) = runs
    assert device == host
    assert device[4] == [True, False] and device[5] == 256.0      # growth after 0-1, backoff at 2
    for i, (a, b) in enumerate(zip(device_values, host_values)):
        _same(f"param {i}", a, b)
    assert device_versions == host_versions and device_steps == host_steps == [6, 6, 5, 5]


def test_optimizer_errors_only_after_a_finite_unscale():
    """An optimizer whose step raises (a NaN learning rate) is not stepped by
    the reference when the gradients are non-finite, so nothing is raised
    and nothing changes; with finite gradients the same error is raised as
    on the host path."""
    rng = np.random.default_rng(64)
    values = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES]
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    errors = []
    for explicit in (False, True):
        params = [nt.Parameter(v, device=DEV) for v in values]
        optimizer = nt.optim.AdamW(params, **KW)
        scaler = nt.GradScaler(init_scale=64.0)
        for p in params:                                          # one ordinary step first
            p.grad = nt.Tensor(np.full(p.shape, 0.5, np.float32), device=DEV)
        scaler.scale(loss)
        assert scaler.step(optimizer)
        scaler.update()
        optimizer.param_groups[0]["lr"] = float("nan")
        snapshot = [(p.numpy(), p._version, optimizer.state[id(p)]["step"]) for p in params]
        for p in params:
            g = np.full(p.shape, 0.5, np.float32)
            g.reshape(-1)[0] = np.inf
            p.grad = nt.Tensor(g, device=DEV)
        scaler.scale(loss)
        if explicit:
            assert not scaler.unscale_(optimizer)
        assert scaler.step(optimizer) is False
        scaler.update()
        assert scaler.get_scale() == 32.0
        for p, (value, version, step) in zip(params, snapshot):
            _same("skipped", p.numpy(), value)
            assert (p._version, optimizer.state[id(p)]["step"]) == (version, step)
        for p in params:
            p.grad = nt.Tensor(np.full(p.shape, 0.5, np.float32), device=DEV)
        scaler.scale(loss)
        if explicit:
            assert scaler.unscale_(optimizer)
        with pytest.raises(Exception) as raised:
            scaler.step(optimizer)
        errors.append((type(raised.value), str(raised.value)))
        with pytest.raises(RuntimeError, match="Call step\\(\\) for every unscaled optimizer before update\\(\\)."):
            scaler.update()
    assert errors[0] == errors[1]


def test_deferred_accumulation_through_step_alone():
    """The last micro-batch's deferred accumulation (accumulate_grads(...,
    defer=True)) is added inside the pre-pass and the pass of step alone,
    with the values, versions and skip of the host path."""
    rng = np.random.default_rng(65)
    values = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES]
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    runs = []
    for explicit in (False, True):
        params, optimizer = _build(values, "c3")
        scaler = nt.GradScaler(init_scale=512.0, growth_interval=2)
        draw = np.random.default_rng(66)
        out = []
        for k in range(5):
            micro = [[(draw.standard_normal(s) * 5e-4 * scaler.get_scale()).astype(np.float32) for s in SHAPES]
                     for _ in range(2)]
            if k == 3:
                micro[1][0].reshape(-1)[9] = np.inf               # in the deferred micro-batch
            for p in params:
                p.grad = None
            nt.accumulate_grads(params, [nt.Tensor(g, dtype="float16", device=DEV) for g in micro[0]])
            nt.accumulate_grads(params, [nt.Tensor(g, dtype="float16", device=DEV) for g in micro[1]], defer=True)
            scaler.scale(loss)
            if explicit:
                scaler.unscale_(optimizer)
            out.append(scaler.step(optimizer))
            scaler.update()
            out.append(scaler.get_scale())
        state = [optimizer.state[id(p)] for p in params]
        runs.append((out, [p.numpy() for p in params] + [s["master"].numpy() for s in state]
                     + [p.grad.numpy() for p in params],
                     [(p._version, p.grad._version, s["step"]) for p, s in zip(params, state)]))
    (device, device_arrays, device_counts), (host, host_arrays, host_counts) = runs
    assert device == host and device[6] is False
    for i, (a, b) in enumerate(zip(device_arrays, host_arrays)):
        _same(f"array {i}", a, b)
    assert device_counts == host_counts


def test_optimizer_subclasses_take_the_synchronizing_path():
    """A subclass of AdamW may do its own work in step(): GradScaler.step and
    fused_step call it only after a finite unscale, as the reference does,
    and give the exact class's results."""

    class Counted(nt.optim.AdamW):
        calls = 0

        def step(self, *args, **kwargs):
            type(self).calls += 1
            return super().step(*args, **kwargs)

    rng = np.random.default_rng(67)
    values = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES]
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    finals = []
    for use_fused in (False, True):
        for cls in (Counted, nt.optim.AdamW):
            Counted.calls = 0
            params = [nt.Parameter(v, device=DEV) for v in values]
            optimizer = cls(params, **KW)
            scaler = nt.GradScaler(init_scale=128.0)
            draw = np.random.default_rng(68)
            for k in range(4):
                grads = [(draw.standard_normal(s) * 1e-3 * 128.0).astype(np.float32) for s in SHAPES]
                if k == 1:
                    grads[2][3] = np.nan
                for p, g in zip(params, grads):
                    p.grad = nt.Tensor(g, device=DEV)
                scaler.scale(loss)
                if use_fused:
                    assert nt.amp.fused_step(optimizer, scaler).updated == (k != 1)
                else:
                    assert scaler.step(optimizer) == (k != 1)
                    scaler.update()
            if cls is Counted:
                assert Counted.calls == 3, use_fused               # not called on the skipped step
            finals.append([p.numpy() for p in params] + [scaler.get_scale()])
    for a, b in zip(finals[0][:-1] + finals[2][:-1], finals[1][:-1] + finals[3][:-1]):
        _same("subclass against AdamW", a, b)
    assert finals[0][-1] == finals[1][-1] and finals[2][-1] == finals[3][-1]
