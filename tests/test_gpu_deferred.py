"""Deferred last-micro-batch accumulation (``accumulate_grads(..., defer=True)``):
the pre-pass and the AdamW pass add the incoming gradient as they read the
stored one (plan column 5).  Every observable result must equal the eager
accumulation's bit for bit: parameters, moments, master weights, norms,
the scale, the gradients read afterwards and version counters.  The eager
path is itself pinned to the reference's accumulate_gradient outputs
(test_gpu_grads.py); one case is also checked against the oracle directly.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd import _native
from oracle import adam as oadam
from oracle import grads as ograds

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
SHAPES = [(64, 33), (4096,), (4097,), (3,), (1,), (0,), (2048, 3), (5, 7)]
SECOND = [0, 2, 3, 4, 6, 7]          # parameters that receive a second micro-batch (1 and 5 do not)
LAYOUTS = [("float32", False), ("bfloat16", True), ("float16", True), ("float16", False)]


def _micro(rng, params, scale):
    return [nt.Tensor((rng.standard_normal(p.shape) * 1e-3 * scale).astype(np.float32), dtype=p.dtype, device=DEV)
            for p in params]


def _run(mode, defer, param_dtype, master, steps=3, skip_second=()):
    rng = np.random.default_rng(7)
    params = [nt.Parameter((rng.standard_normal(s) * 0.05).astype(np.float32), dtype=param_dtype, device=DEV)
              for s in SHAPES]
    optimizer = nt.optim.AdamW(params, lr=1e-3, eps=1e-4, weight_decay=0.1, master_weights=master)   # eps > 0 in float16
    amp = mode in ("api_amp", "fused_amp")
    scaler = nt.GradScaler(init_scale=1024.0) if amp else None
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    norms, versions = [], []
    for step in range(steps):
        optimizer.zero_grad()
        first = _micro(rng, params, 1024.0 if amp else 1.0)
        second = _micro(rng, params, 1024.0 if amp else 1.0)
        if amp and step == 1:
            second[3][...] = np.float32(np.inf)           # a non-finite step: skipped, scale backs off
        nt.accumulate_grads(params, first)
        if step not in skip_second:
            nt.accumulate_grads([params[i] for i in SECOND], [second[i] for i in SECOND], defer=defer)
        if amp:
            scaler.scale(loss)
        if mode == "plain":
            optimizer.step()
        elif mode == "api":
            norms.append(nt.optim.clip_grad_norm_(params, 1.0).item())
            optimizer.step()
        elif mode == "api_amp":
            finite = scaler.unscale_(optimizer)
            if finite:
                norms.append(nt.optim.clip_grad_norm_(params, 1.0).item())
            scaler.step(optimizer)
            scaler.update()
        else:
            result = nt.amp.fused_step(optimizer, scaler, max_norm=1.0)
            norms.append((result.finite, result.norm))
        versions.append([p.grad._version for p in params])
    state = optimizer.state
    out = {
        "params": [p.bits().tobytes() for p in params],
        "states": [[state[id(p)][k].bits().tobytes() for k in sorted(state[id(p)]) if k != "step"] for p in params],
        "steps": [state[id(p)]["step"] for p in params],
        "grads": [p.grad.bits().tobytes() for p in params],
        "norms": norms,
        "versions": versions,
        "param_versions": [p._version for p in params],
        "scale": None if scaler is None else scaler.get_scale(),
    }
    return out


@pytest.mark.parametrize("layout", LAYOUTS, ids=[f"{d}{'-master' if m else ''}" for d, m in LAYOUTS])
@pytest.mark.parametrize("mode", ["plain", "api", "api_amp", "fused", "fused_amp"])
def test_deferred_equals_eager(mode, layout):
    param_dtype, master = layout
    eager = _run(mode, False, param_dtype, master)
    deferred = _run(mode, True, param_dtype, master)
    for key in eager:
        assert deferred[key] == eager[key], key


def test_steps_with_and_without_deferral_replay_exactly():
    """Steps mix deferred and plain gradients, so the step memo is built
    (step 1), replayed (step 2), bypassed (step 3) and rebuilt; results
    equal the eager run's."""
    eager = _run("plain", False, "float32", False, steps=6, skip_second=(1, 2, 4))
    deferred = _run("plain", True, "float32", False, steps=6, skip_second=(1, 2, 4))
    for key in eager:
        assert deferred[key] == eager[key], key


def test_deferred_step_matches_oracle():
    rng = np.random.default_rng(3)
    p0 = (rng.standard_normal(5000) * 0.05).astype(np.float32)
    g1 = (rng.standard_normal(5000) * 1e-3).astype(np.float32)
    g2 = (rng.standard_normal(5000) * 1e-3).astype(np.float32)
    param = nt.Parameter(p0, device=DEV)
    optimizer = nt.optim.AdamW([param], lr=1e-3)
    nt.accumulate_grads([param], [nt.Tensor(g1, device=DEV)])
    incoming = nt.Tensor(g2, device=DEV)
    nt.accumulate_grads([param], [incoming], defer=True)
    assert param.grad._incoming is not None and param.grad._incoming[0] is incoming
    optimizer.step()
    g = ograds.accumulate(ograds.accumulate(None, g1, "float32"), g2, "float32")
    ref, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    oadam.adam_step(ref, g, m, v, 1, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2)
    assert param.numpy().tobytes() == ref.tobytes()
    assert param.grad._incoming is not None                  # the sum was never written ...
    assert param.grad.numpy().tobytes() == g.tobytes()       # ... until it is read
    assert param.grad._incoming is None


def test_read_before_step_sees_the_sum_and_versions_match():
    rng = np.random.default_rng(4)
    values = [(rng.standard_normal(777) * 1e-2).astype(np.float32) for _ in range(2)]
    results = []
    for defer in (False, True):
        param = nt.Parameter(np.zeros(777, np.float32), dtype="bfloat16", device=DEV)
        nt.accumulate_grads([param], [nt.Tensor(values[0], dtype="bfloat16", device=DEV)])
        version = param.grad._version
        nt.accumulate_grads([param], [nt.Tensor(values[1], dtype="bfloat16", device=DEV)], defer=defer)
        assert param.grad._version == version + 1
        results.append(param.grad.bits().tobytes())
    assert results[0] == results[1]


def test_modified_incoming_gradient_raises():
    param = nt.Parameter(np.zeros(64, np.float32), device=DEV)
    nt.accumulate_grads([param], [nt.Tensor(np.ones(64, np.float32), device=DEV)])
    incoming = nt.Tensor(np.ones(64, np.float32), device=DEV)
    nt.accumulate_grads([param], [incoming], defer=True)
    incoming[...] = 5.0
    optimizer = nt.optim.AdamW([param], lr=1e-3)
    with pytest.raises(RuntimeError, match="deferred accumulation"):
        optimizer.step()
    with pytest.raises(RuntimeError, match="deferred accumulation"):
        nt.amp.fused_step(optimizer, None, max_norm=1.0)


def test_zero_grad_keep_buffers_drops_the_deferred_addend():
    param = nt.Parameter(np.zeros(100, np.float32), device=DEV)
    nt.accumulate_grads([param], [nt.Tensor(np.ones(100, np.float32), device=DEV)])
    nt.accumulate_grads([param], [nt.Tensor(np.ones(100, np.float32), device=DEV)], defer=True)
    nt.optim.AdamW([param]).zero_grad(set_to_none=False)
    assert param.grad._incoming is None and not np.any(param.grad.bits())


def test_unaligned_incoming_accumulates_eagerly():
    import torch
    base = torch.zeros(4098, dtype=torch.float32, device=DEV)
    base[1:].copy_(torch.full((4097,), 0.25))
    incoming = nt.Tensor._from_storage(base[1:])             # 4-byte aligned only
    param = nt.Parameter(np.zeros(4097, np.float32), device=DEV)
    nt.accumulate_grads([param], [nt.Tensor(np.full(4097, 0.5, np.float32), device=DEV)])
    nt.accumulate_grads([param], [incoming], defer=True)
    assert param.grad._incoming is None
    assert np.all(param.grad.numpy() == np.float32(0.75))


def test_abi_refuses_incoming_plans_outside_the_pass():
    """Entry points that do not read column 5 refuse a plan that sets it,
    and float64 gradients cannot take one."""
    grads = [nt.Tensor(np.ones(n, np.float32), device=DEV) for n in (4096, 10)]
    addends = [nt.Tensor(np.ones(n, np.float32), device=DEV) for n in (4096, 10)]
    backend = nt.get_backend(DEV)
    layout = (_native.NT_DTYPE_NONE, _native.NT_F32, _native.NT_DTYPE_NONE, _native.NT_DTYPE_NONE)
    rows = [(0, 0, 0, 0, 0, g._numel, 0) for g in grads]
    plan = backend.plan(rows, layout, pointers={1: [g._ptr for g in grads], 5: [addends[0]._ptr, 0]})
    xform = _native.GradXform()
    with pytest.raises(ValueError, match="incoming"):
        _native.call("nt_grad_apply", plan.handle, ctypes.byref(xform), backend.stream())
    with pytest.raises(ValueError, match="incoming"):
        _native.call("nt_grad_zero", plan.handle, backend.stream())
    block = backend.new_ctrl()
    with pytest.raises(ValueError, match="incoming"):
        _native.call("nt_grad_norm_pow", plan.handle, block.data_ptr(), 3.0, -1.0, 1.0, 0, 0, 0, backend.stream())
    # The pre-pass takes it: sum of squares of (1 + 1) over the first tensor, 1 over the second.
    backend.grad_prepass(plan, None)
    backend.grad_finalize(plan, block.data_ptr(), norm_type=2.0)
    assert backend.read_ctrl(block).sumsq == 4.0 * 4096 + 10
    wide = [nt.Tensor(np.ones(8, np.float64), device=DEV)]
    layout64 = (_native.NT_DTYPE_NONE, _native.NT_F64, _native.NT_DTYPE_NONE, _native.NT_DTYPE_NONE)
    with pytest.raises(TypeError, match="float64"):
        backend.plan([(0, 0, 0, 0, 0, 8, 0)], layout64, pointers={1: [wide[0]._ptr], 5: [wide[0]._ptr]})
