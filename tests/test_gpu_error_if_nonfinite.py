"""``fused_step(..., error_if_nonfinite=True)``: clip_grad_norm_'s flag
(optim/clip_grad.py:99-105) on the path without a host wait.

Without a scaler a non-finite norm must change nothing, because the
reference raises before clipping or stepping.  The device skips both, and
the reference's RuntimeError (text pinned by tests/golden/golden.json) is
raised at the first access to the StepResult, or else at the start of the
next fused_step.  With finite gradients the flag changes nothing.  With a
scaler the clip runs only after a finite unscale, so the flag never raises
(training/runner.py:248-249)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import namitorch_amd as nt
from oracle import adam as oadam
from oracle import clip as oclip

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SHAPES = [(301, 17), (4099,)]
KW = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
GOLDEN = json.loads((Path(__file__).parent / "golden" / "golden.json").read_text())


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view({2: np.uint16, 4: np.uint32, 8: np.uint64}[a.itemsize]).copy()


def _setup(seed):
    rng = np.random.default_rng(seed)
    values = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES]
    params = [nt.Parameter(v, device=DEV) for v in values]
    return rng, values, params, nt.optim.AdamW(params, **KW)


def _grads(rng, bad=None):
    grads = [(rng.standard_normal(s) * 1e-2).astype(np.float32) for s in SHAPES]
    if bad is not None:
        grads[1][17] = bad
    return grads


def _attach(params, grads):
    for p, g in zip(params, grads):
        p.grad = nt.Tensor(g, device=DEV)


def _snapshot(params, optimizer):
    out = []
    for p in params:
        state = optimizer.state[id(p)]
        out.append((_bits(p.numpy()), _bits(p.grad.numpy()), state["step"], _bits(state["exp_avg"].numpy()),
                    _bits(state["exp_avg_sq"].numpy()), p._version, p.grad._version, state["exp_avg"]._version))
    return out


def _same_snapshot(a, b):
    for x, y in zip(a, b):
        for u, v in zip(x, y):
            if isinstance(u, np.ndarray):
                assert np.array_equal(u, v)
            else:
                assert u == v


@pytest.mark.parametrize("bad", [np.inf, np.nan])
def test_nonfinite_norm_raises_at_the_result_and_changes_nothing(bad):
    rng, _, params, optimizer = _setup(3)
    _attach(params, _grads(rng))
    assert nt.amp.fused_step(optimizer, max_norm=1.0, error_if_nonfinite=True).updated
    _attach(params, _grads(rng, bad))
    before = _snapshot(params, optimizer)
    result = nt.amp.fused_step(optimizer, max_norm=1.0, error_if_nonfinite=True)
    expected = GOLDEN["errors"]["nonfinite_norm"] if bad == np.inf else \
        "Cannot clip gradients with nonfinite total norm nan."
    for _ in range(2):                                  # every access raises
        with pytest.raises(RuntimeError) as error:
            result.norm
        assert str(error.value) == expected
    _same_snapshot(_snapshot(params, optimizer), before)  # no clip, no step, no version bump
    # raised at the result: the next fused_step runs normally
    _attach(params, _grads(rng))
    assert nt.amp.fused_step(optimizer, max_norm=1.0, error_if_nonfinite=True).updated
    assert optimizer.state[id(params[0])]["step"] == 2


def test_deferred_error_raises_at_the_next_fused_step():
    rng, values, params, optimizer = _setup(5)
    _attach(params, _grads(rng, np.inf))
    nt.amp.fused_step(optimizer, max_norm=1.0, error_if_nonfinite=True)   # result never read
    grads = _grads(rng)
    _attach(params, grads)
    with pytest.raises(RuntimeError, match="Cannot clip gradients with nonfinite total norm inf."):
        nt.amp.fused_step(optimizer, max_norm=1.0, error_if_nonfinite=True)
    assert all(p.grad._pending is None for p in params)                    # raised before any change
    assert optimizer.state[id(params[0])]["step"] == 0
    result = nt.amp.fused_step(optimizer, max_norm=1.0, error_if_nonfinite=True)
    norm = oclip.total_norm([g.astype(np.float64) for g in grads])
    assert abs(result.norm - norm) <= 1e-12 * norm
    coefficient = oclip.clip_coefficient(1.0, result.norm)
    for p, v, g in zip(params, values, grads):
        clipped = np.asarray(oclip.clip_apply(g.astype(np.float64), coefficient, "float32"), np.float32) \
            if coefficient < 1 else g
        want, m, v2 = v.copy(), np.zeros_like(v), np.zeros_like(v)
        oadam.adam_step(want, clipped, m, v2, 1, **KW)
        assert np.array_equal(_bits(p.numpy()), _bits(want))


def test_finite_gradients_unchanged_by_the_flag():
    rng_a, _, params_a, opt_a = _setup(7)
    rng_b, _, params_b, opt_b = _setup(7)
    for k in range(3):
        grads = _grads(rng_a)
        _grads(rng_b)
        _attach(params_a, grads)
        _attach(params_b, grads)
        ra = nt.amp.fused_step(opt_a, max_norm=0.5, error_if_nonfinite=True)
        rb = nt.amp.fused_step(opt_b, max_norm=0.5)
        assert ra.updated and rb.updated and ra.norm == rb.norm, k
    _same_snapshot(_snapshot(params_a, opt_a), _snapshot(params_b, opt_b))


def test_with_a_scaler_the_flag_never_raises():
    rng, _, params, optimizer = _setup(9)
    scaler = nt.GradScaler(init_scale=1.0)
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    for bad in (np.inf, None):
        _attach(params, _grads(rng, bad))
        scaler.scale(loss)
        result = nt.amp.fused_step(optimizer, scaler, max_norm=1.0, error_if_nonfinite=True)
        assert result.finite == (bad is None) and result.updated == (bad is None)
    assert scaler.get_scale() == 0.5
    with pytest.raises(TypeError, match="error_if_nonfinite must be a Python bool."):
        nt.amp.fused_step(optimizer, scaler, max_norm=1.0, error_if_nonfinite=1)
