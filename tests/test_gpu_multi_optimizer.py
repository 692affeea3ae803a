"""Several optimizers sharing one GradScaler iteration, without a host wait.

``amp.fused_step([opt_a, opt_b], scaler, max_norm=...)`` is the reference
loop run over several optimizers: ``unscale_`` of each, ``clip_grad_norm_``
over all their parameters when every ``unscale_`` returned True, ``step``
of each and one ``update`` (amp.py:169-233, training/runner.py:248-251).
As in the reference, an optimizer steps unless its own gradients are
non-finite (GradScaler.step re-checks only them, amp.py:209-217), and the
scale backs off once if any optimizer's are (amp.py:224-233).

Checked against the oracle (``scaler.unscale``, ``clip``, ``adam``,
``scaler.Scaler``) and against the same iterations through the
synchronizing API, with one float32 optimizer and one bfloat16-model /
float32-master optimizer: finite/updated flags, the loss-scale sequence,
step counts and versions exact; the norm within 1e-12 of the oracle's and
bit-equal to the synchronizing path's; parameters, master weights and
moments bit-exact.  Eight optimizers (one device combine's limit) and nine
(the synchronizing fallback) match the reference loop too.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import namitorch_amd as nt
from oracle import adam as oadam
from oracle import clip as oclip
from oracle import lowp
from oracle import scaler as oscaler

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SHAPES_A = [(301, 17), (257,)]
SHAPES_B = [(4099,), (64, 33)]
KW = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
NORM_RTOL = 1e-12


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view({2: np.uint16, 4: np.uint32, 8: np.uint64}[a.itemsize])


def _f64_bits(x) -> int:
    return int(np.float64(x).view(np.uint64))


def _same(label, got, want):
    got, want = np.asarray(got), np.asarray(want)
    nan = np.isnan(got.astype(np.float64)) & np.isnan(want.astype(np.float64))
    assert np.all((_bits(got) == _bits(want)) | nan), label


def _build(values_a, values_b):
    params_a = [nt.Parameter(v, device=DEV) for v in values_a]
    params_b = [nt.Parameter(v, dtype="bfloat16", device=DEV) for v in values_b]
    opt_a = nt.optim.AdamW(params_a, **KW)
    opt_b = nt.optim.AdamW(params_b, master_weights=True, **KW)
    return params_a, params_b, opt_a, opt_b


def _scaled(rng, shapes, dtype, scale, poison):
    out = []
    for k, shape in enumerate(shapes):
        g = rng.standard_normal(shape) * 1e-3 * scale
        if poison is not None and k == len(shapes) - 1:
            g.reshape(-1)[7] = poison
        out.append(lowp.round_to(dtype, g))
    return out


@pytest.mark.parametrize("max_norm", [None, 0.02])
def test_two_optimizers_one_scaler(max_norm):
    rng = np.random.default_rng(41)
    values_a = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES_A]
    values_b = [lowp.round_bf16((rng.standard_normal(s) * 0.02).astype(np.float32)) for s in SHAPES_B]
    fused = _build(values_a, values_b)
    synced = _build(values_a, values_b)
    scaler_f = nt.GradScaler(init_scale=65536.0, growth_interval=3)
    scaler_s = nt.GradScaler(init_scale=65536.0, growth_interval=3)
    oracle_scaler = oscaler.Scaler(65536.0, growth_interval=3)
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    # oracle state
    pa = [v.copy() for v in values_a]
    ma, va = [np.zeros_like(v) for v in pa], [np.zeros_like(v) for v in pa]
    master = [v.astype(np.float32).copy() for v in values_b]
    mb, vb = [np.zeros_like(v) for v in master], [np.zeros_like(v) for v in master]
    steps_a = steps_b = 0
    # growth_interval 3: growth after steps 0-2 and 7-9, backoff at 3, 5 and 6
    poisons = {3: ("a", math.inf), 5: ("b", math.nan), 6: ("a", -math.inf)}
    scales = []
    for k in range(10):
        scale = oracle_scaler.scale
        which, bad = poisons.get(k, (None, None))
        ga = _scaled(rng, SHAPES_A, "float32", scale, bad if which == "a" else None)
        gb = _scaled(rng, SHAPES_B, "bfloat16", scale, bad if which == "b" else None)
        for (params_a, params_b, _, _) in (fused, synced):
            for p, g in zip(params_a, ga):
                p.grad = nt.Tensor(g, device=DEV)
            for p, g in zip(params_b, gb):
                p.grad = nt.Tensor(g, dtype="bfloat16", device=DEV)
        # fused: one call, no host wait
        params_a, params_b, opt_a, opt_b = fused
        scaler_f.scale(loss)
        results = nt.amp.fused_step([opt_a, opt_b], scaler_f, max_norm=max_norm)
        assert isinstance(results, list) and len(results) == 2
        # the synchronizing API, the reference loop over both optimizers
        params_a2, params_b2, opt_a2, opt_b2 = synced
        scaler_s.scale(loss)
        finite_a2, finite_b2 = scaler_s.unscale_(opt_a2), scaler_s.unscale_(opt_b2)
        sync_norm = None
        if finite_a2 and finite_b2 and max_norm is not None:
            sync_norm = nt.optim.clip_grad_norm_(params_a2 + params_b2, max_norm).item()
        updated_a2, updated_b2 = scaler_s.step(opt_a2), scaler_s.step(opt_b2)
        scaler_s.update()
        # oracle
        ua = [oscaler.unscale(g, scale, "float32") for g in ga]
        ub = [oscaler.unscale(g, scale, "bfloat16") for g in gb]
        finite_a, finite_b = oscaler.finite(ua), oscaler.finite(ub)
        want_norm = oclip.total_norm([g.astype(np.float64) for g in ua + ub])
        norm = results[0].norm
        if max_norm is not None:
            assert results[1].norm == norm or (math.isnan(norm) and math.isnan(results[1].norm)), k
            if math.isfinite(want_norm):
                assert abs(norm - want_norm) <= NORM_RTOL * want_norm, (k, norm, want_norm)
            else:
                assert (math.isnan(norm) and math.isnan(want_norm)) or norm == want_norm, (k, norm, want_norm)
            if sync_norm is not None:
                assert _f64_bits(norm) == _f64_bits(sync_norm), (k, norm, sync_norm)
            if finite_a and finite_b:
                coefficient = oclip.clip_coefficient(max_norm, norm)
                if coefficient < 1:
                    ua = [oclip.clip_apply(g.astype(np.float64), coefficient, "float32") for g in ua]
                    ub = [oclip.clip_apply(g.astype(np.float64), coefficient, "bfloat16") for g in ub]
        else:
            assert results[0].norm is None
        if finite_a:
            steps_a += 1
            for i, g in enumerate(ua):
                oadam.adam_step(pa[i], np.asarray(g, np.float32), ma[i], va[i], steps_a, **KW)
        if finite_b:
            steps_b += 1
            for i, g in enumerate(ub):
                oadam.master_step(master[i], np.asarray(g, np.float32), mb[i], vb[i], steps_b, **KW)
        oracle_scaler.update(not (finite_a and finite_b))
        assert [r.finite for r in results] == [finite_a, finite_b] == [finite_a2, finite_b2], k
        assert [r.updated for r in results] == [finite_a, finite_b] == [updated_a2, updated_b2], k
        assert results[0].scale == results[1].scale == oracle_scaler.scale == scaler_s.get_scale(), k
        assert scaler_f.get_scale() == oracle_scaler.scale, k
        scales.append(oracle_scaler.scale)
    # final state: the oracle, and the synchronizing path (versions too)
    for label, (params_a, params_b, opt_a, opt_b) in (("fused", fused), ("synced", synced)):
        for i, p in enumerate(params_a):
            state = opt_a.state[id(p)]
            assert state["step"] == steps_a, (label, i)
            _same(f"{label} a{i} param", p.numpy(), pa[i])
            _same(f"{label} a{i} exp_avg", state["exp_avg"].numpy(), ma[i])
            _same(f"{label} a{i} exp_avg_sq", state["exp_avg_sq"].numpy(), va[i])
        for i, p in enumerate(params_b):
            state = opt_b.state[id(p)]
            assert state["step"] == steps_b, (label, i)
            _same(f"{label} b{i} master", state["master"].numpy(), master[i])
            _same(f"{label} b{i} param", p.numpy(), lowp.round_bf16(master[i]))
            _same(f"{label} b{i} exp_avg", state["exp_avg"].numpy(), mb[i])
            _same(f"{label} b{i} exp_avg_sq", state["exp_avg_sq"].numpy(), vb[i])
    (fa, fb, foa, fob), (sa, sb, soa, sob) = fused, synced
    for p, q in zip(fa + fb, sa + sb):
        assert p._version == q._version and p.grad._version == q.grad._version
    assert (steps_a, steps_b) == (8, 9)
    assert scales == [65536.0, 65536.0, 131072.0, 65536.0, 65536.0, 32768.0, 16384.0, 16384.0, 16384.0, 32768.0]


def test_two_optimizers_without_a_scaler():
    """No scaler: one clip over both optimizers' gradients, then both step."""
    rng = np.random.default_rng(43)
    values_a = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES_A]
    values_b = [lowp.round_bf16((rng.standard_normal(s) * 0.02).astype(np.float32)) for s in SHAPES_B]
    fused, synced = _build(values_a, values_b), _build(values_a, values_b)
    for k in range(3):
        ga = _scaled(rng, SHAPES_A, "float32", 1.0, None)
        gb = _scaled(rng, SHAPES_B, "bfloat16", 1.0, None)
        for (params_a, params_b, _, _) in (fused, synced):
            for p, g in zip(params_a, ga):
                p.grad = nt.Tensor(g, device=DEV)
            for p, g in zip(params_b, gb):
                p.grad = nt.Tensor(g, dtype="bfloat16", device=DEV)
        results = nt.amp.fused_step([fused[2], fused[3]], max_norm=0.02)
        norm = nt.optim.clip_grad_norm_(synced[0] + synced[1], 0.02, error_if_nonfinite=True).item()
        synced[2].step()
        synced[3].step()
        assert [r.updated for r in results] == [True, True]
        assert _f64_bits(results[0].norm) == _f64_bits(norm), k
    for p, q in zip(fused[0] + fused[1], synced[0] + synced[1]):
        _same("param", p.numpy(), q.numpy())
        assert p._version == q._version and p.grad._version == q.grad._version
    for opt_f, opt_s, params_f, params_s in ((fused[2], synced[2], fused[0], synced[0]),
                                             (fused[3], synced[3], fused[1], synced[1])):
        for p, q in zip(params_f, params_s):
            for name in opt_f.state[id(p)]:
                if name != "step":
                    _same(name, opt_f.state[id(p)][name].numpy(), opt_s.state[id(q)][name].numpy())


def test_refusals_match_the_reference():
    """Shared gradients and a repeated optimizer raise unscale_'s errors
    before anything changes."""
    rng = np.random.default_rng(47)
    values_a = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES_A]
    params = [nt.Parameter(v, device=DEV) for v in values_a]
    for p in params:
        p.grad = nt.Tensor(np.ones(p.shape, np.float32), device=DEV)
    first = nt.optim.AdamW(params, **KW)
    second = nt.optim.AdamW(params[:1], **KW)
    scaler = nt.GradScaler()
    scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
    before = [p.grad._version for p in params]
    with pytest.raises(RuntimeError, match="Optimizers cannot share gradients in the same GradScaler iteration."):
        nt.amp.fused_step([first, second], scaler)
    with pytest.raises(RuntimeError, match="unscale_ may be called only once per optimizer between update"):
        nt.amp.fused_step([first, first], scaler)
    assert [p.grad._version for p in params] == before
    assert all(p.grad._pending is None for p in params)
    assert all(len(first.state.get(id(p), {})) == 0 for p in params)
    results = nt.amp.fused_step([first], scaler)                  # a one-element list is one iteration too
    assert [r.updated for r in results] == [True]


@pytest.mark.parametrize("count", [8, 9])
def test_combine_limit(count):
    """Eight optimizers are the most one device combine takes; a ninth makes
    fused_step take the synchronizing API.  Both give the reference loop's
    flags, scales, states and versions bit for bit, with one optimizer's
    gradients non-finite at step 2 (only it skips, the scale backs off)."""
    rng = np.random.default_rng(53 + count)
    sizes = [257 + 64 * i for i in range(count)]
    values = [(rng.standard_normal(n) * 0.02).astype(np.float32) for n in sizes]

    def build():
        params = [nt.Parameter(v, device=DEV) for v in values]
        return params, [nt.optim.AdamW([p], **KW) for p in params]

    (params_f, opts_f), (params_s, opts_s) = build(), build()
    scaler_f = nt.GradScaler(init_scale=1024.0, growth_interval=2)
    scaler_s = nt.GradScaler(init_scale=1024.0, growth_interval=2)
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    for k in range(5):
        grads = [(rng.standard_normal(n) * 1e-3 * scaler_s.get_scale()).astype(np.float32) for n in sizes]
        if k == 2:
            grads[5][11] = np.inf
        for params in (params_f, params_s):
            for p, g in zip(params, grads):
                p.grad = nt.Tensor(g, device=DEV)
        scaler_f.scale(loss)
        results = nt.amp.fused_step(opts_f, scaler_f, max_norm=0.02)
        assert all((r._device_step is not None) == (count <= _native_max()) for r in results), k
        scaler_s.scale(loss)
        finite = [scaler_s.unscale_(opt) for opt in opts_s]
        norm = nt.optim.clip_grad_norm_(params_s, 0.02).item() if all(finite) else None
        updated = [scaler_s.step(opt) for opt in opts_s]
        scaler_s.update()
        assert [r.finite for r in results] == finite, k
        assert [r.updated for r in results] == updated, k
        assert updated == [not (k == 2 and i == 5) for i in range(count)], k
        if norm is not None:
            assert all(_f64_bits(r.norm) == _f64_bits(norm) for r in results), k
        assert results[0].scale == scaler_s.get_scale() == scaler_f.get_scale(), k
    for i, (p, q) in enumerate(zip(params_f, params_s)):
        sf, ss = opts_f[i].state[id(p)], opts_s[i].state[id(q)]
        assert sf["step"] == ss["step"] == (4 if i == 5 else 5), i
        _same(f"param {i}", p.numpy(), q.numpy())
        _same(f"exp_avg {i}", sf["exp_avg"].numpy(), ss["exp_avg"].numpy())
        _same(f"exp_avg_sq {i}", sf["exp_avg_sq"].numpy(), ss["exp_avg_sq"].numpy())
        assert p._version == q._version and p.grad._version == q.grad._version, i
    # growth_interval 2: growth after steps 0-1, backoff at 2, growth after 3-4
    assert scaler_f.get_scale() == 2048.0


def _native_max() -> int:
    from namitorch_amd import _native
    return _native.NT_MAX_COMBINE
