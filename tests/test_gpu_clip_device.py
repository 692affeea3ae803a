"""clip_grad_norm_ with the decision on the device (no host wait).

With nothing pending on the gradients and ``error_if_nonfinite`` False,
``clip_grad_norm_`` leaves the norm, the ``coefficient < 1`` decision
(optim/clip_grad.py:106-111) and the coefficient on the device, and the
AdamW pass that follows reads them there.  These tests check that the path
is taken and that everything the reference defines comes out as on the
host-synchronizing path and the oracle:

* the returned norm's bits and the clipped gradients (float32, float16,
  bfloat16), against ``error_if_nonfinite=True`` (which decides on the
  host) and ``oracle.clip``;
* version counters: one bump when the coefficient is below 1, none
  otherwise (also for a NaN norm, whose coefficient is NaN); an infinite
  norm gives coefficient 0, which clips (zeros, NaN where the gradient was
  infinite);
* several ``clip_grad_norm_`` -> ``step`` iterations against the same
  iterations on the host path: parameters, master weights, moments, step
  counts and versions bit-exact;
* a second clip on top of a pending device clip, and clips that no
  optimizer consumes (the unsettled list stays bounded).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd.optim import clip_grad
from namitorch_amd.tensor import _settle_device_steps, _unsettled_steps
from oracle import adam as oadam
from oracle import clip as oclip
from oracle import lowp

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NORM_RTOL = 1e-12
SHAPES = [(301, 17), (17,), (4099,), (0,), (2048,)]


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(f"u{a.itemsize}")


def _same(a, b) -> bool:
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype, (a.shape, b.shape, a.dtype, b.dtype)
    nan = np.isnan(a.astype(np.float64)) & np.isnan(b.astype(np.float64))
    return bool(np.all((_bits(a) == _bits(b)) | nan))


def _grads(seed, dtype, sigma=1e-2):
    rng = np.random.default_rng(seed)
    return [lowp.round_to(dtype, rng.standard_normal(s) * sigma) for s in SHAPES]


def _params(grads, dtype):
    params = [nt.Parameter(np.zeros(g.shape, np.float32), dtype=dtype, device=DEV) for g in grads]
    for p, g in zip(params, grads):
        p.grad = nt.Tensor(g, dtype=dtype, device=DEV)
    return params


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("ratio", [0.25, 4.0])
def test_device_clip_matches_host_path(dtype, ratio):
    grads = _grads(3, dtype)
    want = oclip.total_norm([g.astype(np.float64) for g in grads])
    max_norm = want * ratio
    device = _params(grads, dtype)
    host = _params(grads, dtype)
    before = [p.grad._version for p in device]
    norm_tensor = nt.optim.clip_grad_norm_(device, max_norm)
    assert all(p.grad._pending is not None and p.grad._pending.device is not None for p in device)
    assert norm_tensor.dtype is nt.float64 and norm_tensor.shape == () and norm_tensor.device.type == "cuda"
    host_norm = nt.optim.clip_grad_norm_(host, max_norm, error_if_nonfinite=True).item()
    norm = norm_tensor.item()
    assert _bits(np.float64(norm)) == _bits(np.float64(host_norm)), (norm, host_norm)
    assert abs(norm - want) <= NORM_RTOL * want
    coefficient = oclip.clip_coefficient(max_norm, norm)
    bump = 1 if coefficient < 1 else 0
    assert [p.grad._version for p in device] == [b + bump for b in before]
    assert [p.grad._version for p in host] == [b + bump for b in before]
    for p, q, g in zip(device, host, grads):
        got = p.grad.numpy()
        expected = oclip.clip_apply(g.astype(np.float64), coefficient, dtype) if bump else g
        assert _same(got, np.asarray(expected).astype(got.dtype)), dtype
        assert _same(got, q.grad.numpy())


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("bad", ["inf", "nan"])
def test_device_clip_nonfinite_norm(dtype, bad):
    grads = _grads(5, dtype)
    grads[2].reshape(-1)[11] = float(bad)
    params = _params(grads, dtype)
    before = [p.grad._version for p in params]
    norm = nt.optim.clip_grad_norm_(params, 1.0).item()
    if bad == "nan":
        assert math.isnan(norm)
        assert [p.grad._version for p in params] == before             # NaN coefficient: no clip
        for p, g in zip(params, grads):
            assert _same(p.grad.numpy(), g.astype(p.grad.numpy().dtype))
    else:
        assert norm == math.inf
        assert [p.grad._version for p in params] == [b + 1 for b in before]   # coefficient 0 clips
        for p, g in zip(params, grads):
            expected = oclip.clip_apply(g.astype(np.float64), 0.0, dtype)
            assert _same(p.grad.numpy(), np.asarray(expected).astype(p.grad.numpy().dtype))


@pytest.mark.parametrize("norm_type", [2.0, math.inf, 3.0])
def test_device_clip_norm_types(norm_type):
    """inf runs on the device too; other p stay on the host path (prescaled pass)."""
    grads = _grads(7, "float32")
    params = _params(grads, "float32")
    want = oclip.total_norm([g.astype(np.float64) for g in grads], norm_type)
    norm = nt.optim.clip_grad_norm_(params, want / 3, norm_type=norm_type)
    on_device = params[0].grad._pending is not None and params[0].grad._pending.device is not None
    assert on_device == (norm_type in (2.0, math.inf))
    assert abs(norm.item() - want) <= NORM_RTOL * want
    coefficient = oclip.clip_coefficient(want / 3, norm.item())
    for p, g in zip(params, grads):
        assert _same(p.grad.numpy(), oclip.clip_apply(g.astype(np.float64), coefficient, "float32"))


@pytest.mark.parametrize("layout", ["float32", "bf16-master"])
def test_clip_then_step_iterations_match_host_path(layout):
    """clip_grad_norm_ -> step, six iterations with fresh gradients, clipped
    on some iterations and not on others, against the same iterations with
    error_if_nonfinite=True (host decision) and against the oracle."""
    master = layout == "bf16-master"
    dtype = "bfloat16" if master else "float32"
    rng = np.random.default_rng(11)
    host_values = [lowp.round_to(dtype, rng.standard_normal(s) * 0.02) for s in SHAPES]

    def build():
        params = [nt.Parameter(h, dtype=dtype, device=DEV) for h in host_values]
        return params, nt.optim.AdamW(params, lr=1e-3, weight_decay=0.1, master_weights=master)

    dev_params, dev_opt = build()
    ref_params, ref_opt = build()
    values = [h.astype(np.float32).copy() for h in host_values]
    m = [np.zeros_like(v) for v in values]
    v2 = [np.zeros_like(v) for v in values]
    for k in range(6):
        grads = [lowp.round_to(dtype, rng.standard_normal(s) * 1e-2) for s in SHAPES]
        norm = oclip.total_norm([g.astype(np.float64) for g in grads])
        max_norm = norm * (0.5 if k % 2 == 0 else 2.0)
        for params in (dev_params, ref_params):
            for p, g in zip(params, grads):
                p.grad = nt.Tensor(g, dtype=dtype, device=DEV)
        got = nt.optim.clip_grad_norm_(dev_params, max_norm)
        dev_opt.step()
        ref = nt.optim.clip_grad_norm_(ref_params, max_norm, error_if_nonfinite=True)
        ref_opt.step()
        assert _bits(np.float64(got.item())) == _bits(np.float64(ref.item())), k
        coefficient = oclip.clip_coefficient(max_norm, ref.item())
        clipped = [oclip.clip_apply(g.astype(np.float64), coefficient, dtype) if coefficient < 1 else g for g in grads]
        for i, g in enumerate(clipped):
            kw = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
            if master:
                oadam.master_step(values[i], np.asarray(g, np.float32), m[i], v2[i], k + 1, **kw)
            else:
                oadam.adam_step(values[i], np.asarray(g, np.float32), m[i], v2[i], k + 1, **kw)
        assert [p.grad._version for p in dev_params] == [p.grad._version for p in ref_params], k
    for i, (p, q) in enumerate(zip(dev_params, ref_params)):
        sp, sq = dev_opt.state[id(p)], ref_opt.state[id(q)]
        assert sp["step"] == sq["step"] == 6
        assert _same(p.numpy(), q.numpy()), i
        want = lowp.round_to("bfloat16", values[i].astype(np.float64)) if master else values[i]
        assert _same(p.numpy(), np.asarray(want).astype(p.numpy().dtype)), i
        for name in ("exp_avg", "exp_avg_sq") + (("master",) if master else ()):
            assert _same(sp[name].numpy(), sq[name].numpy()), (i, name)
        assert _same(sp["exp_avg"].numpy(), m[i]) and _same(sp["exp_avg_sq"].numpy(), v2[i]), i
        assert (p._version, sp["exp_avg"]._version) == (q._version, sq["exp_avg"]._version), i


def test_second_clip_over_pending_device_clip():
    """The second call sees a device-decided transform: it writes it back and
    decides on the host, as two reference clips in a row."""
    grads = _grads(13, "float32")
    params = _params(grads, "float32")
    want = oclip.total_norm([g.astype(np.float64) for g in grads])
    first = nt.optim.clip_grad_norm_(params, want / 2).item()
    second = nt.optim.clip_grad_norm_(params, want / 8).item()
    c1 = oclip.clip_coefficient(want / 2, first)
    once = [oclip.clip_apply(g.astype(np.float64), c1, "float32") for g in grads]
    again = oclip.total_norm([g.astype(np.float64) for g in once])
    assert abs(second - again) <= NORM_RTOL * again
    c2 = oclip.clip_coefficient(want / 8, second)
    for p, g in zip(params, once):
        assert _same(p.grad.numpy(), oclip.clip_apply(g.astype(np.float64), c2, "float32"))


def test_unconsumed_device_clips_stay_bounded():
    """Clips that no optimizer step consumes are settled oldest first once
    the unsettled list is full; every gradient still reads as clipped."""
    grads = _grads(17, "float32")
    want = oclip.total_norm([g.astype(np.float64) for g in grads])
    params = _params(grads, "float32")
    _settle_device_steps()
    kept = []
    for k in range(clip_grad._UNSETTLED_LIMIT + 6):
        for p, g in zip(params, grads):
            p.grad = nt.Tensor(g, device=DEV)
        nt.optim.clip_grad_norm_(params, want / 2)
        kept.append([p.grad for p in params])
        assert len(_unsettled_steps) <= clip_grad._UNSETTLED_LIMIT, k
    coefficient = oclip.clip_coefficient(want / 2, want)
    for k in (0, len(kept) - 1):
        for gradient, g in zip(kept[k], grads):
            assert _same(gradient.numpy(), oclip.clip_apply(g.astype(np.float64), coefficient, "float32")), k
    _settle_device_steps()
    assert not _unsettled_steps


def test_clip_on_one_stream_step_on_another():
    """The control block is the only thing the library orders across
    streams: the pass on another stream waits for the clip's finalize before
    reading it.  Everything else is ordered by the test (uploads and both
    streams synchronized each iteration), and a long run of steps of another
    optimizer queued before the clip keeps its stream busy while the step is
    issued.  Results equal the same clip and step on one stream."""
    grads = _grads(19, "float32", sigma=1.0)
    want = oclip.total_norm([g.astype(np.float64) for g in grads])

    def run(two_streams):
        rng = np.random.default_rng(23)
        hosts = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES]
        first, second = nt.runtime.Stream(0), nt.runtime.Stream(0)
        with nt.runtime.stream(first):
            params = [nt.Parameter(h, device=DEV) for h in hosts]
            busy = nt.Parameter(np.zeros(1 << 24, np.float32), device=DEV)
            busy.grad = nt.Tensor(np.full(1 << 24, 1e-3, np.float32), device=DEV)
        optimizer = nt.optim.AdamW(params, lr=1e-3)
        filler = nt.optim.AdamW([busy], lr=1e-3)
        for k in range(3):
            with nt.runtime.stream(first):
                for p, g in zip(params, grads):
                    p.grad = nt.Tensor(g * np.float32(1 + k), device=DEV)
            first.synchronize()
            second.synchronize()
            with nt.runtime.stream(first):
                for _ in range(4):
                    filler.step()
                nt.optim.clip_grad_norm_(params, want / 4)
            with nt.runtime.stream(second if two_streams else first):
                optimizer.step()
            first.synchronize()
            second.synchronize()
        with nt.runtime.stream(second if two_streams else first):
            state = [optimizer.state[id(p)] for p in params]
            return [p.numpy() for p in params], [s["exp_avg"].numpy() for s in state]

    one_values, one_moments = run(False)
    two_values, two_moments = run(True)
    for a, b in zip(one_values + one_moments, two_values + two_moments):
        assert _same(a, b)


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("norm_type", [2.0, math.inf])
@pytest.mark.parametrize("bad", [None, "inf", "nan"])
def test_get_grad_norm_on_device(dtype, norm_type, bad):
    """get_grad_norm without a host wait: the norm's bits equal the host
    path's (an unclipping clip_grad_norm_ with error_if_nonfinite=True, or
    the reference's NaN/inf), nothing is recorded on the gradients, and a
    following clip_grad_norm_ gives the host path's result."""
    grads = _grads(29, dtype)
    if bad is not None:
        grads[0].reshape(-1)[3] = float(bad)
    params = _params(grads, dtype)
    versions = [p.grad._version for p in params]
    norm = nt.optim.get_grad_norm(params, norm_type=norm_type)
    assert norm.dtype is nt.float64 and norm.shape == () and norm.device.type == "cuda"
    assert all(p.grad._pending is None for p in params)
    assert [p.grad._version for p in params] == versions
    want = oclip.total_norm([g.astype(np.float64) for g in grads], norm_type)
    got = norm.item()
    if bad is None:
        host = _params(grads, dtype)
        host_norm = nt.optim.clip_grad_norm_(host, 1e300, norm_type=norm_type, error_if_nonfinite=True).item()
        assert _bits(np.float64(got)) == _bits(np.float64(host_norm)), (got, host_norm)
        assert abs(got - want) <= NORM_RTOL * want
        clipped = nt.optim.clip_grad_norm_(params, want / 3, norm_type=norm_type).item()
        assert _bits(np.float64(clipped)) == _bits(np.float64(got))
        coefficient = oclip.clip_coefficient(want / 3, got)
        for p, g in zip(params, grads):
            expected = np.asarray(oclip.clip_apply(g.astype(np.float64), coefficient, dtype))
            assert _same(p.grad.numpy(), expected.astype(p.grad.numpy().dtype))
    elif bad == "nan":
        assert math.isnan(got) and math.isnan(want)
    else:
        assert got == want == math.inf


@pytest.mark.parametrize("case", ["max_norm_zero", "all_zero", "all_empty"])
def test_device_clip_edge_cases(case):
    """max_norm 0 (coefficient 0: every gradient becomes a signed zero), all-zero
    gradients (norm 0: coefficient 1e6, no clip) and gradients that are all
    empty (norm 0 over no elements): norm bits, gradients and versions as on
    the host path and the oracle."""
    if case == "all_empty":
        grads = [np.zeros((0,), np.float32), np.zeros((0,), np.float32)]
    elif case == "all_zero":
        grads = [np.zeros(s, np.float32) for s in SHAPES]
    else:
        grads = _grads(31, "float32")
    max_norm = 0.0 if case == "max_norm_zero" else 1.0
    device = _params(grads, "float32")
    host = _params(grads, "float32")
    before = [p.grad._version for p in device]
    got = nt.optim.clip_grad_norm_(device, max_norm)
    assert all(p.grad._pending is not None and p.grad._pending.device is not None for p in device)
    want = oclip.total_norm([g.astype(np.float64) for g in grads])
    host_norm = nt.optim.clip_grad_norm_(host, max_norm, error_if_nonfinite=True).item()
    assert _bits(np.float64(got.item())) == _bits(np.float64(host_norm)) and abs(got.item() - want) <= NORM_RTOL * want
    coefficient = oclip.clip_coefficient(max_norm, got.item())
    bump = 1 if coefficient < 1 else 0
    assert [p.grad._version for p in device] == [b + bump for b in before] == [p.grad._version for p in host]
    for p, q, g in zip(device, host, grads):
        expected = oclip.clip_apply(g.astype(np.float64), coefficient, "float32") if bump else g
        assert _same(p.grad.numpy(), expected) and _same(p.grad.numpy(), q.grad.numpy())


def test_device_clip_then_unscale_then_step():
    """A device-decided clip followed by GradScaler.unscale_ (clipping the
    scaled gradients, an unusual but legal order): unscale_ writes the clip
    back first, so the step uses unscale(clip(g)) as the reference computes
    it, bit for bit against the oracle."""
    from oracle import scaler as oscaler
    rng = np.random.default_rng(37)
    hosts = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in SHAPES]
    params = [nt.Parameter(h, device=DEV) for h in hosts]
    optimizer = nt.optim.AdamW(params, lr=1e-3, weight_decay=0.1)
    scaler = nt.GradScaler(init_scale=1024.0)
    grads = [(rng.standard_normal(s) * 1e-3 * 1024).astype(np.float32) for s in SHAPES]
    for p, g in zip(params, grads):
        p.grad = nt.Tensor(g, device=DEV)
    scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
    want_norm = oclip.total_norm([g.astype(np.float64) for g in grads])
    norm = nt.optim.clip_grad_norm_(params, want_norm / 2)
    assert params[0].grad._pending is not None and params[0].grad._pending.device is not None
    assert scaler.unscale_(optimizer) is True
    assert scaler.step(optimizer) is True
    scaler.update()
    coefficient = oclip.clip_coefficient(want_norm / 2, norm.item())
    for p, h, g in zip(params, hosts, grads):
        clipped = oclip.clip_apply(g.astype(np.float64), coefficient, "float32")
        unscaled = oscaler.unscale(clipped, 1024.0, "float32")
        value, m, v = h.copy(), np.zeros_like(h), np.zeros_like(h)
        oadam.adam_step(value, np.asarray(unscaled, np.float32), m, v, 1, lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
                        weight_decay=0.1)
        assert _same(p.numpy(), value)


@pytest.mark.parametrize("consumer", ["step", "version read"])
def test_cached_norm_after_an_undone_clip_bump(consumer):
    """A device clip that decides not to clip bumps the gradients' versions
    before the decision is known; settling the step lowers them again.  Norm
    statistics cached in between (get_grad_norm over the pending transform
    takes the host path and caches them under the bumped version) must not
    answer for the values written after the settle, whose version equals the
    bumped one again."""
    grads = _grads(23, "float32")
    params = _params(grads, "float32")
    optimizer = nt.optim.AdamW(params, lr=1e-3)
    before = [p.grad._version for p in params]
    want = oclip.total_norm([g.astype(np.float64) for g in grads])
    nt.optim.clip_grad_norm_(params, want * 4)                  # coefficient > 1: no clip, decided on the device
    assert params[0].grad._pending is not None and params[0].grad._pending.device is not None
    cached = nt.optim.get_grad_norm(params).item()              # host path over the pending transform
    assert abs(cached - want) <= NORM_RTOL * want
    if consumer == "step":
        optimizer.step()
        optimizer.state[id(params[0])]["exp_avg"].numpy()
    assert [p.grad._version for p in params] == before          # settled: the bump is undone
    fresh = _grads(29, "float32", sigma=3e-2)
    with nt.no_grad():
        for p, g in zip(params, fresh):
            p.grad.copy_(nt.Tensor(g, device=DEV))
    assert [p.grad._version for p in params] == [b + 1 for b in before]
    want_fresh = oclip.total_norm([g.astype(np.float64) for g in fresh])
    assert abs(want_fresh - want) > 0.5 * want                  # a stale norm would be detected
    got = nt.optim.get_grad_norm(params).item()
    assert abs(got - want_fresh) <= NORM_RTOL * want_fresh, (got, want_fresh, cached)
    host = nt.optim.clip_grad_norm_(params, want_fresh / 2, error_if_nonfinite=True).item()
    assert abs(host - want_fresh) <= NORM_RTOL * want_fresh, (host, want_fresh)
    coefficient = oclip.clip_coefficient(want_fresh / 2, host)
    for p, g in zip(params, fresh):
        assert _same(p.grad.numpy(), oclip.clip_apply(g.astype(np.float64), coefficient, "float32"))


@pytest.mark.parametrize("write", ["copy_", "zero_", "accumulate", "clip"])
def test_versions_when_a_write_lands_before_the_clip_settles(write):
    """A device clip that decides not to clip, followed, before anything
    settles it, by one more write of the gradients: the versions count that
    one write only, as the reference's do (a clip with coefficient >= 1 does
    not write, optim/clip_grad.py:108-111; every other write is one
    copy_, tensor.py:1283-1287)."""
    from namitorch_amd.grads import accumulate_grads
    grads = _grads(31, "float32")
    params = _params(grads, "float32")
    before = [p.grad._version_counter.value for p in params]
    want = oclip.total_norm([g.astype(np.float64) for g in grads])
    nt.optim.clip_grad_norm_(params, want * 4)                  # no clip, decided on the device
    assert params[0].grad._pending is not None and params[0].grad._pending.device is not None
    fresh = _grads(37, "float32")
    if write == "copy_":
        with nt.no_grad():
            for p, g in zip(params, fresh):
                p.grad.copy_(nt.Tensor(g, device=DEV))
        expected = fresh
    elif write == "zero_":
        for p in params:
            p.grad.zero_()
        expected = [np.zeros_like(g) for g in grads]
    elif write == "accumulate":
        accumulate_grads(params, [nt.Tensor(g, device=DEV) for g in fresh])
        expected = [np.float32(a) + np.float32(b) for a, b in zip(grads, fresh)]
    else:
        # a second clip that clips: over the pending device transform it
        # decides on the host (one write)
        nt.optim.clip_grad_norm_(params, want / 2)
        coefficient = oclip.clip_coefficient(want / 2, want)
        expected = [oclip.clip_apply(g.astype(np.float64), coefficient, "float32") for g in grads]
    assert [p.grad._version for p in params] == [b + 1 for b in before], write
    for p, g in zip(params, expected):
        got = p.grad.numpy()
        if write == "clip":
            # the norm itself is the oracle's within NORM_RTOL, so the coefficient may differ in its last bits
            assert np.allclose(got, np.asarray(g, np.float32), rtol=1e-6, atol=0), write
        else:
            assert _same(got, np.asarray(g, np.float32)), write


def test_host_known_norm_reads_without_a_device_round_trip(monkeypatch):
    """After unscale_ the norm is known on the host: clip_grad_norm_'s
    returned device scalar hands it to .item() without reading the device,
    with the bits the device holds; once written in place, .item() reads the
    device again."""
    rng = np.random.default_rng(91)
    params = [nt.Parameter((rng.standard_normal(s) * 0.02).astype(np.float32), device=DEV) for s in SHAPES]
    for p in params:
        p.grad = nt.Tensor((rng.standard_normal(p.shape) * 64.0).astype(np.float32), device=DEV)
    optimizer = nt.optim.AdamW(params)
    scaler = nt.GradScaler(init_scale=1024.0)
    scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
    assert scaler.unscale_(optimizer)
    norm = nt.optim.clip_grad_norm_(params, 0.5, error_if_nonfinite=True)
    reads = []
    original = nt.Tensor.numpy

    def counted(self):
        reads.append(self)
        return original(self)
    monkeypatch.setattr(nt.Tensor, "numpy", counted)
    value = norm.item()
    assert reads == []
    assert isinstance(value, float)
    assert np.float64(value).view(np.uint64) == original(norm).view(np.uint64)   # what the device holds
    norm.copy_(nt.Tensor(np.float64(3.25), device=DEV))
    assert norm.item() == 3.25 and len(reads) == 1
    scaler.step(optimizer)
    scaler.update()
