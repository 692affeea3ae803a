"""Seeded random AMP training sequences against the oracle.

Each run mixes, step by step, ``amp.fused_step``, the reference's call
sequence (``unscale_`` -> ``clip_grad_norm_`` if finite -> ``step`` ->
``update``, training/runner.py:240-254) and, without a clip, ``step`` ->
``update`` alone (``step`` unscales by itself) on one optimizer and one
GradScaler, with a warmup-cosine schedule that advances only after steps
that updated (runner.py:250-253; ``fused_step(..., scheduler=)`` on the
fused steps).  Along the way it injects inf/NaN gradients, changes the clip
threshold, reads step counts and the loss scale right after fused steps
(which must already show a skipped step as skipped), and round-trips the
optimizer's and the scaler's state dicts, or resumes from a checkpoint
archive into new parameters, optimizer, scaler and schedule.

The oracle composes ``scaler.unscale`` -> ``clip.clip_grad_norm`` ->
``adam.master_step`` / ``adam.adam_step`` with ``scaler.Scaler`` and the
schedule's rates (the schedule itself is pinned against the reference's
golden rates in the scheduler tests).  Bars: finite/updated flags, the scale
after every step, step counts and learning rates exact; parameters, master
weights and moments bit-exact (clipped float32/bfloat16 gradients may move
by one unit on a clip coefficient one ulp away, expected well below once
per run, so at most two elements per array may differ by one unit).
"""

from __future__ import annotations

import contextlib

import numpy as np
import pytest

import namitorch_amd as nt
from oracle import adam as oadam
from oracle import clip as oclip
from oracle import lowp
from oracle import scaler as oscaler

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
CASES = 32
STEPS = 8
SIZES = (255, 256, 2047, 2049, 4096, 12289)


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32 if a.itemsize == 4 else np.uint16)


def _close(label, got, want, loose):
    g, w = _bits(got).reshape(-1), _bits(want).reshape(-1)
    bad = np.flatnonzero(g != w)
    if bad.size == 0:
        return
    unit = 1 << 16 if label.endswith("bf16") else 1
    distance = np.abs(g[bad].astype(np.int64) - w[bad].astype(np.int64))
    assert loose and bad.size <= 2 and np.all(distance <= unit), f"{label}: {bad.size} elements differ"


@pytest.mark.parametrize("seed", range(CASES))
def test_random_amp_sequence(seed, tmp_path):
    rng = np.random.default_rng(9000 + seed)
    master = bool(rng.random() < 0.6)
    dtype = "bfloat16" if master else "float32"
    gdtype = str(rng.choice(["bfloat16", "float16"])) if master else "float32"
    shapes = [(int(rng.choice(SIZES)),) for _ in range(int(rng.integers(1, 4)))]
    hosts = [rng.standard_normal(s) * 0.02 for s in shapes]
    hosts = [lowp.round_to("bfloat16", h) if master else h.astype(np.float32) for h in hosts]
    params = [nt.Parameter(h, dtype=dtype, device=DEV) for h in hosts]
    optimizer = nt.optim.AdamW(params, lr=1e-3, weight_decay=0.05, master_weights=master)
    scale0 = float(rng.choice([65536.0, 1024.0, 8.0]))
    interval = int(rng.choice([1, 2, 3]))
    scaler = nt.GradScaler(init_scale=scale0, growth_interval=interval)
    scheduler = nt.optim.WarmupCosine(optimizer, warmup_steps=2, total_steps=STEPS + 2, min_lr=1e-5)
    # Oracle: the schedule's rates from a host-only copy of the same schedule.
    rates_owner = nt.optim.AdamW([nt.Parameter(np.zeros(1, np.float32))], lr=1e-3)
    rates = nt.optim.WarmupCosine(rates_owner, warmup_steps=2, total_steps=STEPS + 2, min_lr=1e-5)
    values = [h.astype(np.float32).copy() for h in hosts]
    m = [np.zeros_like(v) for v in values]
    v2 = [np.zeros_like(v) for v in values]
    oscale = oscaler.Scaler(scale0, 2.0, 0.5, interval)
    count, loose = 0, False
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    log = []
    for step in range(STEPS):
        path = str(rng.choice(["api", "fused"]))
        max_norm = None if rng.random() < 0.4 else float(rng.choice([1e-3, 0.05, 10.0]))
        if path == "api" and max_norm is None and step % 2 == 0:
            path = "step"                                   # step() unscales by itself: nothing to clip between
        grads = [rng.standard_normal(s) * 1e-3 for s in shapes]
        stored = []
        for g in grads:
            scaled = g * oscale.scale
            stored.append(lowp.round_to(gdtype, scaled) if gdtype != "float32" else scaled.astype(np.float32))
        if rng.random() < 0.25:
            k = int(rng.integers(len(shapes)))
            stored[k].reshape(-1)[int(rng.integers(stored[k].size))] = float(rng.choice([np.inf, np.nan]))
        # Oracle.
        unscaled = [oscaler.unscale(s, oscale.scale, gdtype) for s in stored]
        finite = oscaler.finite(unscaled)
        lr = rates_owner.param_groups[0]["lr"]
        if finite:
            if max_norm is not None:
                norm, unscaled = oclip.clip_grad_norm(unscaled, max_norm, 2.0, gdtype)
                loose |= oclip.clip_coefficient(max_norm, norm) < 1
            count += 1
            for i, g in enumerate(unscaled):
                kw = dict(lr=lr, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.05)
                if master:
                    oadam.master_step(values[i], np.asarray(g, np.float32), m[i], v2[i], count, **kw)
                else:
                    oadam.adam_step(values[i], g, m[i], v2[i], count, **kw)
            rates.step()
        oscale.update(not finite)
        # Device.
        scaler.scale(loss)
        for p, s in zip(params, stored):
            p.grad = nt.Tensor(s, dtype=gdtype, device=DEV)
        if path == "step":
            updated = got_finite = scaler.step(optimizer)
            scaler.update()
            if updated:
                scheduler.step()
        elif path == "api":
            got_finite = scaler.unscale_(optimizer)
            if got_finite and max_norm is not None:
                nt.optim.clip_grad_norm_(params, max_norm)
            updated = scaler.step(optimizer)
            scaler.update()
            if updated:
                scheduler.step()
        else:
            result = nt.amp.fused_step(optimizer, scaler, max_norm=max_norm, scheduler=scheduler)
            if rng.random() < 0.5:                          # read the outcome right away, or never
                got_finite, updated = result.finite, result.updated
            else:
                got_finite = updated = finite
        assert got_finite == finite and updated == finite, (step, path)
        if rng.random() < 0.5:                              # reads settle a device-decided step
            assert optimizer.state[id(params[0])].get("step", 0) == count, (step, path)
            assert scaler.get_scale() == oscale.scale, (step, path, scaler.get_scale(), oscale.scale)
            assert scheduler.get_last_lr()[0] == rates_owner.param_groups[0]["lr"], (step, path)
        if rng.random() < 0.15:
            optimizer.load_state_dict(optimizer.state_dict())
            scaler.load_state_dict(scaler.state_dict())
            log.append("reload")
        if rng.random() < 0.12:
            # Resume from a checkpoint archive into new parameters, optimizer,
            # scaler and schedule (training/checkpoint.py:59-174).
            path = str(tmp_path / f"step{step}.nt")
            nt.save_checkpoint(path, {f"p{i}": p for i, p in enumerate(params)}, optimizer, scheduler,
                               scaler=scaler, step=step + 1)
            params = [nt.Parameter(np.zeros(s, np.float32), dtype=dtype, device=DEV) for s in shapes]
            optimizer = nt.optim.AdamW(params, lr=1e-3, weight_decay=0.05, master_weights=master)
            scaler = nt.GradScaler(init_scale=1.0)
            scheduler = nt.optim.WarmupCosine(optimizer, warmup_steps=2, total_steps=STEPS + 2, min_lr=1e-5)
            nt.load_checkpoint(path, {f"p{i}": p for i, p in enumerate(params)}, optimizer, scheduler, scaler=scaler)
            log.append("checkpoint")
        log.append(f"{path}{'' if finite else '!'}{'' if max_norm is None else 'c'}")
    print(f"case {seed}: master={master} g={gdtype} shapes={shapes} scale0={scale0} interval={interval} {log}",
          flush=True)
    assert scaler.get_scale() == oscale.scale
    for i, p in enumerate(params):
        state = optimizer.state.get(id(p), {})
        assert state.get("step", 0) == count, i
        if count == 0:
            continue
        if master:
            _close(f"master[{i}]", state["master"].numpy(), values[i], loose)
            _close(f"param[{i}] bf16", p.numpy(), lowp.round_to("bfloat16", values[i].astype(np.float64)), loose)
        else:
            _close(f"param[{i}]", p.numpy(), values[i], loose)
        _close(f"m[{i}]", state["exp_avg"].numpy(), m[i], loose)
        _close(f"v[{i}]", state["exp_avg_sq"].numpy(), v2[i], loose)
    assert scheduler.get_last_lr()[0] == rates_owner.param_groups[0]["lr"]
    assert optimizer.param_groups[0]["lr"] == rates_owner.param_groups[0]["lr"]


CLIP_CASES = 24


@pytest.mark.parametrize("seed", range(CLIP_CASES))
def test_random_clip_sequence_without_scaler(seed, tmp_path):
    """Seeded runs without a GradScaler, mixing per step ``clip_grad_norm_``
    -> ``step`` (the clip decided on the device when nothing is pending),
    ``fused_step(optimizer, None, max_norm=...)`` and plain steps.  Along the
    way they read ``get_grad_norm``, step on a second library stream, and
    round-trip state dicts or resume from a checkpoint archive into new
    objects.  Oracle: ``clip.clip_grad_norm`` -> ``adam.master_step`` /
    ``adam.adam_step``.  Bars as above; the returned norms within 1e-12 of
    the oracle's."""
    rng = np.random.default_rng(9500 + seed)
    master = bool(rng.random() < 0.5)
    dtype = "bfloat16" if master else "float32"
    gdtype = str(rng.choice(["bfloat16", "float16"])) if master else "float32"
    shapes = [(int(rng.choice(SIZES)),) for _ in range(int(rng.integers(1, 4)))]
    hosts = [rng.standard_normal(s) * 0.02 for s in shapes]
    hosts = [lowp.round_to("bfloat16", h) if master else h.astype(np.float32) for h in hosts]
    params = [nt.Parameter(h, dtype=dtype, device=DEV) for h in hosts]
    optimizer = nt.optim.AdamW(params, lr=1e-3, weight_decay=0.05, master_weights=master)
    values = [h.astype(np.float32).copy() for h in hosts]
    m = [np.zeros_like(v) for v in values]
    v2 = [np.zeros_like(v) for v in values]
    side = nt.runtime.Stream(0)
    count, loose, log = 0, False, []
    for step in range(STEPS):
        path = str(rng.choice(["api", "fused", "plain"]))
        max_norm = None if path == "plain" else float(rng.choice([1e-3, 0.02, 10.0]))
        grads = [rng.standard_normal(s) * 1e-3 for s in shapes]
        stored = [lowp.round_to(gdtype, g) if gdtype != "float32" else g.astype(np.float32) for g in grads]
        # Oracle.
        used = [np.asarray(s, np.float64) for s in stored]
        want_norm = oclip.total_norm(used)
        if max_norm is not None:
            norm, used = oclip.clip_grad_norm(used, max_norm, 2.0, gdtype)
            loose |= oclip.clip_coefficient(max_norm, norm) < 1
        count += 1
        for i, g in enumerate(used):
            kw = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.05)
            if master:
                oadam.master_step(values[i], np.asarray(g, np.float32), m[i], v2[i], count, **kw)
            else:
                oadam.adam_step(values[i], np.asarray(g, np.float32), m[i], v2[i], count, **kw)
        # Device.
        on_side = rng.random() < 0.2
        if on_side:
            # The caller orders its own streams: the side stream starts after the default stream's work.
            side.wait_stream(nt.runtime.Stream.wrap(nt.runtime.current_stream(0)))
        with (nt.runtime.stream(side) if on_side else contextlib.nullcontext()):
            for p, s in zip(params, stored):
                p.grad = nt.Tensor(s, dtype=gdtype, device=DEV)
            if rng.random() < 0.3:
                got = nt.optim.get_grad_norm(params).item()
                assert abs(got - want_norm) <= 1e-12 * want_norm, (step, got, want_norm)
            if path == "api":
                got = nt.optim.clip_grad_norm_(params, max_norm)
                optimizer.step()
                if rng.random() < 0.5:
                    assert abs(got.item() - want_norm) <= 1e-12 * want_norm, (step, got.item(), want_norm)
            elif path == "fused":
                result = nt.amp.fused_step(optimizer, None, max_norm=max_norm)
                if rng.random() < 0.5:
                    assert abs(result.norm - want_norm) <= 1e-12 * want_norm, (step, result.norm, want_norm)
            else:
                optimizer.step()
        if on_side:
            side.synchronize()
        if rng.random() < 0.5:
            assert optimizer.state[id(params[0])].get("step", 0) == count, (step, path)
        if rng.random() < 0.15:
            optimizer.load_state_dict(optimizer.state_dict())
            log.append("reload")
        if rng.random() < 0.12:
            archive = str(tmp_path / f"step{step}.nt")
            nt.save_checkpoint(archive, {f"p{i}": p for i, p in enumerate(params)}, optimizer, None, step=step + 1)
            params = [nt.Parameter(np.zeros(s, np.float32), dtype=dtype, device=DEV) for s in shapes]
            optimizer = nt.optim.AdamW(params, lr=1e-3, weight_decay=0.05, master_weights=master)
            nt.load_checkpoint(archive, {f"p{i}": p for i, p in enumerate(params)}, optimizer, None)
            log.append("checkpoint")
        log.append(f"{path}{'s' if on_side else ''}{'' if max_norm is None else 'c'}")
    print(f"case {seed}: master={master} g={gdtype} shapes={shapes} {log}", flush=True)
    for i, p in enumerate(params):
        state = optimizer.state[id(p)]
        assert state["step"] == count, i
        if master:
            _close(f"master[{i}]", state["master"].numpy(), values[i], loose)
            _close(f"param[{i}] bf16", p.numpy(), lowp.round_to("bfloat16", values[i].astype(np.float64)), loose)
        else:
            _close(f"param[{i}]", p.numpy(), values[i], loose)
        _close(f"m[{i}]", state["exp_avg"].numpy(), m[i], loose)
        _close(f"v[{i}]", state["exp_avg_sq"].numpy(), v2[i], loose)
