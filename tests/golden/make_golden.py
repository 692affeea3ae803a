"""Write golden fixtures from the reference's own NumPy-backend code.

Run in the build container only (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py /root/reference

It imports ``namitorch`` from the given reference checkout, runs small,
seeded cases of the optimizer-step path on the CPU (NumPy) backend and
stores inputs and outputs as ``tests/golden/*.npz`` plus
``tests/golden/golden.json`` (scalar sequences and exception texts).  The
fixtures are data; nothing of the reference is copied.  These pin the
oracle where closed forms cannot: the bit-level operation order of
Adam/AdamW through ``Tensor.copy_``, the float16 array path, the
GradScaler sequence and clip_grad_norm_'s rounding.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SEED = 1337
STEPS = 10


def _grads(n, steps, sigma, dtype, seed_base=SEED + 1000):
    return [(np.random.Generator(np.random.PCG64(seed_base + k)).standard_normal(n, dtype=np.float32) * np.float32(sigma)).astype(dtype)
            for k in range(steps)]


def _params(n, dtype, seed=SEED, sigma=0.02):
    return (np.random.Generator(np.random.PCG64(seed)).standard_normal(n, dtype=np.float32) * np.float32(sigma)).astype(dtype)


def run_adam(nt, cls, p0, grads, **options):
    param = nt.nn.Parameter(p0.copy())
    optimizer = cls([param], **options)
    for grad in grads:
        param._grad = nt.Tensor(grad.copy())
        optimizer.step()
    state = optimizer.state[id(param)]
    return (param._data.copy(), state["exp_avg"]._data.copy(), state["exp_avg_sq"]._data.copy(), state["step"])


def adam_cases(nt):
    cases = {}
    n = 4099
    p0 = _params(n, np.float32)
    grads = _grads(n, STEPS, 1e-3, np.float32)
    base = dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
    variants = {
        "adamw_f32": (nt.optim.AdamW, base),
        "adamw_f32_maximize": (nt.optim.AdamW, dict(base, maximize=True)),
        "adamw_f32_lr0": (nt.optim.AdamW, dict(base, lr=0.0)),
        "adamw_f32_wd0": (nt.optim.AdamW, dict(base, weight_decay=0.0)),
        "adamw_f32_defaults": (nt.optim.AdamW, {}),
        "adam_f32_coupled": (nt.optim.Adam, base),
    }
    for name, (cls, options) in variants.items():
        p, m, v, step = run_adam(nt, cls, p0, grads, **options)
        cases[name] = dict(p0=p0, grads=np.stack(grads), p=p, m=m, v=v, step=np.int64(step),
                           options=json.dumps({k: list(v) if isinstance(v, tuple) else v for k, v in options.items()}))
    # bfloat16-valued float32 gradients: pins the master-weight extension.
    bf = [(g.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32) for g in grads]
    p, m, v, step = run_adam(nt, nt.optim.AdamW, p0, bf, **base)
    cases["adamw_f32_bfgrads"] = dict(p0=p0, grads=np.stack(bf), p=p, m=m, v=v, step=np.int64(step),
                                      options=json.dumps({k: list(v) if isinstance(v, tuple) else v for k, v in base.items()}))
    # Special values: zeros, subnormals, huge, inf and NaN gradients.
    m0 = 64
    sp = _params(m0, np.float32, seed=7)
    g = _grads(m0, 3, 1e-3, np.float32, seed_base=77)
    g[0][:8] = [0.0, -0.0, 1e-40, -1e-42, 3e38, -3e38, np.float32(1e-45), 5e-39]
    g[1][8:12] = [np.inf, -np.inf, np.nan, 0.0]
    p, m, v, step = run_adam(nt, nt.optim.AdamW, sp, g, **base)
    cases["adamw_f32_special"] = dict(p0=sp, grads=np.stack(g), p=p, m=m, v=v, step=np.int64(step),
                                      options=json.dumps({k: list(v) if isinstance(v, tuple) else v for k, v in base.items()}))
    # float16 parameters: the NumPy float16 array path.
    h0 = _params(1000, np.float16, seed=11, sigma=0.5)
    hg = _grads(1000, STEPS, 1e-2, np.float16, seed_base=111)
    hopt = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-4, weight_decay=0.1)
    p, m, v, step = run_adam(nt, nt.optim.AdamW, h0, hg, **hopt)
    cases["adamw_f16"] = dict(p0=h0, grads=np.stack(hg), p=p, m=m, v=v, step=np.int64(step),
                              options=json.dumps({k: list(v) if isinstance(v, tuple) else v for k, v in hopt.items()}))
    # float64 parameters.
    d0 = _params(513, np.float64, seed=13)
    dg = _grads(513, 4, 1e-3, np.float64, seed_base=131)
    p, m, v, step = run_adam(nt, nt.optim.AdamW, d0, dg, **base)
    cases["adamw_f64"] = dict(p0=d0, grads=np.stack(dg), p=p, m=m, v=v, step=np.int64(step),
                              options=json.dumps({k: list(v) if isinstance(v, tuple) else v for k, v in base.items()}))
    for name, arrays in cases.items():
        np.savez(HERE / f"{name}.npz", **arrays)
    return sorted(cases)


def clip_cases(nt):
    rng = np.random.Generator(np.random.PCG64(21))
    shapes = [(37,), (8, 16), (1000,), (3, 5, 7)]
    out = {}
    records = []
    for dtype in (np.float32, np.float16):
        for norm_type in (2.0, 1.0, 3.0, float("inf"), 0.5):
            for max_norm, sigma in ((1.0, 0.5), (1e6, 0.5)):
                grads = [(rng.standard_normal(s) * sigma).astype(dtype) for s in shapes]
                params = [nt.nn.Parameter(np.zeros(s, dtype=dtype)) for s in shapes]
                for param, grad in zip(params, grads):
                    param._grad = nt.Tensor(grad.copy())
                norm = nt.optim.clip_grad_norm_(params, max_norm, norm_type=norm_type)
                key = f"clip_{np.dtype(dtype).name}_{norm_type}_{max_norm:g}"
                for index, (grad, param) in enumerate(zip(grads, params)):
                    out[f"{key}_in{index}"] = grad
                    out[f"{key}_out{index}"] = param.grad._data.copy()
                records.append(dict(key=key, dtype=np.dtype(dtype).name, norm_type=norm_type, max_norm=max_norm,
                                    norm=float(norm._data), count=len(shapes)))
    # Non-finite gradients (no error requested): inf -> coefficient 0 -> NaN/0 grads.
    for label, poison in (("inf", np.inf), ("nan", np.nan)):
        grads = [(rng.standard_normal(s) * 0.5).astype(np.float32) for s in shapes]
        grads[2][5] = poison
        params = [nt.nn.Parameter(np.zeros(s, dtype=np.float32)) for s in shapes]
        for param, grad in zip(params, grads):
            param._grad = nt.Tensor(grad.copy())
        norm = nt.optim.clip_grad_norm_(params, 1.0)
        key = f"clip_nonfinite_{label}"
        for index, (grad, param) in enumerate(zip(grads, params)):
            out[f"{key}_in{index}"] = grad
            out[f"{key}_out{index}"] = param.grad._data.copy()
        records.append(dict(key=key, dtype="float32", norm_type=2.0, max_norm=1.0, norm=float(norm._data), count=len(shapes)))
    # All-zero gradients.
    params = [nt.nn.Parameter(np.zeros(s, dtype=np.float32)) for s in shapes]
    for param in params:
        param._grad = nt.Tensor(np.zeros(param.shape, dtype=np.float32))
    records.append(dict(key="clip_zero", dtype="float32", norm_type=2.0, max_norm=1.0,
                        norm=float(nt.optim.clip_grad_norm_(params, 1.0)._data), count=0))
    np.savez(HERE / "clip.npz", **out)
    return records


def scaler_cases(nt):
    """The runner's AMP sequence (training/runner.py:234-254) on float32 and
    float16 parameters, with an inf at step 4 and a NaN at step 7."""
    results = {}
    arrays = {}
    for dtype, eps, sigma in ((np.float32, 1e-8, 1e-3), (np.float16, 1e-4, 1e-3)):
        n = 777
        p0 = _params(n, dtype, seed=31, sigma=0.5 if dtype == np.float16 else 0.02)
        raw = _grads(n, STEPS, sigma, np.float32, seed_base=3100)
        param = nt.nn.Parameter(p0.copy())
        optimizer = nt.optim.AdamW([param], lr=1e-3, betas=(0.9, 0.999), eps=eps, weight_decay=0.1)
        scaler = nt.amp.GradScaler(init_scale=65536.0, growth_interval=3)
        finite_seq, updated_seq, scale_seq, norm_seq = [], [], [], []
        grads_in = []
        for k in range(STEPS):
            loss = nt.Tensor(np.float32(1.0))
            scaler.scale(loss)
            scaled = (raw[k].astype(np.float64) * scaler.get_scale()).astype(dtype)
            if k == 4:
                scaled[10] = np.inf
            if k == 7:
                scaled[20] = np.nan
            grads_in.append(scaled.copy())
            param._grad = nt.Tensor(scaled)
            finite = scaler.unscale_(optimizer)
            norm = nt.optim.clip_grad_norm_([param], 1.0, error_if_nonfinite=True).item() if finite else None
            updated = scaler.step(optimizer)
            scaler.update()
            finite_seq.append(bool(finite))
            updated_seq.append(bool(updated))
            scale_seq.append(scaler.get_scale())
            norm_seq.append(norm)
        name = f"scaler_{np.dtype(dtype).name}"
        arrays[f"{name}_p0"] = p0
        arrays[f"{name}_grads"] = np.stack(grads_in)
        arrays[f"{name}_p"] = param._data.copy()
        state = optimizer.state[id(param)]
        arrays[f"{name}_m"] = state["exp_avg"]._data.copy()
        arrays[f"{name}_v"] = state["exp_avg_sq"]._data.copy()
        results[name] = dict(finite=finite_seq, updated=updated_seq, scale=scale_seq, norm=norm_seq,
                             step=state["step"], eps=eps)
    # Scale sequence under repeated overflow and growth (no optimizer arithmetic involved).
    param = nt.nn.Parameter(np.zeros(4, dtype=np.float32))
    optimizer = nt.optim.AdamW([param], lr=0.0)
    scaler = nt.amp.GradScaler(init_scale=2.0 ** 120, growth_factor=4.0, backoff_factor=0.25, growth_interval=2)
    pattern = [False, False, False, False, True, False, False, True, True, False, False, False]
    sequence = []
    for overflow in pattern:
        scaler.scale(nt.Tensor(np.float32(1.0)))
        grad = np.ones(4, dtype=np.float32)
        if overflow:
            grad[0] = np.inf
        param._grad = nt.Tensor(grad)
        scaler.step(optimizer)
        scaler.update()
        sequence.append(scaler.get_scale())
    results["scale_sequence"] = dict(pattern=pattern, scale=sequence, init=2.0 ** 120, growth=4.0, backoff=0.25, interval=2)
    np.savez(HERE / "scaler.npz", **arrays)
    return results


def checkpoint_case(nt):
    """A training checkpoint written by the reference's own save_checkpoint
    (training/checkpoint.py:80-110) after 3 AMP steps of the runner sequence on
    a two-group AdamW, plus the parameters/moments/scaler after 2 more steps.
    A resumed optimizer must continue bit for bit."""
    from namitorch.training.checkpoint import save_checkpoint

    class Tiny(nt.nn.Module):
        def __init__(self):
            super().__init__()
            self.weight = nt.nn.Parameter(_params(40 * 48, np.float32, seed=41).reshape(40, 48))
            self.bias = nt.nn.Parameter(_params(40, np.float32, seed=42))

    model = Tiny()
    params = [model.weight, model.bias]
    optimizer = nt.optim.AdamW([{"params": [model.weight], "weight_decay": 0.1},
                                {"params": [model.bias], "weight_decay": 0.0}],
                               lr=1e-3, betas=(0.9, 0.95), eps=1e-8)
    scaler = nt.amp.GradScaler(init_scale=1024.0, growth_interval=2)
    raw = [_grads(p.size, 5, 1e-3, np.float32, seed_base=4100 + 10 * i) for i, p in enumerate(params)]
    arrays = {}
    finite_seq = []
    for k in range(5):
        if k == 3:
            save_checkpoint(HERE / "checkpoint_reference.nt", model, optimizer, step=3, epoch=0,
                            config={"case": "amp-adamw"}, cumulative_tokens=0, scaler=scaler)
        scaler.scale(nt.Tensor(np.float32(1.0)))
        for i, p in enumerate(params):
            g = (raw[i][k].astype(np.float64) * scaler.get_scale()).astype(np.float32).reshape(p.shape)
            if k == 1 and i == 1:
                g[3] = np.inf
            arrays[f"grad{i}_{k}"] = g.copy()
            p._grad = nt.Tensor(g)
        finite = scaler.unscale_(optimizer)
        if finite:
            nt.optim.clip_grad_norm_(params, 1.0, error_if_nonfinite=True)
        scaler.step(optimizer)
        scaler.update()
        finite_seq.append(bool(finite))
    for i, p in enumerate(params):
        state = optimizer.state[id(p)]
        arrays[f"p{i}"] = p._data.copy()
        arrays[f"m{i}"] = state["exp_avg"]._data.copy()
        arrays[f"v{i}"] = state["exp_avg_sq"]._data.copy()
        arrays[f"step{i}"] = np.int64(state["step"])
    np.savez(HERE / "checkpoint_resume.npz", **arrays)
    return dict(finite=finite_seq, scale=scaler.get_scale(), scaler=scaler.state_dict(),
                saved_at=3, steps=5, optimizer_type="namitorch.optim.adam.AdamW")


def scheduler_cases(nt):
    """Learning rates of every scheduler over 14 steps on a two-group AdamW
    (lr 1e-3 and 3e-4), their state_dicts, and construction at last_step=4."""
    from namitorch.optim import lr_scheduler as sched
    specs = {
        "StepLR": dict(step_size=3, gamma=0.5),
        "MultiStepLR": dict(milestones=[2, 5, 9], gamma=0.3),
        "ExponentialLR": dict(gamma=0.9),
        "CosineAnnealingLR": dict(T_max=10, eta_min=1e-5),
        "LinearLR": dict(start_factor=0.25, end_factor=1.0, total_iters=6),
        "WarmupCosine": dict(warmup_steps=3, total_steps=12, min_lr=2e-5),
    }
    out = {}
    for name, config in specs.items():
        results = {}
        for last_step in (0, 4):
            a = nt.nn.Parameter(np.zeros(3, dtype=np.float32))
            b = nt.nn.Parameter(np.zeros(2, dtype=np.float32))
            optimizer = nt.optim.AdamW([{"params": [a]}, {"params": [b], "lr": 3e-4}], lr=1e-3)
            scheduler = getattr(sched, name)(optimizer, last_step=last_step, **config)
            lrs = [[group["lr"] for group in optimizer.param_groups]]
            for _ in range(14):
                scheduler.step()
                lrs.append([group["lr"] for group in optimizer.param_groups])
            results[f"last_step_{last_step}"] = dict(lrs=lrs, state=scheduler.state_dict(),
                                                     last_lr=scheduler.get_last_lr())
        out[name] = dict(config=config, **results)
    errors = {}

    def record(label, fn):
        try:
            fn()
        except Exception as error:  # noqa: BLE001 - the class is part of the record
            errors[label] = [type(error).__name__, str(error)]

    a = nt.nn.Parameter(np.zeros(3, dtype=np.float32))
    optimizer = nt.optim.AdamW([a], lr=1e-3)
    record("warmup_ge_total", lambda: sched.WarmupCosine(optimizer, 5, 5))
    record("min_lr_above_base", lambda: sched.WarmupCosine(optimizer, 1, 5, min_lr=1.0))
    record("step_size_zero", lambda: sched.StepLR(optimizer, 0))
    record("gamma_negative", lambda: sched.ExponentialLR(optimizer, -0.5))
    record("milestones_set", lambda: sched.MultiStepLR(optimizer, {1, 2}))
    record("last_step_bool", lambda: sched.StepLR(optimizer, 2, last_step=True))
    scheduler = sched.StepLR(optimizer, 2)
    optimizer.add_param_group({"params": [nt.nn.Parameter(np.zeros(2, dtype=np.float32))]})
    record("groups_changed", scheduler.step)
    record("load_wrong_type", lambda: sched.ExponentialLR(nt.optim.AdamW([a]), 0.5).load_state_dict(
        sched.StepLR(nt.optim.AdamW([a]), 2).state_dict()))
    out["errors"] = errors
    return out


def schedule_runner_case(nt):
    """The runner's AMP loop (training/runner.py:234-254) with WarmupCosine
    stepping only after updated steps; non-finite grads at steps 2 and 6."""
    from namitorch.optim.lr_scheduler import WarmupCosine
    params = [nt.nn.Parameter(_params(1000, np.float32, seed=51)), nt.nn.Parameter(_params(64, np.float32, seed=52))]
    optimizer = nt.optim.AdamW([{"params": [params[0]], "weight_decay": 0.1},
                                {"params": [params[1]], "weight_decay": 0.0}], lr=2e-3, betas=(0.9, 0.95))
    scheduler = WarmupCosine(optimizer, 3, 12, min_lr=1e-4)
    scaler = nt.amp.GradScaler(init_scale=4096.0, growth_interval=3)
    raw = [_grads(p.size, 10, 1e-3, np.float32, seed_base=5100 + 10 * i) for i, p in enumerate(params)]
    arrays, lr_used, updated_seq, scale_seq = {}, [], [], []
    for i, p in enumerate(params):
        arrays[f"p0_{i}"] = p._data.copy()
    for k in range(10):
        lr_used.append([group["lr"] for group in optimizer.param_groups])
        scaler.scale(nt.Tensor(np.float32(1.0)))
        for i, p in enumerate(params):
            g = (raw[i][k].astype(np.float64) * scaler.get_scale()).astype(np.float32)
            if (k, i) in ((2, 0), (6, 1)):
                g[5] = np.inf if k == 2 else np.nan
            arrays[f"grad{i}_{k}"] = g.copy()
            p._grad = nt.Tensor(g)
        finite = scaler.unscale_(optimizer)
        if finite:
            nt.optim.clip_grad_norm_(params, 1.0, error_if_nonfinite=True)
        updated = scaler.step(optimizer)
        scaler.update()
        if updated:
            scheduler.step()
        updated_seq.append(bool(updated))
        scale_seq.append(scaler.get_scale())
    for i, p in enumerate(params):
        state = optimizer.state[id(p)]
        arrays[f"p{i}"] = p._data.copy()
        arrays[f"m{i}"] = state["exp_avg"]._data.copy()
        arrays[f"v{i}"] = state["exp_avg_sq"]._data.copy()
        arrays[f"step{i}"] = np.int64(state["step"])
    np.savez(HERE / "schedule_runner.npz", **arrays)
    return dict(lr_used=lr_used, updated=updated_seq, scale=scale_seq, last_lr=scheduler.get_last_lr(),
                scheduler_state=scheduler.state_dict(), steps=10)


def accumulate_cases(nt):
    """autograd.accumulate_gradient (autograd.py:198-205): the incoming
    gradient cast to the leaf's dtype, added to the stored one in that dtype
    (or copied when there is none), for leaf dtypes float32/16/64 and incoming
    float16/32/64, with special values (signed zeros, subnormals, values that
    overflow float16, inf, NaN)."""
    from namitorch.autograd import accumulate_gradient
    rng = np.random.Generator(np.random.PCG64(61))
    n = 1031
    specials = np.array([0.0, -0.0, 1e-45, -3e-42, 6e-8, -6e-8, 65504.0, 65520.0, -70000.0, 1e38, 3.4e38,
                         np.inf, -np.inf, np.nan, 1e-300, 1e300], dtype=np.float64)
    arrays = {}
    cases = []
    for leaf in (np.float32, np.float16, np.float64):
        for incoming in (np.float16, np.float32, np.float64):
            key = f"{np.dtype(leaf).name}_{np.dtype(incoming).name}"
            parent = nt.nn.Parameter(np.zeros(n, dtype=leaf))
            existing = (rng.standard_normal(n) * 3.0).astype(leaf)
            values = rng.standard_normal(n) * np.float64(rng.choice([1e-6, 1e-2, 1.0, 1e3], size=n))
            values[: specials.size] = specials
            existing[specials.size: 2 * specials.size] = specials.astype(leaf)
            with np.errstate(over="ignore", invalid="ignore"):
                gradient = values.astype(incoming)
                added = accumulate_gradient(parent, gradient, existing.copy())
                fresh = accumulate_gradient(parent, gradient, None)
            arrays[f"{key}_existing"] = existing
            arrays[f"{key}_incoming"] = gradient
            arrays[f"{key}_added"] = np.asarray(added)
            arrays[f"{key}_fresh"] = np.asarray(fresh)
            cases.append(key)
    np.savez(HERE / "accumulate.npz", **arrays)
    return cases


def serialization_errors(nt, scratch: Path):
    """Exception class names and texts of the archive writer/reader for invalid inputs."""
    from namitorch import serialization as ser
    texts = {}

    def record(name, fn):
        try:
            fn()
        except Exception as error:  # noqa: BLE001 - the class is part of the record
            texts[name] = [type(error).__name__, str(error)]

    cyclic = []
    cyclic.append(cyclic)
    record("save_complex", lambda: ser.save({"x": np.zeros(2, dtype=np.complex128)}, scratch / "e.nt"))
    record("save_cycle", lambda: ser.save(cyclic, scratch / "e.nt"))
    record("save_int_key", lambda: ser.save({1: 2}, scratch / "e.nt"))
    record("save_object", lambda: ser.save({"x": object()}, scratch / "e.nt"))
    (scratch / "garbage.nt").write_bytes(b"not a zip archive")
    record("load_garbage", lambda: ser.load(scratch / "garbage.nt"))
    ser.save({"a": np.arange(4, dtype=np.int32)}, scratch / "ok.nt")
    record("load_max_bytes", lambda: ser.load(scratch / "ok.nt", max_array_bytes=8))
    record("load_max_bytes_type", lambda: ser.load(scratch / "ok.nt", max_array_bytes=-1))
    return texts


def error_texts(nt):
    texts = {}
    half = nt.nn.Parameter(np.zeros(3, dtype=np.float16))
    half._grad = nt.Tensor(np.zeros(3, dtype=np.float16))
    try:
        nt.optim.AdamW([half], eps=1e-8).step()
    except ValueError as error:
        texts["eps_float16"] = str(error)
    p = nt.nn.Parameter(np.zeros(3, dtype=np.float32))
    p._grad = nt.Tensor(np.zeros(3, dtype=np.float32))
    try:
        nt.optim.AdamW([p], fused=True).step()
    except RuntimeError as error:
        texts["fused_true_unsupported"] = str(error)
    try:
        nt.optim.AdamW([p], fused=1)
    except TypeError as error:
        texts["fused_type"] = str(error)
    try:
        nt.optim.AdamW([p], betas=(0.9, 1.0))
    except ValueError as error:
        texts["beta_range"] = str(error)
    scaler = nt.amp.GradScaler()
    try:
        scaler.unscale_(nt.optim.AdamW([p]))
    except RuntimeError as error:
        texts["unscale_before_scale"] = str(error)
    try:
        nt.optim.clip_grad_norm_([p], -1.0)
    except ValueError as error:
        texts["max_norm_negative"] = str(error)
    bad = nt.nn.Parameter(np.zeros(3, dtype=np.float32))
    bad._grad = nt.Tensor(np.array([1.0, np.inf, 0.0], dtype=np.float32))
    try:
        nt.optim.clip_grad_norm_([bad], 1.0, error_if_nonfinite=True)
    except RuntimeError as error:
        texts["nonfinite_norm"] = str(error)
    return texts


SCALAR_LOSSES = [3.0, -2.5, 1.0, 0.0, -0.0, 65504.0, 1e-5, 6.1e-5, 1e30, np.inf, -np.inf, np.nan, 0.1, 1.0 / 3.0]


def scalar_cases(nt):
    """GradScaler.scale (amp.py:137-138) and the runner's loss / accum
    (runner.py:246): Tensor-by-scalar arithmetic with the reference's dtype
    promotion, for float16/32/64 losses."""
    out = {}
    rng = np.random.Generator(np.random.PCG64(61))
    for dtype in (np.float16, np.float32, np.float64):
        with np.errstate(over="ignore", invalid="ignore"):
            loss = np.concatenate([np.asarray(SCALAR_LOSSES, dtype=np.float64),
                                   rng.standard_normal(50) * 4.0]).astype(dtype)
        name = np.dtype(dtype).name
        out[f"{name}_loss"] = loss
        for scale in (65536.0, 3000.0, 0.125):
            scaler = nt.amp.GradScaler(init_scale=scale)
            out[f"{name}_scale_{scale:g}"] = scaler.scale(nt.Tensor(loss.copy()))._data.copy()
        for label, divisor in (("int3", 3), ("int7", 7), ("int1000", 1000), ("float3", 3.0), ("float0.1", 0.1),
                               ("f16_3", np.float16(3.0)), ("f64_3", np.float64(3.0))):
            with np.errstate(over="ignore", invalid="ignore", divide="ignore", under="ignore"):
                out[f"{name}_div_{label}"] = (nt.Tensor(loss.copy()) / divisor)._data.copy()
        for label, factor in (("int3", 3), ("float0.1", 0.1), ("f64_0.1", np.float64(0.1))):
            with np.errstate(over="ignore", invalid="ignore", under="ignore"):
                out[f"{name}_mul_{label}"] = (nt.Tensor(loss.copy()) * factor)._data.copy()
    np.savez(HERE / "scalar_ops.npz", **out)
    return sorted(out)


def clip_f64_cases(nt):
    """clip_grad_norm_ on float64 gradients whose squares leave the float64
    range (|g| ~ 1e200 and 1e-200) and at ordinary magnitudes, p = 2 and 3."""
    rng = np.random.Generator(np.random.PCG64(67))
    shapes = [(37,), (8, 16), (1000,)]
    out = {}
    records = []
    for label, magnitude, max_norm in (("huge", 1e200, 1e199), ("tiny", 1e-200, 1e-210), ("unit", 1.0, 1.0)):
        for norm_type in (2.0, 3.0):
            grads = [rng.standard_normal(s) * magnitude for s in shapes]
            params = [nt.nn.Parameter(np.zeros(s, dtype=np.float64)) for s in shapes]
            for param, grad in zip(params, grads):
                param._grad = nt.Tensor(grad.copy())
            with np.errstate(under="ignore"):
                norm = nt.optim.clip_grad_norm_(params, max_norm, norm_type=norm_type)
            key = f"clip64_{label}_{norm_type:g}"
            for index, (grad, param) in enumerate(zip(grads, params)):
                out[f"{key}_in{index}"] = grad
                out[f"{key}_out{index}"] = param.grad._data.copy()
            records.append(dict(key=key, norm_type=norm_type, max_norm=max_norm, norm=float(norm._data),
                                count=len(shapes)))
    out["records"] = np.asarray(json.dumps(records))
    np.savez(HERE / "clip_f64.npz", **out)
    return [record["key"] for record in records]


DEVICE_SPELLINGS = ["cpu", "cuda", "cuda:0", "cuda:1", "cuda:01", "cuda:", "cpu:0", "gpu", "cuda:12", "CUDA",
                    "cuda:१", "cuda: 1", " cuda", "cuda:-1", 5, None]
DEVICE_INDICES = [None, 0, 1, -1, True, 1.0, 2]


def device_cases(nt):
    """Device(value, index) outcomes (namitorch/device.py): the string or the
    exception class and message, for spellings x index arguments, and for
    Device copies."""
    from namitorch.device import Device

    def outcome(value, index):
        try:
            made = Device(value, index)
            return ["ok", str(made), repr(made)]
        except Exception as error:            # the outcome is the fixture
            return [type(error).__name__, str(error)]

    records = [[value, index, outcome(value, index)] for value in DEVICE_SPELLINGS for index in DEVICE_INDICES]
    copies = [[value, index, outcome(Device(value), index)] for value in ("cpu", "cuda:3") for index in DEVICE_INDICES]
    (HERE / "devices.json").write_text(json.dumps({"spellings": records, "copies": copies}, indent=1) + "\n")
    return len(records) + len(copies)


# Fixture sets that write their own files (and keep their records there);
# `--only name,...` regenerates just those.
def package_checkpoint_case(nt):
    """The format's other direction: ``checkpoint_package.nt`` is written by
    this package's save_checkpoint (namitorch_amd/checkpoint.py) from the
    seeded host state of ``package_state.build``, and the reference's
    load_checkpoint (training/checkpoint.py:131-174) restores it into the
    reference's own model, AdamW, WarmupCosine and GradScaler.  What the
    reference restored is stored: the arrays in ``package_checkpoint.npz``,
    the rest in ``package_checkpoint.json``."""
    sys.path.insert(0, str(HERE.parents[1]))
    sys.path.insert(0, str(HERE))
    import namitorch_amd as ours
    import package_state
    from namitorch_amd import checkpoint as our_checkpoint
    from namitorch.optim.lr_scheduler import WarmupCosine
    from namitorch.training.checkpoint import load_checkpoint

    named, optimizer, scheduler, scaler = package_state.build(ours)
    path = HERE / "checkpoint_package.nt"
    our_checkpoint.save_checkpoint(path, named, optimizer, scheduler, scaler=scaler, **package_state.SAVE)

    class Tiny(nt.nn.Module):
        def __init__(self):
            super().__init__()
            self.weight = nt.nn.Parameter(np.zeros((40, 48), np.float32))
            self.bias = nt.nn.Parameter(np.zeros(40, np.float32))

    model = Tiny()
    theirs = nt.optim.AdamW([{"params": [model.weight], "weight_decay": 0.1},
                             {"params": [model.bias], "weight_decay": 0.0}], lr=2e-3, betas=(0.9, 0.95), eps=1e-8)
    their_scheduler = WarmupCosine(theirs, 3, 12, min_lr=1e-4)
    their_scaler = nt.amp.GradScaler()
    info = load_checkpoint(path, model, theirs, their_scheduler, scaler=their_scaler)
    arrays = {}
    groups = []
    for index, (name, parameter) in enumerate((("weight", model.weight), ("bias", model.bias))):
        state = theirs.state[id(parameter)]
        arrays[f"{name}"] = parameter._data.copy()
        arrays[f"{name}_exp_avg"] = state["exp_avg"]._data.copy()
        arrays[f"{name}_exp_avg_sq"] = state["exp_avg_sq"]._data.copy()
        arrays[f"{name}_step"] = np.int64(state["step"])
    for group in theirs.param_groups:
        groups.append({key: (list(value) if isinstance(value, tuple) else value)
                       for key, value in group.items() if key != "params"})
    np.savez(HERE / "package_checkpoint.npz", **arrays)
    record = dict(info={key: value for key, value in info.items() if key != "load_result"},
                  load_result=repr(info["load_result"]), param_groups=groups,
                  scheduler=their_scheduler.state_dict(), last_lr=their_scheduler.get_last_lr(),
                  scaler=their_scaler.state_dict(), scale=their_scaler.get_scale())
    (HERE / "package_checkpoint.json").write_text(json.dumps(record, indent=1, sort_keys=True) + "\n")
    return record


STANDALONE = {"scalar_ops": scalar_cases, "clip_f64": clip_f64_cases, "devices": device_cases,
              "package_checkpoint": package_checkpoint_case}


def main(reference: str, only: list[str] | None = None) -> None:
    sys.path.insert(0, reference)
    import namitorch as nt  # the reference, on its NumPy (CPU) backend
    if only:
        for name in only:
            print(name, STANDALONE[name](nt))
        return
    for function in STANDALONE.values():
        function(nt)
    golden = {
        "source": "renderityai/NamiTorch NumPy backend (optim/adam.py, optim/clip_grad.py, amp.py)",
        "numpy": np.__version__,
        "adam_cases": adam_cases(nt),
        "clip": clip_cases(nt),
        "scaler": scaler_cases(nt),
        "errors": error_texts(nt),
        "checkpoint": checkpoint_case(nt),
        "schedulers": scheduler_cases(nt),
        "schedule_runner": schedule_runner_case(nt),
        "accumulate": accumulate_cases(nt),
    }
    import tempfile
    with tempfile.TemporaryDirectory() as scratch:
        golden["serialization_errors"] = serialization_errors(nt, Path(scratch))
    (HERE / "golden.json").write_text(json.dumps(golden, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    arguments = [argument for argument in sys.argv[1:] if not argument.startswith("--only=")]
    selected = [argument.split("=", 1)[1] for argument in sys.argv[1:] if argument.startswith("--only=")]
    main(arguments[0] if arguments else "/root/reference", selected[0].split(",") if selected else None)
