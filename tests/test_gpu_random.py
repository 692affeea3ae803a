"""Seeded random compositions of the optimizer step against the oracle.

Each case draws, from its seed, a parameter layout (float32, float16 or
float64 parameters and gradients, or low-precision parameters with float32
master weights and float32 or bfloat16 moments), one or two parameter groups
with their own options (lr including 0, betas including beta1 = 0, eps,
weight decay, maximize, the fused switch; Adam with coupled decay or AdamW),
tensors of ragged sizes around the kernels' slice and task boundaries,
gradients with subnormal and (without a scaler) non-finite values, storage
adopted from PyTorch at offsets that break 16-byte alignment, and
optionally a GradScaler (scales that are and are not powers of two, a seeded
inf or NaN, growth within the run), clipping (active, inactive, or to zero
with max_norm 0) and a second micro-batch accumulated eagerly or deferred,
into freshly assigned gradients or into gradients zeroed in place by
``zero_grad(set_to_none=False)``.  Three steps run through the reference's call sequence
(``unscale_`` -> ``clip_grad_norm_`` if finite -> ``step`` -> ``update``,
training/runner.py:240-254) and through ``amp.fused_step``; both are
compared with the oracle composed on the host (``grads.accumulate`` ->
``scaler.unscale`` -> ``clip.clip_grad_norm`` -> ``adam.adam_step`` /
``adam.master_step``).

Bars: found_inf/updated flags, step counts and the loss scale exact; norms
within 1e-12 relative; parameters, master weights and moments bit-exact
(NaN equal to NaN whatever its payload).  A
clip coefficient a few float64 ulps away from the oracle's (the norms agree
to 1e-12, not bit for bit) can move a clipped gradient across a rounding
boundary of its dtype, which for these sizes is expected well below once per
run; a case whose clip was active therefore allows at most two elements per
array that differ, by at most two units of the stored type.  For float64
gradients the clipped value is the float64 product itself, so every element
depends on the coefficient's last bits (about one in ten moves by an ulp):
with an active clip the float64 layout is compared to 1e-10 relative, the
norm's 1e-12 carried through m, v and the update.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import namitorch_amd as nt
from oracle import adam as oadam
from oracle import clip as oclip
from oracle import grads as ograds
from oracle import lowp
from oracle import scaler as oscaler

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
STEPS = 3
CASES = 120
NORM_RTOL = 1e-12
SIZES = (1, 3, 255, 256, 257, 1000, 2047, 2048, 2049, 4095, 4096, 4097, 8191, 12289, 65537, 100003)
SHAPES_2D = ((3, 1000), (768, 3), (64, 65), (2, 2048))


def _host(values: np.ndarray, dtype: str) -> np.ndarray:
    """Host representation of `values` (float64) stored in `dtype`:
    bfloat16 as bfloat16-valued float32."""
    if dtype == "bfloat16":
        return lowp.round_to("bfloat16", values)
    return values.astype(dtype)


def _draw_case(seed: int) -> dict:
    rng = np.random.default_rng(seed)
    layout = str(rng.choice(["f32", "f32", "f16", "f64", "master", "master"]))
    if layout == "master":
        param_dtype = str(rng.choice(["bfloat16", "float16"]))
        grad_dtype = str(rng.choice(["bfloat16", "float16"]))
        state_dtype = str(rng.choice(["float32", "bfloat16"]))
    else:
        param_dtype = grad_dtype = {"f32": "float32", "f16": "float16", "f64": "float64"}[layout]
        state_dtype = None
    kind = "adam" if layout != "master" and rng.random() < 0.25 else "adamw"
    count = int(rng.integers(1, 6))
    shapes = []
    for _ in range(count):
        if rng.random() < 0.25:
            shapes.append(SHAPES_2D[int(rng.integers(len(SHAPES_2D)))])
        else:
            shapes.append((int(rng.choice(SIZES)),))
    groups = []
    order = [int(i) for i in rng.permutation(count)]
    cut = int(rng.integers(1, count)) if count > 1 and rng.random() < 0.5 else count
    for members in (order[:cut], order[cut:]):
        if not members:
            continue
        eps = [1e-4, 1e-3] if layout == "f16" else [1e-8, 1e-6]
        fused = [None, False, True] if layout == "f32" else [None, False]
        group = dict(members=sorted(members), lr=float(rng.choice([0.0, 1e-3, 3e-4], p=[0.15, 0.45, 0.4])),
                     betas=(float(rng.choice([0.9, 0.8, 0.0])), float(rng.choice([0.999, 0.95]))),
                     eps=float(rng.choice(eps)), weight_decay=float(rng.choice([0.0, 0.01, 0.1])),
                     maximize=bool(rng.random() < 0.3))
        fused_choice = fused[int(rng.integers(len(fused)))]
        if kind == "adamw":
            group["fused"] = fused_choice
        groups.append(group)
    amp = bool(rng.random() < 0.5)
    scale = float(rng.choice([65536.0, 1024.0, 3.0, 0.5])) if amp else 1.0
    interval = int(rng.choice([1, 2, 2000]))
    poison = None
    if amp and rng.random() < 0.5:
        tensor = int(rng.integers(count))
        poison = (int(rng.integers(STEPS)), tensor, int(rng.integers(int(np.prod(shapes[tensor])))),
                  float(rng.choice([np.inf, -np.inf, np.nan])))
    sigma = 1e-2 if layout == "f16" else 1e-3
    clip = bool(rng.random() < 0.5)
    # Accumulation keeps the parameter's dtype (autograd.py:198-205 refuses others).
    accumulate = bool(rng.random() < 0.3) and grad_dtype == param_dtype
    defer = bool(rng.random() < 0.5)
    zeroed = accumulate and bool(rng.random() < 0.4)
    # Tensors adopted from another framework at an element offset that breaks
    # 16-byte alignment (the kernels' scalar paths), per tensor.
    misalign = bool(rng.random() < 0.25)
    offsets = [int(rng.integers(0, 8)) if misalign else 0 for _ in range(count)]
    # Without a scaler: subnormal and non-finite gradient values at seeded places.
    specials = []
    if not amp and rng.random() < 0.3:
        tiny = {"float32": 1e-40, "float64": 1e-310, "float16": 3e-8, "bfloat16": 1e-40}[grad_dtype]
        for value in (tiny, -tiny, float(rng.choice([np.inf, -np.inf, np.nan]))):
            tensor = int(rng.integers(count))
            specials.append((int(rng.integers(STEPS)), tensor, int(rng.integers(int(np.prod(shapes[tensor])))), value))
    params = [_host(rng.standard_normal(s) * 0.02, param_dtype) for s in shapes]
    grads, incoming = [], []
    for step in range(STEPS):
        grads.append([_host(rng.standard_normal(s) * sigma * scale, grad_dtype) for s in shapes])
        incoming.append([_host(rng.standard_normal(s) * sigma * scale, grad_dtype) for s in shapes])
        if poison is not None and poison[0] == step:
            grads[step][poison[1]].reshape(-1)[poison[2]] = poison[3]
        for at, tensor, element, value in specials:
            if at == step:
                grads[step][tensor].reshape(-1)[element] = _host(np.array([value]), grad_dtype)[0]
    # A max_norm around the typical unscaled norm: clipping active on some steps.
    typical = sigma * math.sqrt(sum(int(np.prod(s)) for s in shapes)) * (1.4 if accumulate else 1.0)
    max_norm = (0.0 if rng.random() < 0.1 else float(typical * rng.uniform(0.3, 2.0))) if clip else None
    return dict(seed=seed, kind=kind, layout=layout, param_dtype=param_dtype, grad_dtype=grad_dtype,
                state_dtype=state_dtype, shapes=shapes, groups=groups, amp=amp, scale=scale, interval=interval,
                poison=poison, specials=specials, max_norm=max_norm, accumulate=accumulate, defer=defer,
                zeroed=zeroed, params=params, grads=grads, incoming=incoming, offsets=offsets)


def _oracle(case: dict) -> dict:
    gdtype = case["grad_dtype"]
    master_mode = case["layout"] == "master"
    state_bf16 = case["state_dtype"] == "bfloat16"
    if master_mode:
        values = [p.astype(np.float32) for p in case["params"]]
    else:
        values = [p.copy() for p in case["params"]]
    m = [np.zeros(v.shape, dtype=v.dtype) for v in values]
    v2 = [np.zeros(v.shape, dtype=v.dtype) for v in values]
    options = {}
    for group in case["groups"]:
        for i in group["members"]:
            options[i] = group
    scaler = oscaler.Scaler(case["scale"], 2.0, 0.5, case["interval"]) if case["amp"] else None
    count, flags, norms, clipped_any = 0, [], [], False
    for step in range(STEPS):
        grads = case["grads"][step]
        if case["zeroed"] and step > 0:
            # zero_grad(set_to_none=False), then this micro-batch accumulated into the zeros.
            grads = [ograds.accumulate(np.zeros_like(g), g, gdtype) for g in grads]
        if case["accumulate"]:
            grads = [ograds.accumulate(g, h, gdtype) for g, h in zip(grads, case["incoming"][step])]
        if scaler is not None:
            grads = [oscaler.unscale(g, scaler.scale, gdtype) for g in grads]
            finite = oscaler.finite(grads)
        else:
            finite = True
        norm = None
        if case["max_norm"] is not None and finite:
            norm, grads = oclip.clip_grad_norm(grads, case["max_norm"], 2.0, gdtype)
            clipped_any |= oclip.clip_coefficient(case["max_norm"], norm) < 1
        if finite:
            count += 1
            for i, g in enumerate(grads):
                o = options[i]
                kw = dict(lr=o["lr"], betas=o["betas"], eps=o["eps"], weight_decay=o["weight_decay"],
                          maximize=o["maximize"])
                if master_mode:
                    oadam.master_step(values[i], np.asarray(g, dtype=np.float32), m[i], v2[i], count,
                                      state_bf16=state_bf16, **kw)
                else:
                    oadam.adam_step(values[i], g, m[i], v2[i], count, decoupled=case["kind"] == "adamw", **kw)
        if scaler is not None:
            scaler.update(not finite)
        flags.append(finite)
        norms.append(norm)
    copies = [oadam.copy_out(x, case["param_dtype"]) for x in values] if master_mode else values
    return dict(values=values, m=m, v=v2, copies=copies, count=count, flags=flags, norms=norms,
                scale=scaler.scale if scaler is not None else None, clipped=clipped_any)


def _adopted(host: np.ndarray, dtype: str, offset: int, parameter: bool = False):
    """`host` on the device in `dtype`; with an offset, as a view that starts
    `offset` elements into a larger PyTorch allocation (adopted, not copied)."""
    if offset == 0:
        return (nt.Parameter if parameter else nt.Tensor)(host, dtype=dtype, device=DEV)
    import torch
    kind = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16,
            "float64": torch.float64}[dtype]
    base = torch.zeros(host.size + offset, dtype=kind, device=DEV)
    view = base[offset:].view(host.shape)
    view.copy_(torch.from_numpy(np.ascontiguousarray(host)).to(DEV).to(kind))    # exact: host holds dtype values
    if not parameter:
        return nt.Tensor._from_storage(view)
    adopted = nt.Parameter.__new__(nt.Parameter)
    nt.Tensor._initialize(adopted, view, True)
    return adopted


def _device(case: dict, path: str) -> dict:
    offsets = case["offsets"]
    params = [_adopted(p, case["param_dtype"], o, parameter=True) for p, o in zip(case["params"], offsets)]
    groups = [dict(params=[params[i] for i in g["members"]],
                   **{k: value for k, value in g.items() if k != "members"}) for g in case["groups"]]
    master_mode = case["layout"] == "master"
    if case["kind"] == "adam":
        optimizer = nt.optim.Adam(groups)
    else:
        optimizer = nt.optim.AdamW(groups, master_weights=master_mode,
                                   state_dtype=case["state_dtype"] if master_mode else None)
    scaler = nt.GradScaler(init_scale=case["scale"], growth_factor=2.0, backoff_factor=0.5,
                           growth_interval=case["interval"]) if case["amp"] else None
    flags, norms = [], []
    for step in range(STEPS):
        if scaler is not None:
            scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
        arrived = [_adopted(g, case["grad_dtype"], (o * 3) % 8) for g, o in zip(case["grads"][step], offsets)]
        if case["zeroed"] and step > 0:
            optimizer.zero_grad(set_to_none=False)
            nt.accumulate_grads(params, arrived)
        else:
            for p, g in zip(params, arrived):
                p.grad = g
        if case["accumulate"]:
            incoming = [_adopted(h, case["grad_dtype"], (o * 5) % 8) for h, o in zip(case["incoming"][step], offsets)]
            nt.accumulate_grads(params, incoming, defer=case["defer"])
        if path == "api":
            finite = scaler.unscale_(optimizer) if scaler is not None else True
            norm = None
            if case["max_norm"] is not None and finite:
                norm = nt.optim.clip_grad_norm_(params, case["max_norm"]).item()
            if scaler is not None:
                updated = scaler.step(optimizer)
                scaler.update()
            else:
                optimizer.step()
                updated = True
        else:
            result = nt.amp.fused_step(optimizer, scaler, max_norm=case["max_norm"])
            finite = result.finite if scaler is not None else True
            updated = result.updated
            norm = result.norm if finite else None
        assert updated == finite, (path, step)
        flags.append(finite)
        norms.append(norm)
    out = dict(flags=flags, norms=norms, scale=scaler.get_scale() if scaler is not None else None,
               copies=[p.numpy() for p in params], steps=[], m=[], v=[], values=[])
    for p in params:
        state = optimizer.state.get(id(p), {})
        out["steps"].append(state.get("step", 0))
        out["m"].append(state["exp_avg"].numpy() if "exp_avg" in state else None)
        out["v"].append(state["exp_avg_sq"].numpy() if "exp_avg_sq" in state else None)
        out["values"].append(state["master"].numpy() if master_mode and "master" in state else None)
    return out


def _compare(label: str, got: np.ndarray, want: np.ndarray, loose: bool) -> None:
    got = np.ascontiguousarray(got).reshape(-1)
    want = np.ascontiguousarray(want).reshape(-1)
    assert got.shape == want.shape and got.dtype == want.dtype, (label, got.dtype, want.dtype)
    if loose and got.dtype == np.float64:
        finite = np.isfinite(want)
        scale = float(np.max(np.abs(want[finite]), initial=0.0))
        close = np.isclose(got, want, rtol=1e-10, atol=1e-12 * scale, equal_nan=True) | (got == want)
        assert np.all(close), f"{label}: {np.count_nonzero(~close)} of {got.size} elements beyond 1e-10"
        return
    unsigned = {2: np.uint16, 4: np.uint32, 8: np.uint64}[got.itemsize]
    signed = {2: np.int16, 4: np.int32, 8: np.int64}[got.itemsize]
    both_nan = np.isnan(got.astype(np.float64)) & np.isnan(want.astype(np.float64))
    bad = np.flatnonzero((got.view(unsigned) != want.view(unsigned)) & ~both_nan)
    if bad.size == 0:
        return
    assert loose and bad.size <= 2, f"{label}: {bad.size} of {got.size} elements differ, e.g. {got[bad[:3]]} vs {want[bad[:3]]}"
    unit = 1 << 16 if label.endswith("bf16") else 1
    distance = np.abs(got.view(signed)[bad].astype(np.int64) - want.view(signed)[bad].astype(np.int64))
    assert np.all(distance <= 2 * unit), f"{label}: differences beyond two units"


def _bf16(dtype: str | None) -> str:
    return " bf16" if dtype == "bfloat16" else ""


@pytest.mark.parametrize("seed", range(CASES))
def test_random_composition_matches_oracle(seed):
    case = _draw_case(1000 + seed)
    print(f"case {seed}: {case['kind']} {case['layout']} p={case['param_dtype']} g={case['grad_dtype']} s={case['state_dtype']} "
          f"shapes={case['shapes']} amp={case['amp']} scale={case['scale']} poison={case['poison']} "
          f"clip={case['max_norm']} accumulate={case['accumulate']} defer={case['defer']} zeroed={case['zeroed']} "
          f"offsets={case['offsets']} "
          f"specials={case['specials']}", flush=True)
    want = _oracle(case)
    loose = want["clipped"]
    for path in ("api", "fused"):
        got = _device(case, path)
        assert got["flags"] == want["flags"], (path, got["flags"], want["flags"])
        assert got["scale"] == want["scale"], (path, got["scale"], want["scale"])
        for step, (a, b) in enumerate(zip(got["norms"], want["norms"])):
            if b is None:
                continue
            if math.isfinite(b):
                assert abs(a - b) <= NORM_RTOL * b, (path, step, a, b)
            else:
                assert (math.isnan(a) and math.isnan(b)) or a == b, (path, step, a, b)
        master_mode = case["layout"] == "master"
        state = case["state_dtype"] if master_mode else case["param_dtype"]
        for i in range(len(case["shapes"])):
            assert got["steps"][i] == want["count"], (path, i, got["steps"][i], want["count"])
            if want["count"] == 0:
                continue
            _compare(f"{path} param[{i}]{_bf16(case['param_dtype'])}", got["copies"][i], want["copies"][i], loose)
            _compare(f"{path} m[{i}]{_bf16(state)}", got["m"][i], want["m"][i], loose)
            _compare(f"{path} v[{i}]{_bf16(state)}", got["v"][i], want["v"][i], loose)
            if master_mode:
                _compare(f"{path} master[{i}]", got["values"][i], want["values"][i], loose)
