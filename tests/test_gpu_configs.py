"""The benchmark configurations as composed 10-step runs against the oracle.

Each run goes through the reference's call sequence (``unscale_`` ->
``clip_grad_norm_`` -> ``step`` -> ``update``, training/runner.py:248-251)
and through ``amp.fused_step``, and is compared with the oracle's
``scaler.unscale`` -> ``clip.clip_grad_norm`` -> ``adam.master_step`` /
``adam.adam_step`` composed on the host (evaluated slice-wise on a thread
pool by ``oracle.parallel``, which gives the oracle's bits):

* C2: the full GPT-2-124M list (148 tensors, 124,439,808 parameters), float32
  AdamW in the two ``decay_parameter_groups`` groups (runner.py:83-90);
* C3: the full GPT-2-124M list with AMP: bfloat16 model + float32 master,
  float16 gradients f16(N(0, 1e-3) * 65536), one +inf in a matrix at step 3
  (GradScaler(65536, x2, x0.5, 2000)) or one NaN in a vector at step 6 (a
  growth_interval 3 variant that grows, backs off and grows again), at a
  seeded element; the whole state is compared after the step that follows
  the skipped one and after the last step;
* C4: the full GPT-1.3B list (292 tensors, 1,315,819,520 parameters):
  float32 master, bfloat16 parameters/moments/gradients, clip_grad_norm_ at
  1.0 (active every step); both paths step in lockstep on the same
  gradients, which come from the device's generator and are copied back for
  the oracle;
* C5: the full Llama-7B list (291 tensors, 6,738,415,616 parameters) through
  ``fused_step`` for two steps: bfloat16 model + float32 master and moments,
  bfloat16 gradients scaled by 65536, clip at 1.0.  The norm's oracle streams
  the gradients back one tensor at a time (``parallel.total_norm_streamed``);
  a seeded sample of whole tensors (the embedding, the head, the final norm
  and five others) is stepped by the oracle and compared;
* C4/8 and C5/8: one rank's slices of an 8-way sharded step (every tensor's
  flat storage cut in eight) through ``fused_step``, the whole state of every
  slice compared.

Bars (the path's target tolerances): found_inf flags, skip decisions and the
loss-scale sequence bit-exact; norms within 1e-12 relative; float32 master,
parameters and moments bit-exact, and model copies and bfloat16 moments
equal to the oracle's RNE values.  A clip coefficient one float64 ulp away
from the oracle's can move a clipped gradient across a rounding boundary;
for bfloat16 gradients that has a probability of about 2**-43 per element, so
any such element is allowed only within one unit of the storage type and at
a rate below 1e-6.
"""

from __future__ import annotations

import gc
import math

import numpy as np
import pytest
import torch

import namitorch_amd as nt
from namitorch_amd.param_lists import decay_mask, gpt2_shapes, gpt_1p3b_shapes, llama7b_shapes, total_params
from oracle import clip as oclip
from oracle import lowp, parallel
from oracle import scaler as oscaler

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
STEPS = 10
NORM_RTOL = 1e-12
OPTIONS = dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8)


@pytest.fixture(scope="module")
def pool():
    with parallel.Pool() as threads:
        yield threads


def _normals(pool, shapes, seed, sigma):
    """float32 N(0, sigma) per tensor, each from its own PCG64 stream
    (SeedSequence(seed).spawn), drawn in parallel."""
    streams = np.random.SeedSequence(seed).spawn(len(shapes))

    def draw(shape, stream):
        values = np.random.Generator(np.random.PCG64(stream)).standard_normal(shape, dtype=np.float32)
        values *= np.float32(sigma)
        return values

    return pool.run([lambda s=s, q=q: draw(s, q) for s, q in zip(shapes, streams)])


def _say(message):
    print(message, flush=True)


def _compare(label, got, want, unit_bits=None, allow_rate=0.0):
    """Bit-exact, or (allow_rate > 0) mismatches within one unit of the
    storage type (unit_bits: 16 for bfloat16 values held as float32) at a
    rate below allow_rate."""
    got = np.ascontiguousarray(got).reshape(-1)
    want = np.ascontiguousarray(want).reshape(-1)
    assert got.shape == want.shape and got.dtype == want.dtype, label
    bad = np.flatnonzero(got.view(np.uint32 if got.itemsize == 4 else np.uint16)
                         != want.view(np.uint32 if want.itemsize == 4 else np.uint16))
    if bad.size == 0:
        return 0
    assert bad.size <= allow_rate * got.size, f"{label}: {bad.size} of {got.size} elements differ"
    step = 1 << (32 - unit_bits) if unit_bits else 1
    distance = np.abs(got.view(np.int32)[bad].astype(np.int64) - want.view(np.int32)[bad].astype(np.int64))
    assert np.all(distance <= step), f"{label}: differences beyond one unit"
    return int(bad.size)


def _release():
    """Return the device memory of finished runs (both allocators)."""
    gc.collect()
    torch.cuda.synchronize()
    nt.runtime.empty_cache(0)
    torch.cuda.empty_cache()


def _device_normals(shapes, seed, sigma, dtype):
    """dtype(N(0, sigma)) per tensor from the device's generator."""
    generator = torch.Generator(device=DEV).manual_seed(seed)
    return [torch.randn(shape, generator=generator, device=DEV, dtype=torch.float32).mul_(sigma).to(dtype)
            for shape in shapes]


def _host_bf16(pool, tensor):
    """A bfloat16 device tensor as bfloat16-valued float32 on the host."""
    bits = tensor.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    return pool.mapped(lowp.bf16_to_f32, bits, np.float32)


def _groups(params, shapes, weight_decay=0.1):
    mask = decay_mask(shapes)
    return [{"params": [p for p, m in zip(params, mask) if m], "weight_decay": weight_decay},
            {"params": [p for p, m in zip(params, mask) if not m], "weight_decay": 0.0}]


# ---- C2 --------------------------------------------------------------------------------------------
def test_c2_full_gpt2_fp32_ten_steps(pool):
    shapes = gpt2_shapes()
    assert len(shapes) == 148 and total_params(shapes) == 124_439_808
    host = _normals(pool, shapes, 1337, 0.02)
    params = [nt.Parameter(h, device=DEV) for h in host]
    optimizer = nt.optim.AdamW(_groups(params, shapes), **OPTIONS)
    ref_p = [h.copy() for h in host]
    ref_m = [np.zeros_like(h) for h in host]
    ref_v = [np.zeros_like(h) for h in host]
    decays = [0.1 if m else 0.0 for m in decay_mask(shapes)]
    for step in range(1, STEPS + 1):
        grads = _normals(pool, shapes, 1337 + 1000 + step, 1e-3)
        for p, g in zip(params, grads):
            p.grad = nt.Tensor(g, device=DEV)
        optimizer.step()
        for i, g in enumerate(grads):
            parallel.adam_step(pool, ref_p[i], g, ref_m[i], ref_v[i], step, weight_decay=decays[i], **OPTIONS)
        _say(f"C2 step {step} done")
    for i, p in enumerate(params):
        state = optimizer.state[id(p)]
        _compare(f"p[{i}]", p.numpy(), ref_p[i])
        _compare(f"m[{i}]", state["exp_avg"].numpy(), ref_m[i])
        _compare(f"v[{i}]", state["exp_avg_sq"].numpy(), ref_v[i])
        assert state["step"] == STEPS


# ---- C3 --------------------------------------------------------------------------------------------
def _c3_oracle(pool, shapes, host, grads16, growth_interval, snapshot_step):
    """Oracle trajectory of the C3 recipe: flags, scales, the state after
    step index `snapshot_step` (master, m, v, copies) and the final state."""
    master = [h.copy() for h in host]
    m = [np.zeros_like(h) for h in host]
    v = [np.zeros_like(h) for h in host]
    decays = [0.1 if k else 0.0 for k in decay_mask(shapes)]
    scaler = oscaler.Scaler(65536.0, 2.0, 0.5, growth_interval)
    finite_flags, scales, count = [], [], 0
    snapshot = None
    for index, grads in enumerate(grads16):
        unscaled = [parallel.unscale(pool, g, scaler.scale, "float16") for g in grads]
        finite = parallel.finite(pool, unscaled)
        if finite:
            count += 1
            for i, u in enumerate(unscaled):
                parallel.master_step(pool, master[i], u, m[i], v[i], count, weight_decay=decays[i], **OPTIONS)
        scaler.update(not finite)
        finite_flags.append(finite)
        scales.append(scaler.scale)
        if index == snapshot_step:
            snapshot = ([x.copy() for x in master], [x.copy() for x in m], [x.copy() for x in v],
                        [parallel.round_bf16(pool, x) for x in master], count)
    copies = [parallel.round_bf16(pool, x) for x in master]
    return finite_flags, scales, master, m, v, copies, count, snapshot


def _compare_c3_state(mode, params, optimizer, master, m, v, copies, count):
    for i, p in enumerate(params):
        state = optimizer.state[id(p)]
        assert state["step"] == count
        _compare(f"{mode} master[{i}]", state["master"].numpy(), master[i])
        _compare(f"{mode} m[{i}]", state["exp_avg"].numpy(), m[i])
        _compare(f"{mode} v[{i}]", state["exp_avg_sq"].numpy(), v[i])
        _compare(f"{mode} copy[{i}]", p.numpy(), copies[i])


@pytest.mark.parametrize("poison,growth_interval,bad_step,kind", [(np.inf, 2000, 3, "matrix"), (np.nan, 3, 6, "vector")])
def test_c3_gpt2_amp_ten_steps(pool, poison, growth_interval, bad_step, kind):
    shapes = gpt2_shapes()
    host = [parallel.round_bf16(pool, h) for h in _normals(pool, shapes, 1337, 0.02)]
    pick = np.random.Generator(np.random.PCG64(7))
    candidates = [i for i, shape in enumerate(shapes) if (len(shape) >= 2) == (kind == "matrix")]
    bad_tensor = candidates[int(pick.integers(0, len(candidates)))]
    bad_element = int(pick.integers(0, int(np.prod(shapes[bad_tensor]))))
    grads16 = []
    for step in range(STEPS):
        values = _normals(pool, shapes, 1337 + 1000 + step, 1e-3)
        step_grads = pool.run([lambda g=g: (g * np.float32(65536.0)).astype(np.float16) for g in values])
        if step == bad_step:
            step_grads[bad_tensor].reshape(-1)[bad_element] = poison
        grads16.append(step_grads)
    after = bad_step + 1                          # the step after the skipped one
    finite_flags, scales, master, m, v, copies, count, snapshot = _c3_oracle(pool, shapes, host, grads16,
                                                                             growth_interval, after)
    assert finite_flags.count(False) == 1 and not finite_flags[bad_step]
    if growth_interval == 3:
        assert max(scales) > 65536.0              # the run grows the scale
        assert scales[bad_step] < scales[bad_step - 1]   # and backs off at the skip
    _say(f"C3 oracle done: skip at step {bad_step} (tensor {bad_tensor}, {kind}), scales {scales}")
    for mode in ("api", "fused"):
        params = [nt.Parameter(h, dtype="bfloat16", device=DEV) for h in host]
        optimizer = nt.optim.AdamW(_groups(params, shapes), master_weights=True, **OPTIONS)
        scaler = nt.GradScaler(init_scale=65536.0, growth_factor=2.0, backoff_factor=0.5,
                               growth_interval=growth_interval)
        for step, grads in enumerate(grads16):
            scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
            for p, g in zip(params, grads):
                p.grad = nt.Tensor(g, device=DEV)
            if mode == "api":
                finite = scaler.unscale_(optimizer)
                updated = scaler.step(optimizer)
                scaler.update()
            else:
                result = nt.amp.fused_step(optimizer, scaler)
                finite, updated = result.finite, result.updated
            assert finite == finite_flags[step] and updated == finite_flags[step], (mode, step)
            assert scaler.get_scale() == scales[step], (mode, step)
            if step == after:
                _compare_c3_state(f"{mode} step {step}", params, optimizer, *snapshot)
        _compare_c3_state(mode, params, optimizer, master, m, v, copies, count)
        _say(f"C3 {mode} matches the oracle after step {after} and at the end")
        del params, optimizer


# ---- C4 --------------------------------------------------------------------------------------------
def test_c4_full_gpt1p3b_bf16_clip_ten_steps(pool):
    shapes = gpt_1p3b_shapes()
    assert len(shapes) == 292 and total_params(shapes) == 1_315_819_520
    host = [parallel.round_bf16(pool, h) for h in _normals(pool, shapes, 1337, 0.02)]
    master = [h.copy() for h in host]
    m = [np.zeros_like(h) for h in host]
    v = [np.zeros_like(h) for h in host]
    decays = [0.1 if k else 0.0 for k in decay_mask(shapes)]
    modes = ("api", "fused")
    params = {mode: [nt.Parameter(h, dtype="bfloat16", device=DEV) for h in host] for mode in modes}
    del host
    optimizers = {mode: nt.optim.AdamW(_groups(params[mode], shapes), master_weights=True, state_dtype="bfloat16",
                                       **OPTIONS) for mode in modes}
    for step in range(1, STEPS + 1):
        grads = _device_normals(shapes, 1337 + 1000 + step, 1e-3, torch.bfloat16)
        for mode in modes:
            for p, g in zip(params[mode], grads):
                p.grad = nt.Tensor(g)                 # a copy in the library's memory
        got = {"api": nt.optim.clip_grad_norm_(params["api"], 1.0)}
        optimizers["api"].step()
        got["fused"] = nt.amp.fused_step(optimizers["fused"], None, max_norm=1.0).norm
        # Oracle: clip at 1.0 (always active here), then the master step with bfloat16 moments.
        host_grads = [_host_bf16(pool, g) for g in grads]
        del grads
        norm = parallel.total_norm_streamed(pool, len(host_grads), lambda i: host_grads[i])
        coefficient = oclip.clip_coefficient(1.0, norm)
        assert coefficient < 1
        for i, g in enumerate(host_grads):
            clipped = parallel.clip_apply(pool, g, coefficient, "bfloat16")
            parallel.master_step(pool, master[i], clipped, m[i], v[i], step, weight_decay=decays[i], state_bf16=True,
                                 **OPTIONS)
        del host_grads
        for mode in modes:
            value = got[mode].item() if mode == "api" else got[mode]
            assert abs(value - norm) <= NORM_RTOL * norm, (mode, step, value, norm)
        _say(f"C4 step {step}: norm {norm:.9g}")
    for mode in modes:
        flips = 0
        for i, p in enumerate(params[mode]):
            state = optimizers[mode].state[id(p)]
            assert state["step"] == STEPS
            flips += _compare(f"{mode} master[{i}]", state["master"].numpy(), master[i], unit_bits=32, allow_rate=1e-6)
            flips += _compare(f"{mode} m[{i}]", state["exp_avg"].numpy(), m[i], unit_bits=16, allow_rate=1e-6)
            flips += _compare(f"{mode} v[{i}]", state["exp_avg_sq"].numpy(), v[i], unit_bits=16, allow_rate=1e-6)
            flips += _compare(f"{mode} copy[{i}]", p.numpy(), lowp.round_bf16(master[i]), unit_bits=16,
                              allow_rate=1e-6)
        _say(f"C4 {mode} matches the oracle over the full list ({flips} elements one unit away)")
    del params, optimizers
    _release()


# ---- C5 --------------------------------------------------------------------------------------------
def test_c5_full_llama7b_amp_clip_two_steps(pool):
    """Two fused steps over the whole Llama-7B list; the norm, flags and scale
    against the oracle over every gradient, the state of a seeded sample of
    whole tensors against the oracle's steps of those tensors."""
    shapes = llama7b_shapes()
    assert len(shapes) == 291 and total_params(shapes) == 6_738_415_616
    pick = np.random.Generator(np.random.PCG64(11))
    sample = sorted({0, len(shapes) - 1, len(shapes) - 2}
                    | {int(i) for i in pick.choice(np.arange(1, len(shapes) - 2), 5, replace=False)})
    decays = [0.1 if k else 0.0 for k in decay_mask(shapes)]
    scale = 65536.0
    weights = _device_normals(shapes, 1337, 0.02, torch.bfloat16)
    params = [nt.Parameter(w) for w in weights]
    master = {i: _host_bf16(pool, weights[i]) for i in sample}
    del weights
    m = {i: np.zeros_like(master[i]) for i in sample}
    v = {i: np.zeros_like(master[i]) for i in sample}
    optimizer = nt.optim.AdamW(_groups(params, shapes), master_weights=True, **OPTIONS)
    scaler = nt.GradScaler(init_scale=scale)
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    for step in range(1, 3):
        grads = _device_normals(shapes, 2337 + step, 1e-3 * scale, torch.bfloat16)
        for p, g in zip(params, grads):
            p.grad = nt.Tensor(g)
        scaler.scale(loss)
        result = nt.amp.fused_step(optimizer, scaler, max_norm=1.0)
        kept = {}

        def fetch(index):
            unscaled = parallel.unscale(pool, _host_bf16(pool, grads[index]), scale, "bfloat16")
            if index in sample:
                kept[index] = unscaled
            return unscaled

        norm = parallel.total_norm_streamed(pool, len(shapes), fetch)
        assert math.isfinite(norm)
        coefficient = oclip.clip_coefficient(1.0, norm)
        assert coefficient < 1
        assert result.finite and result.updated and result.scale == scale
        assert abs(result.norm - norm) <= NORM_RTOL * norm, (step, result.norm, norm)
        for i in sample:
            clipped = parallel.clip_apply(pool, kept[i], coefficient, "bfloat16")
            parallel.master_step(pool, master[i], clipped, m[i], v[i], step, weight_decay=decays[i], **OPTIONS)
        del grads, kept
        _say(f"C5 step {step}: norm {norm:.9g}")
    flips = 0
    for i in sample:
        state = optimizer.state[id(params[i])]
        assert state["step"] == 2
        flips += _compare(f"master[{i}]", state["master"].numpy(), master[i], unit_bits=32, allow_rate=1e-6)
        flips += _compare(f"m[{i}]", state["exp_avg"].numpy(), m[i], unit_bits=32, allow_rate=1e-6)
        flips += _compare(f"v[{i}]", state["exp_avg_sq"].numpy(), v[i], unit_bits=32, allow_rate=1e-6)
        flips += _compare(f"copy[{i}]", params[i].numpy(), lowp.round_bf16(master[i]), unit_bits=16, allow_rate=1e-6)
    _say(f"C5 sample {sample} matches the oracle ({flips} elements one unit away)")
    del params, optimizer, scaler
    _release()


# ---- C4/8 and C5/8: one GPU's share of an 8-way sharded step ------------------------------------------
@pytest.mark.parametrize("config", ["c4s8", "c5s8"])
def test_sharded_slices_fused(pool, config):
    """One rank's slices of an 8-way sharded step (every tensor's flat storage
    cut in eight; the benchmark's C4/8 and C5/8): each slice keeps its
    tensor's weight-decay group.  C4/8 (292 slices, 164 M parameters):
    bfloat16 moments, clip at 1.0, four fused steps.  C5/8 (291 slices, 842 M
    parameters): float32 moments, AMP at 65536 with clip at 1.0, three fused
    steps.  The whole state against the oracle."""
    from namitorch_amd.param_lists import shard_shapes
    full = gpt_1p3b_shapes() if config == "c4s8" else llama7b_shapes()
    shapes = shard_shapes(full, 8)
    amp = config == "c5s8"
    steps = 3 if amp else 4
    assert len(shapes) == len(full) and total_params(shapes) == (164_477_440 if config == "c4s8" else 842_301_952)
    decays = [0.1 if k else 0.0 for k in decay_mask(full)]
    scale = 65536.0 if amp else 1.0
    weights = _device_normals(shapes, 4242, 0.02, torch.bfloat16)
    params = [nt.Parameter(w) for w in weights]
    master = [_host_bf16(pool, w) for w in weights]
    del weights
    m = [np.zeros_like(h) for h in master]
    v = [np.zeros_like(h) for h in master]
    groups = [{"params": [p for p, d in zip(params, decays) if d], "weight_decay": 0.1},
              {"params": [p for p, d in zip(params, decays) if not d], "weight_decay": 0.0}]
    optimizer = nt.optim.AdamW(groups, master_weights=True, state_dtype="bfloat16" if not amp else None, **OPTIONS)
    scaler = nt.GradScaler(init_scale=scale) if amp else None
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    for step in range(1, steps + 1):
        grads = _device_normals(shapes, 5242 + step, 1e-3 * scale, torch.bfloat16)
        for p, g in zip(params, grads):
            p.grad = nt.Tensor(g)
        if amp:
            scaler.scale(loss)
        result = nt.amp.fused_step(optimizer, scaler, max_norm=1.0)
        host = [_host_bf16(pool, g) for g in grads]
        del grads
        if amp:
            host = [parallel.unscale(pool, g, scale, "bfloat16") for g in host]
        norm = parallel.total_norm_streamed(pool, len(host), lambda i: host[i])
        assert math.isfinite(norm)
        coefficient = oclip.clip_coefficient(1.0, norm)
        assert coefficient < 1
        assert result.finite and result.updated
        assert abs(result.norm - norm) <= NORM_RTOL * norm, (step, result.norm, norm)
        if amp:
            assert result.scale == scale
        for i, g in enumerate(host):
            clipped = parallel.clip_apply(pool, g, coefficient, "bfloat16")
            parallel.master_step(pool, master[i], clipped, m[i], v[i], step, weight_decay=decays[i],
                                 state_bf16=not amp, **OPTIONS)
        del host
        _say(f"{config} step {step}: norm {norm:.9g}")
    moment_bits = 32 if amp else 16
    flips = 0
    for i, p in enumerate(params):
        state = optimizer.state[id(p)]
        assert state["step"] == steps
        flips += _compare(f"master[{i}]", state["master"].numpy(), master[i], unit_bits=32, allow_rate=1e-6)
        flips += _compare(f"m[{i}]", state["exp_avg"].numpy(), m[i], unit_bits=moment_bits, allow_rate=1e-6)
        flips += _compare(f"v[{i}]", state["exp_avg_sq"].numpy(), v[i], unit_bits=moment_bits, allow_rate=1e-6)
        flips += _compare(f"copy[{i}]", p.numpy(), lowp.round_bf16(master[i]), unit_bits=16, allow_rate=1e-6)
    _say(f"{config} matches the oracle over every slice ({flips} elements one unit away)")
    del params, optimizer, scaler
    _release()
