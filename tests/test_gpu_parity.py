"""GPU parity: the gfx950 kernels against the oracle and the reference's
golden fixtures.  Every test here needs an MI355X and the built library;
nothing falls back to the CPU.

Bars: bit-identical for float32/float16/float64 AdamW, unscale, found_inf,
skip decisions and the loss-scale sequence; clipped gradients bit-identical
(the clip coefficient comes from a float64 norm whose summation order
differs from NumPy's, so the test allows the norm 1e-12 relative);
model copies and bfloat16 moments bit-identical to RNE of the float32
values.
"""

import json
import math

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd import _native
from oracle import adam as oadam
from oracle import clip as oclip
from oracle import lowp
from oracle import scaler as oscaler

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NORM_RTOL = 1e-12   # float64 norm: fixed device order vs NumPy pairwise order


def _same(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype, (a.shape, b.shape, a.dtype, b.dtype)
    nan = np.isnan(a.astype(np.float64)) & np.isnan(b.astype(np.float64))
    same = (a.view(f"u{a.itemsize}") == b.view(f"u{b.itemsize}")) | nan
    return bool(np.all(same)), int(np.count_nonzero(~same))


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def test_library_is_native_gfx950():
    lib = _native.load()
    count = _native.c_int32()
    _native.check(lib.nt_device_count(_native.ctypes.byref(count)))
    assert count.value >= 1
    buf = _native.ctypes.create_string_buffer(64)
    _native.check(lib.nt_device_arch(0, buf, 64))
    assert buf.value.decode().startswith("gfx950"), buf.value
    assert type(nt.get_backend(DEV)).__name__ == "HIPBackend"


GOLDEN_ADAM = ["adamw_f32", "adamw_f32_maximize", "adamw_f32_lr0", "adamw_f32_wd0", "adamw_f32_defaults",
               "adam_f32_coupled", "adamw_f32_special", "adamw_f16", "adamw_f64"]


@pytest.mark.parametrize("name", GOLDEN_ADAM)
@pytest.mark.parametrize("fused", [None, False])
def test_adam_api_matches_reference_golden(golden_dir, name, fused):
    data = np.load(golden_dir / f"{name}.npz")
    options = json.loads(str(data["options"]))
    if "betas" in options:
        options["betas"] = tuple(options["betas"])
    param = nt.Parameter(data["p0"], device=DEV)
    if name.startswith("adam_"):
        optimizer = nt.optim.Adam([param], **options)
    else:
        optimizer = nt.optim.AdamW([param], fused=fused, **options)
    for grad in data["grads"]:
        param.grad = nt.Tensor(grad, device=DEV)
        optimizer.step()
    state = optimizer.state[id(param)]
    for label, got, want in (("p", param.numpy(), data["p"]), ("m", state["exp_avg"].numpy(), data["m"]),
                             ("v", state["exp_avg_sq"].numpy(), data["v"])):
        ok, bad = _same(got, want)
        assert ok, f"{name} {label}: {bad} elements differ"
    assert state["step"] == int(data["step"])


def test_per_tensor_hook_matches_reference_golden(golden_dir):
    """The reference's backend.adamw.run protocol (nt_adamw_f32)."""
    import torch
    data = np.load(golden_dir / "adamw_f32.npz")
    backend = nt.get_backend(DEV)
    p = torch.from_numpy(data["p0"].copy()).to(DEV)
    m = torch.zeros_like(p)
    v = torch.zeros_like(p)
    assert backend.adamw.supports(p, p.clone(), m, v)
    assert not backend.adamw.supports(p, p, m, v)          # overlapping
    assert not backend.adamw.supports(p.double(), p.double())
    for step, grad in enumerate(data["grads"], start=1):
        g = torch.from_numpy(grad).to(DEV)
        coefficients = oadam.coefficients(np.float32, 3e-4, (0.9, 0.999), 1e-8, 0.1, step)
        assert backend.adamw.run(p, g, m, v, coefficients=coefficients, maximize=False, update_parameter=True)
    assert _same(p.cpu().numpy(), data["p"])[0]
    assert _same(m.cpu().numpy(), data["m"])[0]
    assert _same(v.cpu().numpy(), data["v"])[0]
    empty = torch.empty(0, device=DEV)
    assert backend.adamw.run(empty, empty.clone(), empty.clone(), empty.clone(), coefficients=coefficients,
                             maximize=False, update_parameter=True) is False


def _small_gpt_shapes():
    from namitorch_amd.param_lists import gpt2_shapes
    return gpt2_shapes(vocab=1001, ctx=67, d=72, layers=2)


def _make_params(shapes, dtype, seed=1337, sigma=0.02):
    rng = _rng(seed)
    return [(rng.standard_normal(int(np.prod(s)), dtype=np.float32) * np.float32(sigma)).reshape(s).astype(dtype)
            for s in shapes]


def _make_grads(shapes, step, sigma=1e-3, dtype=np.float32):
    rng = _rng(1337 + 1000 + step)
    return [(rng.standard_normal(int(np.prod(s)), dtype=np.float32) * np.float32(sigma)).reshape(s).astype(dtype)
            for s in shapes]


def _groups(params):
    decay = [p for p in params if p.ndim >= 2]
    rest = [p for p in params if p.ndim < 2]
    return [{"params": decay, "weight_decay": 0.1}, {"params": rest, "weight_decay": 0.0}]


def test_multi_tensor_fp32_gpt_layout_ten_steps():
    """C2 layout at reduced width: 28 tensors, 2 decay groups, odd sizes."""
    shapes = _small_gpt_shapes()
    host = _make_params(shapes, np.float32)
    params = [nt.Parameter(h, device=DEV) for h in host]
    optimizer = nt.optim.AdamW(_groups(params), lr=3e-4, betas=(0.9, 0.999), eps=1e-8)
    ref_p = [h.copy() for h in host]
    ref_m = [np.zeros_like(h) for h in host]
    ref_v = [np.zeros_like(h) for h in host]
    for step in range(1, 11):
        grads = _make_grads(shapes, step)
        for param, grad in zip(params, grads):
            param.grad = nt.Tensor(grad, device=DEV)
        optimizer.step()
        for i, grad in enumerate(grads):
            wd = 0.1 if len(shapes[i]) >= 2 else 0.0
            oadam.adam_step(ref_p[i], grad, ref_m[i], ref_v[i], step, lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd)
    for i, param in enumerate(params):
        state = optimizer.state[id(param)]
        assert _same(param.numpy(), ref_p[i])[0], shapes[i]
        assert _same(state["exp_avg"].numpy(), ref_m[i])[0]
        assert _same(state["exp_avg_sq"].numpy(), ref_v[i])[0]


@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 2047, 2048, 2049, 16383, 16384, 16385, 40000])
def test_adamw_sizes_and_tails(n):
    rng = _rng(n + 5)
    p0 = (rng.standard_normal(n) * 0.1).astype(np.float32)
    param = nt.Parameter(p0, device=DEV)
    optimizer = nt.optim.AdamW([param], lr=1e-3, weight_decay=0.1)
    rp, rm, rv = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for step in range(1, 4):
        g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
        param.grad = nt.Tensor(g, device=DEV)
        optimizer.step()
        oadam.adam_step(rp, g, rm, rv, step, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
    assert _same(param.numpy(), rp)[0]
    assert optimizer.state[id(param)]["step"] == 3
    # fused semantics: no version bump for empty tensors
    assert param._version == (0 if n == 0 else 3)


def test_adamw_unaligned_storage_scalar_path():
    import torch
    base = torch.zeros(4099 + 1, dtype=torch.float32, device=DEV)
    rng = _rng(3)
    p0 = (rng.standard_normal(4099) * 0.1).astype(np.float32)
    view = base[1:]
    view.copy_(torch.from_numpy(p0))
    param = nt.Parameter.__new__(nt.Parameter)
    nt.Tensor._initialize(param, view, True)
    assert param._ptr % 16 != 0
    g = (rng.standard_normal(4099) * 1e-2).astype(np.float32)
    param.grad = nt.Tensor(g, device=DEV)
    optimizer = nt.optim.AdamW([param], lr=1e-3)
    optimizer.step()
    rp, rm, rv = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    oadam.adam_step(rp, g, rm, rv, 1, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2)
    assert _same(param.numpy(), rp)[0]


def test_more_than_sixteen_coefficient_slots():
    """17 parameter groups with distinct lr in one step -> two launches."""
    rng = _rng(17)
    hosts = [(rng.standard_normal(100 + i) * 0.1).astype(np.float32) for i in range(17)]
    params = [nt.Parameter(h, device=DEV) for h in hosts]
    groups = [{"params": [p], "lr": 1e-3 * (i + 1)} for i, p in enumerate(params)]
    optimizer = nt.optim.AdamW(groups)
    grads = [(rng.standard_normal(h.size) * 1e-2).astype(np.float32) for h in hosts]
    for p, g in zip(params, grads):
        p.grad = nt.Tensor(g, device=DEV)
    optimizer.step()
    for i, (p, h, g) in enumerate(zip(params, hosts, grads)):
        rp, rm, rv = h.copy(), np.zeros_like(h), np.zeros_like(h)
        oadam.adam_step(rp, g, rm, rv, 1, lr=1e-3 * (i + 1), betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2)
        assert _same(p.numpy(), rp)[0], i


def test_per_parameter_step_counts_differ():
    """Params whose step counts diverge (one had no grad) use their own bias corrections."""
    rng = _rng(23)
    a0 = (rng.standard_normal(300) * 0.1).astype(np.float32)
    b0 = (rng.standard_normal(301) * 0.1).astype(np.float32)
    a, b = nt.Parameter(a0, device=DEV), nt.Parameter(b0, device=DEV)
    optimizer = nt.optim.AdamW([a, b], lr=1e-3)
    ra, rb = [a0.copy(), np.zeros_like(a0), np.zeros_like(a0)], [b0.copy(), np.zeros_like(b0), np.zeros_like(b0)]
    steps = {"a": 0, "b": 0}
    for k in range(5):
        ga = (rng.standard_normal(300) * 1e-2).astype(np.float32)
        gb = (rng.standard_normal(301) * 1e-2).astype(np.float32)
        a.grad = nt.Tensor(ga, device=DEV)
        b.grad = None if k in (1, 2) else nt.Tensor(gb, device=DEV)
        optimizer.step()
        steps["a"] += 1
        oadam.adam_step(*ra[:1], ga, *ra[1:], steps["a"], lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2)
        if b.grad is not None:
            steps["b"] += 1
            oadam.adam_step(*rb[:1], gb, *rb[1:], steps["b"], lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2)
    assert _same(a.numpy(), ra[0])[0] and _same(b.numpy(), rb[0])[0]
    assert optimizer.state[id(b)]["step"] == 3


# ---- master weights / low precision --------------------------------------------------------
@pytest.mark.parametrize("param_dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("grad_dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("state_dtype", [None, "bfloat16"])
def test_master_weights_match_oracle(param_dtype, grad_dtype, state_dtype):
    shapes = [(67, 33), (33,), (1000,), (5, 7, 9)]
    rng = _rng(99)
    host = [(rng.standard_normal(s) * 0.05).astype(np.float32) for s in shapes]
    host_lp = [lowp.round_bf16(h) if param_dtype == "bfloat16" else h.astype(param_dtype).astype(np.float32) for h in host]
    params = [nt.Parameter(h, dtype=param_dtype, device=DEV) for h in host_lp]
    optimizer = nt.optim.AdamW(params, lr=1e-3, weight_decay=0.1, master_weights=True, state_dtype=state_dtype)
    masters = [h.copy() for h in host_lp]
    ms = [np.zeros_like(h) for h in host_lp]
    vs = [np.zeros_like(h) for h in host_lp]
    for step in range(1, 6):
        for i, (p, s) in enumerate(zip(params, shapes)):
            g32 = (rng.standard_normal(s) * 1e-3).astype(np.float32)
            g = lowp.round_bf16(g32) if grad_dtype == "bfloat16" else g32.astype(grad_dtype).astype(np.float32)
            p.grad = nt.Tensor(g, dtype=grad_dtype, device=DEV)
            oadam.master_step(masters[i], g, ms[i], vs[i], step, lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
                              weight_decay=0.1, state_bf16=state_dtype == "bfloat16")
        optimizer.step()
    for i, p in enumerate(params):
        state = optimizer.state[id(p)]
        assert _same(state["master"].numpy(), masters[i])[0]
        assert _same(state["exp_avg"].numpy(), ms[i])[0]
        assert _same(state["exp_avg_sq"].numpy(), vs[i])[0]
        copy = oadam.copy_out(masters[i], param_dtype)   # float16 array, or float32 values for bf16/fp32
        assert _same(p.numpy(), copy)[0]


# ---- GradScaler / clip -----------------------------------------------------------------------
@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_grad_scaler_sequence_matches_reference_golden(golden_dir, dtype):
    golden = json.loads((golden_dir / "golden.json").read_text())["scaler"][f"scaler_{dtype}"]
    arrays = np.load(golden_dir / "scaler.npz")
    name = f"scaler_{dtype}"
    param = nt.Parameter(arrays[f"{name}_p0"], device=DEV)
    optimizer = nt.optim.AdamW([param], lr=1e-3, betas=(0.9, 0.999), eps=golden["eps"], weight_decay=0.1)
    scaler = nt.GradScaler(init_scale=65536.0, growth_interval=3)
    for k, grad in enumerate(arrays[f"{name}_grads"]):
        scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
        param.grad = nt.Tensor(grad, device=DEV)
        finite = scaler.unscale_(optimizer)
        norm = nt.optim.clip_grad_norm_([param], 1.0, error_if_nonfinite=True).item() if finite else None
        updated = scaler.step(optimizer)
        scaler.update()
        assert finite == golden["finite"][k] and updated == golden["updated"][k]
        assert scaler.get_scale() == golden["scale"][k]
        if norm is not None:
            assert abs(norm - golden["norm"][k]) <= NORM_RTOL * golden["norm"][k]
    state = optimizer.state[id(param)]
    assert state["step"] == golden["step"]
    assert _same(param.numpy(), arrays[f"{name}_p"])[0]
    assert _same(state["exp_avg"].numpy(), arrays[f"{name}_m"])[0]
    assert _same(state["exp_avg_sq"].numpy(), arrays[f"{name}_v"])[0]


def test_unscaled_grads_visible_in_place():
    rng = _rng(41)
    g = (rng.standard_normal(5001) * 70).astype(np.float16)
    param = nt.Parameter(np.zeros(5001, dtype=np.float16), device=DEV)
    optimizer = nt.optim.AdamW([param], eps=1e-4)
    scaler = nt.GradScaler(init_scale=3000.0)
    scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
    param.grad = nt.Tensor(g, device=DEV)
    version = param.grad._version
    assert scaler.unscale_(optimizer)
    assert param.grad._version == version + 1
    assert _same(param.grad.numpy(), oscaler.unscale(g, 3000.0))[0]


def _bits(array: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(array).view({2: np.uint16, 4: np.uint32}[array.dtype.itemsize])


@pytest.mark.parametrize("scale", [65536.0, 3.0])
def test_float16_signed_zeros_match_numpy(scale):
    """Every float16 result is its float32 operation rounded once, -0 included
    (NumPy's float16 arithmetic).  Products that are -0 (0 x negative, and
    negative values that unscale below the smallest float16 subnormal) stay
    -0 in the unscaled gradients read back, in the float16 AdamW update
    (beta1 = 0, maximize: m = 0*m + 1*(-g)) and in the float32-master pass
    that unscales float16 gradients itself."""
    n = 4099
    g = np.zeros(n, dtype=np.float16)
    g[1::4] = np.float16(-0.0)
    g[2::4] = np.float16(-6e-8)                  # the smallest float16 subnormal, negative
    g[3::4] = (_rng(3).standard_normal(n)[3::4] * 1e-3).astype(np.float16)
    # Unscaled in place and read back.
    param = nt.Parameter(np.zeros(n, dtype=np.float16), device=DEV)
    optimizer = nt.optim.AdamW([param], eps=1e-4)
    scaler = nt.GradScaler(init_scale=scale)
    scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
    param.grad = nt.Tensor(g, device=DEV)
    assert scaler.unscale_(optimizer)
    want = oscaler.unscale(g, scale, "float16")
    assert np.signbit(want).sum() > n // 4
    assert np.array_equal(_bits(param.grad.numpy()), _bits(want))
    # float16 AdamW steps whose moments are -0 where the gradient is 0.
    p0 = (_rng(4).standard_normal(n) * 0.02).astype(np.float16)
    grads = [(_rng(5 + k).standard_normal(n) * 1e-2).astype(np.float16) for k in range(2)]
    grads[1][::3] = np.float16(0.0)
    param = nt.Parameter(p0, device=DEV)
    options = dict(lr=1e-3, betas=(0.0, 0.95), eps=1e-4, weight_decay=0.0, maximize=True)
    optimizer = nt.optim.AdamW([param], **options)
    ref_p, ref_m, ref_v = p0.copy(), np.zeros(n, np.float16), np.zeros(n, np.float16)
    for step, grad in enumerate(grads, start=1):
        param.grad = nt.Tensor(grad, device=DEV)
        optimizer.step()
        oadam.adam_step(ref_p, grad, ref_m, ref_v, step, **options)
    state = optimizer.state[id(param)]
    assert np.signbit(ref_m[::3]).sum() > 0
    assert np.array_equal(_bits(state["exp_avg"].numpy()), _bits(ref_m))
    assert np.array_equal(_bits(state["exp_avg_sq"].numpy()), _bits(ref_v))
    assert np.array_equal(_bits(param.numpy()), _bits(ref_p))
    # The float32-master pass unscales the float16 gradient itself (fused
    # path): after a first step leaves negative moments, the unscaled +0 and
    # -0 of the second step's gradient give m = -0 and +0 respectively.
    bf = nt.Parameter(lowp.round_bf16(p0.astype(np.float32)), dtype="bfloat16", device=DEV)
    optimizer = nt.optim.AdamW([bf], master_weights=True, **options)
    scaler = nt.GradScaler(init_scale=scale, growth_interval=1000)
    master = lowp.round_bf16(p0.astype(np.float32))
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    first = (grads[0].astype(np.float32) * np.float32(scale)).astype(np.float16)
    for step, stored in enumerate((first, g), start=1):
        scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
        bf.grad = nt.Tensor(stored, device=DEV)
        assert nt.amp.fused_step(optimizer, scaler).updated
        unscaled = oscaler.unscale(stored, scale, "float16")
        oadam.master_step(master, unscaled.astype(np.float32), m, v, step, **options)
    assert (np.signbit(m) & (m == 0)).sum() > 0 and ((~np.signbit(m)) & (m == 0)).sum() > 0
    state = optimizer.state[id(bf)]
    assert np.array_equal(_bits(state["exp_avg"].numpy()), _bits(m))
    assert np.array_equal(_bits(state["exp_avg_sq"].numpy()), _bits(v))
    assert np.array_equal(_bits(state["master"].numpy()), _bits(master))


def test_unscale_overflow_to_inf_in_grad_dtype():
    """scale < 1: finite float16 grads overflow after division -> found_inf."""
    param = nt.Parameter(np.zeros(10, dtype=np.float16), device=DEV)
    optimizer = nt.optim.AdamW([param], eps=1e-4)
    scaler = nt.GradScaler(init_scale=0.5)
    scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
    g = np.full(10, 1.0, dtype=np.float16)
    g[3] = 60000.0
    param.grad = nt.Tensor(g, device=DEV)
    assert scaler.unscale_(optimizer) is False
    assert scaler.step(optimizer) is False
    scaler.update()
    assert scaler.get_scale() == 0.25
    assert np.array_equal(param.numpy(), np.zeros(10, dtype=np.float16))


def test_clip_matches_reference_golden(golden_dir):
    data = np.load(golden_dir / "clip.npz")
    records = json.loads((golden_dir / "golden.json").read_text())["clip"]
    for record in records:
        key = record["key"]
        if record["count"] == 0:
            continue
        grads = [data[f"{key}_in{i}"] for i in range(record["count"])]
        params = [nt.Parameter(np.zeros(g.shape, dtype=g.dtype), device=DEV) for g in grads]
        for p, g in zip(params, grads):
            p.grad = nt.Tensor(g, device=DEV)
        norm = nt.optim.clip_grad_norm_(params, record["max_norm"], norm_type=record["norm_type"]).item()
        want = record["norm"]
        assert (math.isnan(norm) and math.isnan(want)) or norm == want or abs(norm - want) <= NORM_RTOL * abs(want), key
        for i, p in enumerate(params):
            ok, bad = _same(p.grad.numpy(), data[f"{key}_out{i}"])
            assert ok, f"{key}[{i}]: {bad} differ"


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_clip_single_rounding_from_float64(dtype):
    rng = _rng(57)
    g32 = (rng.standard_normal(20001) * 3).astype(np.float32)
    g = lowp.round_bf16(g32) if dtype == "bfloat16" else g32.astype(dtype).astype(np.float32)
    param = nt.Parameter(np.zeros(g.shape, dtype=np.float32), dtype=dtype, device=DEV)
    param.grad = nt.Tensor(g, dtype=dtype, device=DEV)
    norm = nt.optim.clip_grad_norm_([param], 1.0).item()
    want = oclip.total_norm([g.astype(np.float64)])
    assert abs(norm - want) <= NORM_RTOL * want
    coefficient = oclip.clip_coefficient(1.0, norm)
    expected = oclip.clip_apply(g.astype(np.float64), coefficient, dtype)
    got = param.grad.numpy()      # float16 array, or float32 values for bf16/fp32
    assert _same(got, expected)[0]


# ---- device-decided step (fused_step) ---------------------------------------------------------
def _run_sequence(mode, shapes, param_dtype, grad_dtype, state_dtype, amp, max_norm, inf_step, steps=6):
    rng = _rng(71)
    host = [(rng.standard_normal(s) * 0.05).astype(np.float32) for s in shapes]
    params = [nt.Parameter(lowp.round_bf16(h) if param_dtype == "bfloat16" else h, dtype=param_dtype, device=DEV)
              for h in host]
    optimizer = nt.optim.AdamW(params, lr=1e-3, weight_decay=0.1, master_weights=True, state_dtype=state_dtype)
    scaler = nt.GradScaler(init_scale=65536.0, growth_interval=2) if amp else None
    grng = _rng(72)
    trace = []
    for k in range(steps):
        scale = 65536.0 if amp else 1.0
        grads = [(grng.standard_normal(s) * 1e-3 * scale).astype(np.float32) for s in shapes]
        if k == inf_step:
            grads[-1].reshape(-1)[7] = np.inf
        for p, g in zip(params, grads):
            p.grad = nt.Tensor(g, dtype=grad_dtype, device=DEV)
        if amp:
            scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
        if mode == "api":
            if amp:
                finite = scaler.unscale_(optimizer)
                if finite and max_norm is not None:
                    nt.optim.clip_grad_norm_(params, max_norm)
                updated = scaler.step(optimizer)
                scaler.update()
            else:
                if max_norm is not None:
                    nt.optim.clip_grad_norm_(params, max_norm)
                optimizer.step()
                updated = True
        else:
            result = nt.amp.fused_step(optimizer, scaler, max_norm=max_norm)
            updated = result.updated
        trace.append((updated, scaler.get_scale() if amp else 1.0,
                      [p.grad.numpy() for p in params], [p.grad._version for p in params]))
    state = [optimizer.state[id(p)] for p in params]
    final = dict(params=[p.numpy() for p in params], master=[s["master"].numpy() for s in state],
                 m=[s["exp_avg"].numpy() for s in state], v=[s["exp_avg_sq"].numpy() for s in state],
                 step=[s["step"] for s in state], versions=[(p._version, s["exp_avg"]._version) for p, s in zip(params, state)])
    return trace, final


@pytest.mark.parametrize("config", [
    dict(param_dtype="bfloat16", grad_dtype="float16", state_dtype=None, amp=True, max_norm=None, inf_step=2),     # C3-like
    dict(param_dtype="bfloat16", grad_dtype="bfloat16", state_dtype="bfloat16", amp=False, max_norm=0.01, inf_step=-1),  # C4-like
    dict(param_dtype="bfloat16", grad_dtype="bfloat16", state_dtype=None, amp=True, max_norm=0.01, inf_step=3),   # C5-like
    dict(param_dtype="float32", grad_dtype="float32", state_dtype=None, amp=True, max_norm=1e6, inf_step=1),
])
def test_fused_step_matches_api_sequence(config):
    shapes = [(301, 17), (17,), (4099,)]
    api_trace, api_final = _run_sequence("api", shapes, **config)
    dev_trace, dev_final = _run_sequence("fused", shapes, **config)
    for k, (a, d) in enumerate(zip(api_trace, dev_trace)):
        assert a[0] == d[0] and a[1] == d[1], (k, a[:2], d[:2])
        for ga, gd in zip(a[2], d[2]):
            assert _same(ga, gd)[0], k
        assert a[3] == d[3], (k, a[3], d[3])
    for key in ("params", "master", "m", "v"):
        for x, y in zip(api_final[key], dev_final[key]):
            assert _same(x, y)[0], key
    assert api_final["step"] == dev_final["step"]
    assert api_final["versions"] == dev_final["versions"]
    if config["inf_step"] >= 0:
        assert not api_trace[config["inf_step"]][0]


@pytest.mark.parametrize("scale", [None, 65536.0, 1.0, 3.0, 2.0 ** 30])
@pytest.mark.parametrize("magnitude", ["normal", "tiny", "subnormal", "nonfinite", "nan"])
def test_fp16_grad_norm_paths(scale, magnitude):
    """Pre-pass exactness on float16 gradients, which are unscaled and
    rounded element by element: unscaled values that land in the float16
    subnormal range, float16 subnormal inputs, values that overflow to inf
    on storage and NaN give the oracle's norm and found_inf, with no scale,
    a power-of-two scale whose inverse is a float16 value (65536, 1: the
    packed float16 path), one whose inverse is not (2**30), and any other
    scale."""
    rng = _rng(93)
    n = 70001
    g32 = (rng.standard_normal(n) * 4.0).astype(np.float32)
    if magnitude == "tiny":
        g32[::991] *= np.float32(1e-4)          # unscaled by 65536: float16 subnormals
    elif magnitude == "subnormal":
        g32[5] = np.float32(3e-7)               # float16 subnormal inputs
        g32[60000] = np.float32(-1e-6)
    elif magnitude == "nonfinite":
        g32[77] = np.inf
        g32[4099] = np.float32(7e4)             # overflows float16 on storage
    elif magnitude == "nan":
        g32[8200] = np.nan
        g32[9000] = -np.inf
    g = g32.astype(np.float16)
    param = nt.Parameter(np.zeros(n, dtype=np.float32), dtype="float16", device=DEV)
    param.grad = nt.Tensor(g, dtype="float16", device=DEV)
    if scale is None:
        norm = nt.optim.clip_grad_norm_([param], 1e30).item()
        want = oclip.total_norm([g.astype(np.float64)])
    else:
        optimizer = nt.optim.AdamW([param], master_weights=True)
        scaler = nt.GradScaler(init_scale=scale)
        scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
        finite = scaler.unscale_(optimizer)
        unscaled = oscaler.unscale(g, scale, "float16")
        assert finite == oscaler.finite([unscaled])
        norm = nt.optim.clip_grad_norm_([param], 1e30).item()
        want = oclip.total_norm([unscaled.astype(np.float64)])
    if math.isfinite(want):
        assert abs(norm - want) <= NORM_RTOL * want, (norm, want)
    else:
        assert (math.isnan(norm) and math.isnan(want)) or norm == want, (norm, want)


@pytest.mark.parametrize("scale", [None, 65536.0, 3.0])
@pytest.mark.parametrize("magnitude", ["normal", "huge", "tiny", "subnormal"])
def test_bf16_grad_norm_paths(scale, magnitude):
    """Pre-pass exactness: the raw-square fast path, its per-workgroup range
    check and the element-by-element fallback all give the oracle's norm and
    found_inf on bfloat16 gradients."""
    rng = _rng(91)
    n = 70001
    g32 = (rng.standard_normal(n) * 0.5).astype(np.float32)
    if magnitude == "huge":
        g32[::997] *= np.float32(3e25)
    elif magnitude == "tiny":
        g32[::991] *= np.float32(1e-25)
    elif magnitude == "subnormal":
        g32[5] = np.float32(1e-39)
        g32[60000] = np.float32(-5e-40)
    g = lowp.round_bf16(g32)
    param = nt.Parameter(np.zeros(n, dtype=np.float32), dtype="bfloat16", device=DEV)
    param.grad = nt.Tensor(g, dtype="bfloat16", device=DEV)
    if scale is None:
        norm = nt.optim.clip_grad_norm_([param], 1e30).item()
        want = oclip.total_norm([g.astype(np.float64)])
    else:
        optimizer = nt.optim.AdamW([param], master_weights=True)
        scaler = nt.GradScaler(init_scale=scale)
        scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
        finite = scaler.unscale_(optimizer)
        unscaled = oscaler.unscale(g, scale, "bfloat16")
        assert finite == oscaler.finite([unscaled])
        norm = nt.optim.clip_grad_norm_([param], 1e30).item()
        want = oclip.total_norm([unscaled.astype(np.float64)])
    assert abs(norm - want) <= NORM_RTOL * want, (norm, want)


@pytest.mark.parametrize("edit", ["new_gradient", "gradient_requires_grad", "parameter_frozen", "gradient_to_none",
                                  "inf_written"])
def test_scaler_step_checks_edits_after_unscale(edit):
    """GradScaler.step after unscale_ (amp.py:196-217): a replaced, removed
    or re-attached gradient, or a frozen parameter, raises the reference's
    error before anything is stepped; a gradient rewritten in place (here
    with an inf) is checked for finiteness again and skips the step, so the
    scale backs off."""
    import re
    params = [nt.Parameter(np.full(300, 0.5, np.float32), device=DEV) for _ in range(3)]
    for p in params:
        p.grad = nt.Tensor(np.full(300, 1e-2 * 1024, np.float32), device=DEV)
    optimizer = nt.optim.AdamW(params, lr=1e-3)
    scaler = nt.GradScaler(init_scale=1024.0)
    scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
    assert scaler.unscale_(optimizer) is True
    before = [p.numpy().copy() for p in params]
    changed = re.escape("Optimizer gradients changed after unscale_; clipping must modify the existing gradients in-place.")
    if edit == "new_gradient":
        params[1].grad = nt.Tensor(np.full(300, 1e-2, np.float32), device=DEV)
        with pytest.raises(RuntimeError, match=changed):
            scaler.step(optimizer)
    elif edit == "gradient_requires_grad":
        params[1].grad.requires_grad = True
        with pytest.raises(RuntimeError, match=re.escape("GradScaler requires detached floating gradients.")):
            scaler.step(optimizer)
    elif edit == "parameter_frozen":
        params[2].requires_grad = False
        with pytest.raises(RuntimeError, match=changed):
            scaler.step(optimizer)
    elif edit == "gradient_to_none":
        params[0].grad = None
        with pytest.raises(RuntimeError, match=changed):
            scaler.step(optimizer)
    else:
        params[1].grad[...] = nt.Tensor(np.full(300, np.inf, np.float32), device=DEV)
        assert scaler.step(optimizer) is False
        scaler.update()
        assert scaler.get_scale() == 512.0
    for p, b in zip(params, before):
        assert np.array_equal(p.numpy(), b)
    assert all(optimizer.state.get(id(p), {}).get("step", 0) == 0 for p in params)
