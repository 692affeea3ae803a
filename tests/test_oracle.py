"""Pins of the CPU oracle (no GPU).

Each oracle function is checked against something other than itself:
golden fixtures written by the reference's own code (tests/golden), closed
forms, invariants, library routines (torch's RNE bfloat16 conversion,
math.fsum) or exact rational arithmetic.
"""

import json
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import adam, arith, clip, grads, lowp, scaler

GOLDEN_CASES = ["adamw_f32", "adamw_f32_maximize", "adamw_f32_lr0", "adamw_f32_wd0", "adamw_f32_defaults",
                "adam_f32_coupled", "adamw_f32_bfgrads", "adamw_f32_special", "adamw_f16", "adamw_f64"]


def _load(golden_dir, name):
    data = np.load(golden_dir / f"{name}.npz")
    options = json.loads(str(data["options"]))
    return data, options


def run_oracle(data, options, decoupled=True):
    p = data["p0"].copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    full = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2, maximize=False)
    full.update(options)
    full["betas"] = tuple(full["betas"])
    for step, grad in enumerate(data["grads"], start=1):
        adam.adam_step(p, grad, m, v, step, decoupled=decoupled, **full)
    return p, m, v


def _same(a, b):
    """Bit-identical up to NaN payloads."""
    a = np.asarray(a)
    b = np.asarray(b)
    nan = np.isnan(a.astype(np.float64)) & np.isnan(b.astype(np.float64))
    return bool(np.all((a.view(f"u{a.itemsize}") == b.view(f"u{b.itemsize}")) | nan))


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_adam_oracle_matches_reference_golden(golden_dir, name):
    data, options = _load(golden_dir, name)
    p, m, v = run_oracle(data, options, decoupled=not name.startswith("adam_"))
    assert _same(p, data["p"]) and _same(m, data["m"]) and _same(v, data["v"])
    assert int(data["step"]) == len(data["grads"])


def test_adam_oracle_step1_closed_form():
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(10000) * 1e-3).astype(np.float32)
    p = np.zeros_like(g)
    m = np.zeros_like(g)
    v = np.zeros_like(g)
    adam.adam_step(p, g, m, v, 1, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0)
    expected = -1e-3 * g.astype(np.float64) / (np.abs(g.astype(np.float64)) + 1e-8)
    assert np.allclose(p, expected, rtol=2e-6, atol=0)
    assert np.allclose(m, 0.1 * g.astype(np.float64), rtol=1e-6)
    assert np.allclose(v, 0.001 * g.astype(np.float64) ** 2, rtol=1e-6)


def test_adam_oracle_zero_gradient_leaves_params_and_decays_moments():
    p = np.linspace(-1, 1, 257, dtype=np.float32)
    m = np.full_like(p, 0.5)
    v = np.full_like(p, 0.25)
    before = p.copy()
    adam.adam_step(p, np.zeros_like(p), m, v, 3, lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0)
    # m/bc1 and sqrt(v/bc2) are nonzero, so the update is not zero; check the moments exactly
    assert np.all(m == np.float32(0.9) * np.float32(0.5))
    assert np.all(v == np.float32(0.999) * np.float32(0.25))
    p2 = before.copy()
    m2 = np.zeros_like(p2)
    v2 = np.zeros_like(p2)
    adam.adam_step(p2, np.zeros_like(p2), m2, v2, 1, lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0)
    assert np.array_equal(p2, before)


def test_adam_oracle_within_float64_bound_over_ten_steps():
    rng = np.random.default_rng(9)
    p0 = (rng.standard_normal(5000) * 0.02).astype(np.float32)
    grads = [(rng.standard_normal(5000) * 1e-3).astype(np.float32) for _ in range(10)]
    p = p0.copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for step, grad in enumerate(grads, start=1):
        adam.adam_step(p, grad, m, v, step, lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
    p64, m64, v64 = adam.adam_f64_reference(p0, grads, lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
    # float32 rounding of p (|p| < 0.1, three rounded operations per step)
    # bounds the drift from the exact recurrence by ~1e-8 over 10 steps; a
    # dropped or wrong term moves p by O(lr) = 3e-4.
    assert np.max(np.abs(p - p64)) < 1e-7
    assert np.max(np.abs(m - m64)) < 1e-9


def test_adam_oracle_op_order_is_observable():
    """A transposed operand order changes float32 bits, so the golden match
    above really pins the order: (c2*g)*g differs from c2*(g*g) here."""
    g = np.float32(1.1920929e-07) * np.arange(1, 2000, dtype=np.float32) + np.float32(0.3)
    c2 = np.float32(1 - 0.999)
    assert np.any((c2 * g) * g != c2 * (g * g))


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    values = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * np.float32(3.0),
        (np.arange(0, 65536, dtype=np.uint32) << 16 | 0x8000).view(np.float32),   # exact ties
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-40, -1e-44], dtype=np.float32),
    ])
    finite = np.isfinite(values)
    ours = lowp.f32_to_bf16(values)
    ref = torch.from_numpy(values.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours[finite], ref[finite])


def test_bf16_roundtrip_all_patterns():
    bits = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    values = lowp.bf16_to_f32(bits)
    back = lowp.f32_to_bf16(values)
    keep = ~np.isnan(values)
    assert np.array_equal(back[keep], bits[keep])
    assert np.all(np.isnan(lowp.bf16_to_f32(back[~keep])))


def _exact_bf16(value: float) -> int:
    """Nearest bfloat16 by exact rational comparison (ties to even)."""
    target = Fraction(value)
    best = None
    sign = 0x8000 if value < 0 else 0
    magnitude = abs(target)
    lo_bits = int(np.array([abs(value)], dtype=np.float32).view(np.uint32)[0]) >> 16
    candidates = [c for c in range(max(0, lo_bits - 2), min(0x7F80, lo_bits + 3))]
    for bits in candidates:
        candidate = Fraction(float(lowp.bf16_to_f32(np.array([bits], dtype=np.uint16))[0]))
        distance = abs(candidate - magnitude)
        key = (distance, bits % 2)
        if best is None or key < best[0]:
            best = (key, bits)
    return sign | best[1]


def test_f64_to_bf16_single_rounding_exact():
    rng = np.random.default_rng(3)
    values = rng.standard_normal(3000) * np.exp(rng.uniform(-60, 60, 3000))
    # ties at float64 precision: midpoints of neighbouring bf16 values
    bits = np.arange(0x3F00, 0x3F40, dtype=np.uint16)
    lo = lowp.bf16_to_f32(bits).astype(np.float64)
    hi = lowp.bf16_to_f32(bits + 1).astype(np.float64)
    ties = (lo + hi) / 2
    values = np.concatenate([values, ties, -ties])
    ours = lowp.f64_to_bf16(values)
    for value, got in zip(values, ours):
        assert got == _exact_bf16(float(value)), value


def test_f64_to_bf16_differs_from_double_rounding():
    """Values where f64->f32->bf16 double rounding is wrong (pins the single rounding)."""
    one = 1.0
    ulp_bf16 = 2.0 ** -7
    value = one + ulp_bf16 / 2 + 2.0 ** -40   # just above a tie; f32 rounding lands on the tie
    assert float(np.float32(value)) == one + ulp_bf16 / 2
    bits = lowp.f64_to_bf16(np.array([value]))[0]
    assert lowp.bf16_to_f32(np.array([bits], dtype=np.uint16))[0] == np.float32(one + ulp_bf16)


def test_clip_oracle_matches_reference_golden(golden_dir):
    data = np.load(golden_dir / "clip.npz")
    records = json.loads((golden_dir / "golden.json").read_text())["clip"]
    for record in records:
        if record["count"] == 0:
            continue
        key = record["key"]
        grads = [data[f"{key}_in{i}"] for i in range(record["count"])]
        norm, clipped = clip.clip_grad_norm(grads, record["max_norm"], record["norm_type"])
        assert (math.isnan(norm) and math.isnan(record["norm"])) or norm == record["norm"], key
        for index, out in enumerate(clipped):
            assert _same(out, data[f"{key}_out{index}"]), (key, index)


def test_clip_oracle_l2_norm_against_fsum():
    rng = np.random.default_rng(4)
    grads = [rng.standard_normal(n).astype(np.float32) for n in (1, 17, 1000, 4096)]
    exact = math.sqrt(math.fsum(float(x) ** 2 for g in grads for x in g.astype(np.float64)))
    assert abs(clip.total_norm(grads, 2.0) - exact) <= 1e-13 * exact
    assert clip.total_norm(grads, float("inf")) == max(float(np.max(np.abs(g))) for g in grads)
    one = math.fsum(abs(float(x)) for g in grads for x in g)
    assert abs(clip.total_norm(grads, 1.0) - one) <= 1e-12 * one


def test_clip_oracle_special_cases():
    zeros = [np.zeros(5, dtype=np.float32)]
    assert clip.total_norm(zeros) == 0.0
    assert clip.total_norm([np.array([1.0, np.inf], dtype=np.float32)]) == math.inf
    assert math.isnan(clip.total_norm([np.array([np.inf, np.nan], dtype=np.float32)]))
    grads = [np.array([0.1, -0.2], dtype=np.float32)]
    norm, out = clip.clip_grad_norm(grads, 10.0)
    assert _same(out[0], grads[0])


def test_scaler_oracle_matches_reference_golden(golden_dir):
    golden = json.loads((golden_dir / "golden.json").read_text())["scaler"]
    arrays = np.load(golden_dir / "scaler.npz")
    for dtype in ("float32", "float16"):
        name = f"scaler_{dtype}"
        record = golden[name]
        sc = scaler.Scaler(65536.0, growth_interval=3)
        p = arrays[f"{name}_p0"].copy()
        m = np.zeros_like(p)
        v = np.zeros_like(p)
        step = 0
        for k, scaled in enumerate(arrays[f"{name}_grads"]):
            assert sc.scale == (65536.0 if k == 0 else record["scale"][k - 1])
            g = scaler.unscale(scaled, sc.scale)
            finite = scaler.finite([g])
            assert finite == record["finite"][k]
            if finite:
                norm, (g,) = clip.clip_grad_norm([g], 1.0)
                assert norm == record["norm"][k]
                step += 1
                adam.adam_step(p, g, m, v, step, lr=1e-3, betas=(0.9, 0.999), eps=record["eps"], weight_decay=0.1)
            sc.update(not finite)
            assert sc.scale == record["scale"][k]
        assert step == record["step"]
        assert _same(p, arrays[f"{name}_p"]) and _same(m, arrays[f"{name}_m"]) and _same(v, arrays[f"{name}_v"])


def test_scaler_oracle_sequence_closed_form(golden_dir):
    record = json.loads((golden_dir / "golden.json").read_text())["scaler"]["scale_sequence"]
    sc = scaler.Scaler(record["init"], record["growth"], record["backoff"], record["interval"])
    expected, s, tracker = [], record["init"], 0
    for overflow in record["pattern"]:
        sc.update(overflow)
        if overflow:
            s, tracker = max(s * record["backoff"], float(np.finfo(np.float32).tiny)), 0
        else:
            tracker += 1
            if tracker == record["interval"]:
                s, tracker = min(s * record["growth"], float(np.finfo(np.float32).max)), 0
        expected.append(float(np.float32(s)))
        assert sc.scale == expected[-1]
    assert expected == record["scale"]


def test_unscale_oracle_exactness():
    rng = np.random.default_rng(8)
    g = (rng.standard_normal(10000) * 60).astype(np.float16)
    assert np.array_equal(scaler.unscale(g, 65536.0), (g.astype(np.float32) * np.float32(2.0 ** -16)).astype(np.float16))
    odd = 3000.0
    q = scaler.unscale(g.astype(np.float32), odd)
    exact = np.array([float(np.float32(float(x) / odd)) for x in g.astype(np.float32)], dtype=np.float32)
    assert np.array_equal(q, exact)


ACCUMULATE_KEYS = [f"{leaf}_{incoming}" for leaf in ("float32", "float16", "float64")
                   for incoming in ("float16", "float32", "float64")]


@pytest.mark.parametrize("key", ACCUMULATE_KEYS)
def test_accumulate_oracle_matches_reference_golden(golden_dir, key):
    data = np.load(golden_dir / "accumulate.npz")
    leaf = key.split("_")[0]
    added = grads.accumulate(data[f"{key}_existing"], data[f"{key}_incoming"], leaf)
    fresh = grads.accumulate(None, data[f"{key}_incoming"], leaf)
    assert added.dtype == data[f"{key}_added"].dtype and fresh.dtype == data[f"{key}_fresh"].dtype
    assert added.tobytes() == data[f"{key}_added"].tobytes()
    assert fresh.tobytes() == data[f"{key}_fresh"].tobytes()


def test_accumulate_oracle_bf16_against_torch_and_exact_sums():
    rng = np.random.default_rng(17)
    existing = lowp.round_bf16((rng.standard_normal(5000) * 10.0).astype(np.float32))
    incoming = (rng.standard_normal(5000) * np.float32(rng.choice([1e-3, 1.0, 1e3], 5000))).astype(np.float32)
    got = grads.accumulate(existing, incoming, "bfloat16")
    # torch: cast the incoming to bfloat16 (RNE), add in float32, round once.
    t_in = torch.from_numpy(incoming).to(torch.bfloat16).to(torch.float32)
    want = (torch.from_numpy(existing) + t_in).to(torch.bfloat16).to(torch.float32).numpy()
    assert got.tobytes() == want.tobytes()
    # Exponents within 15 of each other: the float32 sum of two bfloat16 values is exact.
    a = lowp.round_bf16(np.float32([1.5, -3.0, 1024.0]))
    b = lowp.round_bf16(np.float32([2.0 ** -10, 0.75, -1.0 / 32]))
    exact = a.astype(np.float64) + b.astype(np.float64)
    assert np.array_equal((a + b).astype(np.float64), exact)
    assert grads.accumulate(None, incoming, "bfloat16").tobytes() == t_in.numpy().tobytes()


# ---- Tensor-by-scalar arithmetic (GradScaler.scale, loss / accum) -------------------------
SCALAR_OPERANDS = {"int3": 3, "int7": 7, "int1000": 1000, "float3": 3.0, "float0.1": 0.1,
                   "f16_3": np.float16(3.0), "f64_3": np.float64(3.0), "f64_0.1": np.float64(0.1)}


def scalar_fixture_cases(data):
    """(key, loss, operand, op) for every entry of scalar_ops.npz."""
    cases = []
    for key in sorted(data):
        if key.endswith("_loss"):
            continue
        dtype, op, label = key.split("_", 2)
        if op == "scale":
            operand = float(label)
            op = "mul"
        else:
            operand = SCALAR_OPERANDS[label]
        cases.append((key, data[f"{dtype}_loss"], operand, op))
    return cases


def test_scalar_oracle_matches_reference_golden(golden_dir):
    data = np.load(golden_dir / "scalar_ops.npz")
    cases = scalar_fixture_cases(data)
    assert len(cases) == 39
    for key, loss, operand, op in cases:
        got = arith.scalar_op(loss, operand, op)
        assert got.dtype == data[key].dtype, key
        assert got.tobytes() == data[key].tobytes(), key


def test_scalar_oracle_promotion_closed_form():
    """float16 loss times the loss scale is float32 and exact for powers of
    two; division is IEEE true division in the promoted dtype."""
    loss = np.float16([3.0, -2.5, 65504.0, 1e-5])
    scaled = arith.scale_loss(loss, 65536.0)
    assert scaled.dtype == np.float32
    assert np.array_equal(scaled, loss.astype(np.float32) * np.float32(65536.0))
    assert np.isfinite(scaled).all()                   # float16 itself would overflow
    q = arith.scalar_op(np.float32([1.0, 2.0, 10.0]), 3, "div")
    assert [float(x) for x in q] == [float(np.float32(Fraction(n, 3))) for n in (1, 2, 10)]


# ---- float64 gradient norms whose squares leave the float64 range -------------------------
def test_clip_oracle_float64_extremes_match_reference_golden(golden_dir):
    data = np.load(golden_dir / "clip_f64.npz")
    records = json.loads(str(data["records"]))
    assert len(records) == 6
    for record in records:
        key = record["key"]
        grads = [data[f"{key}_in{i}"] for i in range(record["count"])]
        with np.errstate(under="ignore"):
            norm, clipped = clip.clip_grad_norm(grads, record["max_norm"], record["norm_type"])
        assert norm == record["norm"], key
        for i, g in enumerate(clipped):
            assert g.tobytes() == data[f"{key}_out{i}"].tobytes(), (key, i)


def test_clip_float64_direct_sum_fails_where_prescale_is_needed(golden_dir):
    """The reference's max-abs prescale matters for float64: sqrt(sum g^2)
    overflows at |g| ~ 1e200 and underflows at 1e-200, while the prescaled
    norm is finite and positive (the device switches to the prescaled pass
    there)."""
    data = np.load(golden_dir / "clip_f64.npz")
    for key, bad in (("clip64_huge_2", math.inf), ("clip64_tiny_2", 0.0)):
        grads = [data[f"{key}_in{i}"] for i in range(3)]
        with np.errstate(over="ignore", under="ignore"):
            direct = math.sqrt(sum(float(np.sum(g * g)) for g in grads))
        assert direct == bad
        assert 0 < clip.total_norm(grads) < math.inf


def test_clip_norm_formulations_round_differently():
    """sqrt(sum g^2) and the reference's amax*power(sum (g/amax)^2, 0.5) are
    different roundings of the same real number: on ordinary data they differ
    in the last bits but stay within 1e-12 relative, the tolerance the device
    norm is held to."""
    rng = np.random.default_rng(5)
    differ = 0
    for trial in range(200):
        grads = [(rng.standard_normal(int(rng.integers(1, 400))) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32)
                 for _ in range(3)]
        direct = math.sqrt(sum(float(np.sum(g.astype(np.float64) ** 2)) for g in grads))
        reference = clip.total_norm(grads)
        differ += direct != reference
        assert abs(direct - reference) <= 1e-12 * reference
    assert differ > 0


# ---- chunked evaluation (oracle.parallel) -----------------------------------------------
def test_parallel_oracle_equals_plain_oracle():
    """Slice-wise, threaded evaluation gives the plain oracle's bits: sizes
    straddle the 1 Mi-element slice boundary; moments in float32 and bfloat16;
    norms with the per-tensor order kept."""
    from oracle import parallel
    rng = np.random.default_rng(77)
    sizes = [parallel.SLICE + 4097, 3, parallel.SLICE, 70001]
    options = dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
    with parallel.Pool(4) as pool:
        for n in sizes:
            p = (rng.standard_normal(n) * 0.02).astype(np.float32)
            g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
            m = (rng.standard_normal(n) * 1e-4).astype(np.float32)
            v = np.abs(rng.standard_normal(n) * 1e-6).astype(np.float32)
            a = [x.copy() for x in (p, g, m, v)]
            b = [x.copy() for x in (p, g, m, v)]
            adam.adam_step(*a, 3, **options)
            parallel.adam_step(pool, *b, 3, **options)
            assert all(x.tobytes() == y.tobytes() for x, y in zip(a, b))
            mb, vb = lowp.round_bf16(m), lowp.round_bf16(v)
            a = [p.copy(), lowp.round_bf16(g), mb.copy(), vb.copy()]
            b = [x.copy() for x in a]
            adam.master_step(*a, 3, state_bf16=True, **options)
            parallel.master_step(pool, *b, 3, state_bf16=True, **options)
            assert all(x.tobytes() == y.tobytes() for x, y in zip(a, b))
            g16 = (g * 65536).astype(np.float16)
            assert parallel.unscale(pool, g16, 65536.0, "float16").tobytes() == scaler.unscale(g16, 65536.0, "float16").tobytes()
            assert parallel.clip_apply(pool, g, 0.3, "bfloat16").tobytes() == clip.clip_apply(g, 0.3, "bfloat16").tobytes()
            assert parallel.round_bf16(pool, p).tobytes() == lowp.round_bf16(p).tobytes()
        grads = [(rng.standard_normal(n) * 1e-3).astype(np.float32) for n in sizes]
        for order in (2.0, 3.0, np.inf):
            assert parallel.total_norm(pool, grads, order) == clip.total_norm(grads, order)
        grads[1][1] = np.nan
        assert math.isnan(parallel.total_norm(pool, grads)) and not parallel.finite(pool, grads)


def test_parallel_exact_sum_and_streamed_norm():
    """exact_sum equals np.sum of a float64 vector bit for bit (sizes around
    NumPy's 8192-element reduction blocks and the pool's slices, values over
    many magnitudes, so a different summation order shows), and
    total_norm_streamed equals clip.total_norm for p = 2, 3 and inf, with
    non-finite gradients, zeros and empty tensors.  A sum in another order
    (plain pairwise over the whole vector) differs on the same inputs."""
    from oracle import parallel
    rng = np.random.default_rng(2024)
    block = parallel.SUM_BLOCK
    sizes = [0, 1, 7, block - 1, block, block + 1, 3 * block + 5, parallel._SUM_SLICE + 17, 2 * parallel._SUM_SLICE]
    differs = 0
    with parallel.Pool(4) as pool:
        for n in sizes:
            values = rng.standard_normal(n) * np.exp2(rng.integers(-40, 40, n))
            assert parallel.exact_sum(pool, values) == np.sum(values, dtype=np.float64), n
            if n > block:
                halves = np.sum(values[: n // 2], dtype=np.float64) + np.sum(values[n // 2:], dtype=np.float64)
                differs += halves != np.sum(values, dtype=np.float64)
        assert differs > 0                                    # the check can tell orders apart
        grads = [(rng.standard_normal(n) * 1e-3 * np.exp2(rng.integers(-8, 8))).astype(np.float32)
                 for n in (block * 3 + 1, 5, 0, parallel.SLICE + 3, 70001)]
        for order in (2.0, 3.0, np.inf):
            got = parallel.total_norm_streamed(pool, len(grads), lambda i: grads[i], order)
            assert got == clip.total_norm(grads, order), order
        zeros = [np.zeros(10, np.float32), np.zeros(0, np.float32)]
        assert parallel.total_norm_streamed(pool, 2, lambda i: zeros[i]) == clip.total_norm(zeros) == 0.0
        for poison in (np.inf, np.nan):
            bad = [g.copy() for g in grads]
            bad[3][7] = poison
            got = parallel.total_norm_streamed(pool, len(bad), lambda i: bad[i])
            want = clip.total_norm(bad)
            assert (math.isnan(got) and math.isnan(want)) or got == want


def test_reference_step_equals_adam_step():
    """reference_step (adam_step plus the reference's copy_ staging and state
    check, timed by the CPU baseline) gives adam_step's bits, float32 and
    float16, decoupled and coupled decay, and raises on a negative
    exp_avg_sq as the reference's state check does."""
    rng = np.random.default_rng(5)
    for dtype, decoupled in ((np.float32, True), (np.float32, False), (np.float16, True)):
        p = (rng.standard_normal(1000) * 0.02).astype(dtype)
        m = (rng.standard_normal(1000) * 1e-4).astype(dtype)
        v = np.abs(rng.standard_normal(1000) * 1e-6).astype(dtype)
        a = [p.copy(), m.copy(), v.copy()]
        b = [p.copy(), m.copy(), v.copy()]
        for step in range(1, 4):
            g = (rng.standard_normal(1000) * 1e-3).astype(dtype)
            options = dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, decoupled=decoupled)
            adam.adam_step(a[0], g, a[1], a[2], step, **options)
            adam.reference_step(b[0], g, b[1], b[2], step, **options)
            assert all(x.tobytes() == y.tobytes() for x, y in zip(a, b))
    v[3] = -1.0
    with pytest.raises(ValueError, match="nonnegative"):
        adam.reference_step(p, p, m, v, 1, lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
