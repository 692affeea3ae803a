"""GPU numerics of the loss-scaling arithmetic and of gradient norms in the
places where a fused step or float64 gradients meet the reference API.

* Tensor-by-scalar arithmetic (``GradScaler.scale``, ``loss / accum``)
  against the reference's own outputs (scalar_ops.npz): result dtype and
  bits identical.
* Norm and clip read after ``fused_step`` see the unscaled gradients, as the
  reference's in-place ``unscale_`` leaves them.
* float64 gradients whose squares leave the float64 range: the norm follows
  the reference's max-abs prescale (clip_f64.npz), on the API path and in
  ``fused_step``.
* A fused AMP step queued on another stream than the previous one reads the
  previous step's control block in order (bit-identical to one stream).

Bars: bit-identical results and dtypes; norms within 1e-12 relative (their
last bits depend on the summation order and, in the reference, on the host's
NumPy ``power``); clipped float64 gradients bit-identical to
``f64(g) * coef`` for the device's coefficient.
"""

import json
import math

import numpy as np
import pytest

import namitorch_amd as nt
from oracle import adam as oadam
from oracle import arith
from oracle import clip as oclip
from oracle import lowp
from oracle import scaler as oscaler
from test_oracle import scalar_fixture_cases

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NORM_RTOL = 1e-12


def _bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype != b.dtype or a.shape != b.shape:
        return False
    nan = np.isnan(a.astype(np.float64)) & np.isnan(b.astype(np.float64))
    return bool(np.all((a.view(f"u{a.itemsize}") == b.view(f"u{b.itemsize}")) | nan))


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def test_scalar_ops_match_reference_golden(golden_dir):
    data = np.load(golden_dir / "scalar_ops.npz")
    for key, loss, operand, op in scalar_fixture_cases(data):
        tensor = nt.Tensor(loss, device=DEV)
        if key.split("_")[1] == "scale":
            result = nt.GradScaler(init_scale=operand).scale(tensor)
        else:
            result = tensor * operand if op == "mul" else tensor / operand
        assert result.dtype.name == data[key].dtype.name, key
        assert _bits_equal(result.numpy(), data[key]), key


def test_scaled_float16_loss_is_finite_float32():
    """A float16 loss of 3.0 scaled by 65536 is the float32 196608, not a
    float16 overflow to inf, on the host-held and the device-held scale."""
    loss = nt.Tensor(np.float16([3.0, -1.5]), device=DEV)
    scaler = nt.GradScaler()
    scaled = scaler.scale(loss)
    assert scaled.dtype is nt.float32
    assert scaled.numpy().tolist() == [196608.0, -98304.0]
    # After a fused step the scale lives in the device control block.
    param = nt.Parameter(np.zeros(8, dtype=np.float32), device=DEV)
    optimizer = nt.optim.AdamW([param])
    param.grad = nt.Tensor(np.ones(8, dtype=np.float32), device=DEV)
    nt.amp.fused_step(optimizer, scaler)
    scaled = scaler.scale(loss)
    assert scaled.dtype is nt.float32
    assert scaled.numpy().tolist() == [196608.0, -98304.0]
    bf = nt.Tensor(np.float32([3.0]), dtype="bfloat16", device=DEV)
    assert nt.GradScaler().scale(bf).dtype is nt.float32


@pytest.mark.parametrize("divisor", [3, 7, 3.0, np.float64(10.0)])
def test_loss_division_is_true_division(divisor):
    rng = _rng(61)
    for dtype in (np.float16, np.float32, np.float64):
        loss = (rng.standard_normal(4097) * 5).astype(dtype)
        got = (nt.Tensor(loss, device=DEV) / divisor).numpy()
        want = arith.scalar_op(loss, divisor, "div")
        assert _bits_equal(got, want), (dtype, divisor)


@pytest.mark.parametrize("grad_dtype", ["float16", "bfloat16", "float32"])
def test_norm_and_clip_after_fused_step_see_unscaled_gradients(grad_dtype):
    """get_grad_norm / clip_grad_norm_ called after an AMP fused_step (for
    example to log the norm) use the unscaled gradients, and a clip recorded
    then is applied when the gradients are read."""
    rng = _rng(3)
    shapes = [(301, 17), (17,), (4099,)]
    params = [nt.Parameter(np.zeros(s, dtype=np.float32), dtype="bfloat16" if grad_dtype == "bfloat16" else grad_dtype,
                           device=DEV) for s in shapes]
    optimizer = nt.optim.AdamW(params, master_weights=True)
    scaler = nt.GradScaler(init_scale=1024.0)
    scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
    stored = []
    for p, s in zip(params, shapes):
        g32 = (rng.standard_normal(s) * 1e-3 * 1024).astype(np.float32)
        g = lowp.round_bf16(g32) if grad_dtype == "bfloat16" else g32.astype(grad_dtype).astype(np.float32)
        stored.append(g)
        p.grad = nt.Tensor(g, dtype=grad_dtype, device=DEV)
    result = nt.amp.fused_step(optimizer, scaler)
    assert result.updated
    unscaled = [oscaler.unscale(g.astype(grad_dtype) if grad_dtype != "bfloat16" else g, 1024.0, grad_dtype)
                for g in stored]
    want = oclip.total_norm([u.astype(np.float64) for u in unscaled])
    norm = nt.optim.get_grad_norm(params).item()
    assert abs(norm - want) <= NORM_RTOL * want, (norm, want)
    max_norm = want / 4
    norm = nt.optim.clip_grad_norm_(params, max_norm).item()
    assert abs(norm - want) <= NORM_RTOL * want
    coefficient = oclip.clip_coefficient(max_norm, norm)
    assert coefficient < 1
    for p, u in zip(params, unscaled):
        expected = oclip.clip_apply(u.astype(np.float64), coefficient, grad_dtype)
        assert _bits_equal(p.grad.numpy(), expected.astype(p.grad.numpy().dtype))


def test_clip_float64_extremes_match_reference_golden(golden_dir):
    data = np.load(golden_dir / "clip_f64.npz")
    for record in json.loads(str(data["records"])):
        key = record["key"]
        grads = [data[f"{key}_in{i}"] for i in range(record["count"])]
        params = [nt.Parameter(np.zeros(g.shape), dtype="float64", device=DEV) for g in grads]
        for p, g in zip(params, grads):
            p.grad = nt.Tensor(g, device=DEV)
        norm = nt.optim.clip_grad_norm_(params, record["max_norm"], norm_type=record["norm_type"]).item()
        want = record["norm"]
        assert math.isfinite(norm) and norm > 0, key
        assert abs(norm - want) <= NORM_RTOL * want, (key, norm, want)
        coefficient = oclip.clip_coefficient(record["max_norm"], norm)
        for i, (p, g) in enumerate(zip(params, grads)):
            got = p.grad.numpy()
            with np.errstate(under="ignore"):
                assert _bits_equal(got, g * coefficient), (key, i)
            np.testing.assert_allclose(got, data[f"{key}_out{i}"], rtol=1e-12, atol=0)


@pytest.mark.parametrize("magnitude,max_norm", [(1e200, 1e199), (1e-200, 1e-210), (1.0, 1.0)])
def test_fused_step_float64_extreme_gradients(magnitude, max_norm):
    """fused_step's device-side norm for float64 gradients switches to the
    prescaled pass where squares leave the float64 range; the step then
    equals the host-synchronizing API sequence and the oracle."""
    rng = _rng(11)
    shapes = [(64, 33), (1000,)]
    host = [rng.standard_normal(s) * 0.02 for s in shapes]
    grads = [rng.standard_normal(s) * magnitude for s in shapes]

    def run(fused):
        params = [nt.Parameter(h, dtype="float64", device=DEV) for h in host]
        optimizer = nt.optim.AdamW(params, lr=1e-3, weight_decay=0.1)
        for p, g in zip(params, grads):
            p.grad = nt.Tensor(g, device=DEV)
        if fused:
            norm = nt.amp.fused_step(optimizer, None, max_norm=max_norm).norm
        else:
            norm = nt.optim.clip_grad_norm_(params, max_norm).item()
            optimizer.step()
        return norm, [p.numpy() for p in params]

    fused_norm, fused_params = run(True)
    api_norm, api_params = run(False)
    want = oclip.total_norm(grads)
    assert abs(fused_norm - want) <= NORM_RTOL * want and abs(api_norm - want) <= NORM_RTOL * want
    coefficient = oclip.clip_coefficient(max_norm, api_norm)
    for h, g, fp, ap in zip(host, grads, fused_params, api_params):
        ref = h.copy()
        m, v = np.zeros_like(ref), np.zeros_like(ref)
        with np.errstate(under="ignore"):
            clipped = g * coefficient if coefficient < 1 else g
        oadam.adam_step(ref, clipped, m, v, 1, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
        np.testing.assert_allclose(ap, ref, rtol=1e-12, atol=0)
        np.testing.assert_allclose(fp, ref, rtol=1e-12, atol=0)


def test_fused_steps_on_alternating_streams_match_one_stream():
    """Each fused AMP step reads the previous step's control block (the loss
    scale and the scaler state); switching streams between steps orders that
    read after the previous finalize."""
    import torch
    rng = _rng(29)
    shapes = [(129, 31), (4099,)]
    host = [(rng.standard_normal(s) * 0.05).astype(np.float32) for s in shapes]
    grads = [[(rng.standard_normal(s) * 1e-3 * 65536).astype(np.float16) for s in shapes] for _ in range(6)]
    grads[2][1][5] = np.inf

    def run(streams):
        params = [nt.Parameter(lowp.round_bf16(h), dtype="bfloat16", device=DEV) for h in host]
        optimizer = nt.optim.AdamW(params, lr=1e-3, weight_decay=0.1, master_weights=True)
        scaler = nt.GradScaler(growth_interval=2)
        updated = []
        torch.cuda.synchronize()
        for k, step_grads in enumerate(grads):
            stream = streams[k % len(streams)]
            if k:
                # As a caller must: the new stream waits for the previous
                # step's writes of parameters and moments.
                stream.wait_stream(streams[(k - 1) % len(streams)])
            with torch.cuda.stream(stream):
                scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
                for p, g in zip(params, step_grads):
                    p.grad = nt.Tensor(g, device=DEV)
                updated.append(nt.amp.fused_step(optimizer, scaler, max_norm=1.0).updated)
        torch.cuda.synchronize()
        state = [optimizer.state[id(p)] for p in params]
        return updated, scaler.get_scale(), [s["master"].numpy() for s in state], [p.numpy() for p in params]

    one = run([torch.cuda.current_stream()])
    two = run([torch.cuda.Stream(), torch.cuda.Stream()])
    assert one[0] == two[0] and one[0][2] is False
    assert one[1] == two[1]
    for a, b in zip(one[2] + one[3], two[2] + two[3]):
        assert _bits_equal(a, b)


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_clip_error_if_nonfinite_matches_reference(golden_dir, dtype):
    """clip_grad_norm_(error_if_nonfinite=True) on an infinite norm raises the
    reference's RuntimeError text (tests/golden/golden.json, clip_grad.py:104-105)
    before anything is clipped; a NaN norm says nan; without the flag the
    norm is returned and nothing is raised."""
    want = json.loads((golden_dir / "golden.json").read_text())["errors"]["nonfinite_norm"]
    values = (np.arange(5000, dtype=np.float32) % 7 - 3) * np.float32(0.25)
    for poison, text in ((np.inf, want), (np.nan, want.replace("inf", "nan"))):
        host = values.copy()
        host[4097] = poison
        param = nt.Parameter(np.zeros(5000, np.float32), dtype=dtype, device=DEV)
        param.grad = nt.Tensor(host, dtype=dtype, device=DEV)
        before = param.grad.bits().copy()
        with pytest.raises(RuntimeError) as error:
            nt.optim.clip_grad_norm_([param], 1.0, error_if_nonfinite=True)
        assert str(error.value) == text
        assert np.array_equal(param.grad.bits(), before)
        norm = nt.optim.clip_grad_norm_([param], 1.0).item()
        assert (math.isnan(norm) if poison != poison else norm == math.inf)
