"""nt_amp_flat_stats_noalloc, the entry point that allocates nothing.

It is the plan-free variant of nt_amp_prepass + nt_amp_finalize over one
flat gradient buffer, with its partials in the library's fixed device array.
Each case runs both on the same inputs, called through the C ABI, twice in a
row with the second call on a smaller input (the shared array keeps the
first call's partials; the second must not read them).

Bar: the control blocks agree field by field — amax, flags, skip, clip
decision and scaler state exactly; the float64 sum of squares, norm and clip
coefficient within 1e-12 relative (the two reduce in different orders).  The
sum of squares is compared only for finite gradients: with an inf or NaN
present the norm is inf or NaN and the sum has no defined value.
"""

import ctypes
import math

import pytest
import torch

from namitorch_amd import _native

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
F32, F16, BF16, NONE = _native.NT_F32, _native.NT_F16, _native.NT_BF16, _native.NT_DTYPE_NONE
TORCH = {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}
EXACT = ("amax", "scale", "scale_used", "found_inf", "has_nan", "clip", "skip", "growth_tracker", "iterations", "skipped")
CLOSE = ("sumsq", "norm", "clip_coef")
UPDATE = _native.NT_FINALIZE_SCALER_UPDATE | _native.NT_FINALIZE_CLIP_IF_FINITE


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _read(block):
    torch.cuda.synchronize()
    return _native.AmpCtrl.from_buffer_copy(block.cpu().numpy().tobytes())


def _carry(scale, tracker):
    block = torch.zeros(ctypes.sizeof(_native.AmpCtrl), dtype=torch.uint8, device=DEV)
    _native.call("nt_ctrl_reset", block.data_ptr(), scale, tracker, _stream())
    return block


def _with_plan(grad, code, scale, unscale, carry, norm_type, max_norm, flags):
    table = (_native.MtTensor * 1)()
    table[0] = _native.MtTensor(None, grad.data_ptr(), None, None, None, grad.numel(), 0, 0)
    layout = _native.MtLayout(NONE, code, NONE, NONE)
    handle = ctypes.c_void_p()
    _native.call("nt_plan_create", 0, table, 1, ctypes.byref(layout), 0, _stream(), ctypes.byref(handle))
    try:
        block = torch.zeros(ctypes.sizeof(_native.AmpCtrl), dtype=torch.uint8, device=DEV)
        carry_ptr = None if carry is None else carry.data_ptr()
        _native.call("nt_amp_prepass", handle, scale, unscale, carry_ptr, _stream())
        _native.call("nt_amp_finalize", handle, block.data_ptr(), carry_ptr, norm_type, max_norm, flags, 2.0, 0.5, 3,
                     None, _stream())
        return _read(block)
    finally:
        torch.cuda.synchronize()
        _native.load().nt_plan_destroy(handle)


def _no_alloc(grad, code, scale, unscale, carry, norm_type, max_norm, flags, count=None):
    block = torch.zeros(ctypes.sizeof(_native.AmpCtrl), dtype=torch.uint8, device=DEV)
    _native.call("nt_amp_flat_stats_noalloc", 0, grad.data_ptr(), code, grad.numel() if count is None else count,
                 scale, unscale, block.data_ptr(), None if carry is None else carry.data_ptr(), norm_type, max_norm,
                 flags, 2.0, 0.5, 3, _stream())
    return _read(block)


def _agree(a, b, label):
    for name in EXACT:
        x, y = getattr(a, name), getattr(b, name)
        assert x == y or (isinstance(x, float) and math.isnan(x) and math.isnan(y)), (label, name, x, y)
    for name in CLOSE:
        x, y = getattr(a, name), getattr(b, name)
        if name == "sumsq" and b.found_inf:
            continue            # not defined once a gradient is non-finite (the norm is inf or NaN then)
        if math.isnan(x) or math.isnan(y) or math.isinf(x) or math.isinf(y) or y == 0:
            assert x == y or (math.isnan(x) and math.isnan(y)), (label, name, x, y)
        else:
            assert abs(x - y) <= 1e-12 * abs(y), (label, name, x, y)


def _grads(code, n, seed, scale=65536.0, poison=None):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    values = torch.randn(n, generator=gen, device=DEV) * (1e-3 * scale)
    if poison is not None:
        values[n // 3] = poison
    return values.to(TORCH[code])


CASES = [
    # (first call: dtype, count, poison), (second call: smaller), scale, unscale, carry, norm_type, max_norm, flags
    ((BF16, 3_000_003, None), (BF16, 70_001, None), 65536.0, 1, None, 2.0, 1.0, 0),
    ((F16, 2_500_000, None), (F16, 4_099, math.inf), 65536.0, 1, (65536.0, 2), 2.0, 1.0, UPDATE),
    ((F32, 1_048_577, None), (F32, 33, math.nan), 1.0, 0, None, math.inf, 0.5, 0),
    ((BF16, 9_999_999, None), (F16, 1, None), 3000.0, 1, (3000.0, 0), 2.0, -1.0, UPDATE),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_noalloc_matches_plan_entry_points_twice(case):
    first, second, scale, unscale, carry_spec, norm_type, max_norm, flags = CASES[case]
    for call, (code, n, poison) in enumerate((first, second)):
        grad = _grads(code, n, seed=100 * case + call, scale=scale if unscale else 1.0, poison=poison)
        carry = None if carry_spec is None else _carry(*carry_spec)
        want = _with_plan(grad, code, scale, unscale, carry, norm_type, max_norm, flags)
        got = _no_alloc(grad, code, scale, unscale, carry, norm_type, max_norm, flags)
        _agree(got, want, (case, call))
        assert bool(got.found_inf) == (poison is not None)


def test_noalloc_unaligned_and_empty_buffers():
    base = _grads(F32, 100_003, seed=7, scale=1.0)
    view = base[1:]                                  # 4-byte aligned only: the element-by-element path
    assert view.data_ptr() % 16 != 0
    _agree(_no_alloc(view, F32, 1.0, 0, None, 2.0, 1.0, 0), _with_plan(view, F32, 1.0, 0, None, 2.0, 1.0, 0),
           "unaligned")
    empty = torch.empty(0, dtype=torch.bfloat16, device=DEV)
    got = _no_alloc(empty, BF16, 1.0, 0, None, 2.0, 1.0, 0)
    assert got.sumsq == 0.0 and got.norm == 0.0 and not got.found_inf and got.iterations == 1


def test_noalloc_rejects_what_it_cannot_hold():
    """Argument errors are reported before anything is launched."""
    block = torch.zeros(ctypes.sizeof(_native.AmpCtrl), dtype=torch.uint8, device=DEV)
    grad = torch.zeros(8, device=DEV)
    call = _native.load().nt_amp_flat_stats_noalloc
    status = call(0, grad.data_ptr(), F32, (1 << 40) + 1, 1.0, 0, block.data_ptr(), None, 2.0, 1.0, 0, 2.0, 0.5, 3,
                  _stream())
    assert status == _native.NT_ERR_VALUE
    assert b"exceeds the maximum of 2**40 elements" in _native.load().nt_last_error()
    with pytest.raises(ValueError, match="norm_type must be 2"):
        _native.call("nt_amp_flat_stats_noalloc", 0, grad.data_ptr(), F32, 8, 1.0, 0, block.data_ptr(), None, 3.0,
                     1.0, 0, 2.0, 0.5, 3, _stream())
    with pytest.raises(TypeError, match="float32, float16 or bfloat16"):
        _native.call("nt_amp_flat_stats_noalloc", 0, grad.data_ptr(), _native.NT_F64, 8, 1.0, 0, block.data_ptr(),
                     None, 2.0, 1.0, 0, 2.0, 0.5, 3, _stream())
    with pytest.raises(ValueError, match="control block is NULL"):
        _native.call("nt_amp_flat_stats_noalloc", 0, grad.data_ptr(), F32, 8, 1.0, 0, None, None, 2.0, 1.0, 0, 2.0,
                     0.5, 3, _stream())
    torch.cuda.synchronize()
    assert not block.any()                           # nothing ran
