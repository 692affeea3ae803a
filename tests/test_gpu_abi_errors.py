"""The C ABI's argument checks, entry point by entry point: each bad call
returns the documented status (raised here as ValueError for NT_ERR_VALUE,
TypeError for NT_ERR_TYPE, RuntimeError for NT_ERR_HIP) with a message that
names the problem, before anything is launched; a failed HIP query does not
leak into the next launch's check; and a good call leaves nt_last_error
empty.  Every call here fails during validation or is a no-op."""

from __future__ import annotations

import ctypes

import pytest
import torch

from namitorch_amd import _native

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
F32, F16, BF16, F64, NONE = _native.NT_F32, _native.NT_F16, _native.NT_BF16, _native.NT_F64, _native.NT_DTYPE_NONE
TORCH = {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16, F64: torch.float64}


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _lib():
    return _native.load()


def _call(name, *args):
    _native.call(name, *args)


def _rows(layout, sizes, slots=None, keep=None):
    """Plan rows over fresh device buffers for `layout` (param, grad, state, copy)."""
    keep = [] if keep is None else keep
    rows = []
    for index, n in enumerate(sizes):
        def buffer(code):
            if code == NONE:
                return None
            t = torch.zeros(max(n, 1), dtype=TORCH[code], device=DEV)
            keep.append(t)
            return t.data_ptr()
        p, g, s1, s2, c = buffer(layout[0]), buffer(layout[1]), buffer(layout[2]), buffer(layout[2]), buffer(layout[3])
        rows.append(_native.MtTensor(p, g, s1, s2, c, n, 0 if slots is None else slots[index], 0))
    return rows, keep


def _plan(layout, sizes, slots=None, keep=None):
    rows, keep = _rows(layout, sizes, slots, keep)
    handle = ctypes.c_void_p()
    _call("nt_plan_create", 0, (_native.MtTensor * max(1, len(rows)))(*rows), len(rows),
          ctypes.byref(_native.MtLayout(*layout)), 0, _stream(), ctypes.byref(handle))
    return handle, keep


def _coefs(n=1):
    record = _native.AdamWCoefs(1e-3, 0.9, 0.999, 0.1, 0.001, 1e-8, 0.0, 1.0, 0.1, 0.001, 0, 1, 0, 0)
    return (_native.AdamWCoefs * n)(*([record] * n))


@pytest.fixture
def plans():
    created = []

    def make(layout, sizes, slots=None):
        handle, keep = _plan(layout, sizes, slots)
        created.append((handle, keep))
        return handle

    yield make
    torch.cuda.synchronize()
    for handle, _ in created:
        _call("nt_plan_destroy", handle)


def test_queries_and_copies():
    with pytest.raises(ValueError, match="count is NULL"):
        _call("nt_device_count", None)
    with pytest.raises(ValueError, match="arch buffer is empty"):
        _call("nt_device_arch", 0, None, 64)
    with pytest.raises(ValueError, match="arch buffer is empty"):
        _call("nt_device_arch", 0, ctypes.create_string_buffer(8), 0)
    device = torch.zeros(2, device=DEV)
    host = (ctypes.c_float * 2)()
    with pytest.raises(ValueError, match="NULL pointer"):
        _call("nt_memcpy_d2h", None, device.data_ptr(), 8, _stream())
    with pytest.raises(ValueError, match="NULL pointer"):
        _call("nt_memcpy_h2d", device.data_ptr(), None, 8, _stream())
    _call("nt_memcpy_d2h", None, None, 0, _stream())                      # zero bytes: nothing to do
    _call("nt_memcpy_d2h", ctypes.addressof(host), device.data_ptr(), 8, _stream())
    assert _lib().nt_last_error() == b""


def test_failed_hip_query_does_not_leak_into_the_next_launch(plans):
    """hipGetDeviceProperties on a missing device fails; the next launch's
    check must still see only its own launch."""
    with pytest.raises(RuntimeError, match="hipGetDeviceProperties"):
        _call("nt_device_arch", 1_000_000, ctypes.create_string_buffer(64), 64)
    plan = plans((F32, F32, F32, NONE), [4096])
    _call("nt_adamw_mt", plan, _coefs(), 1, None, _stream())
    torch.cuda.synchronize()
    assert _lib().nt_last_error() == b""


def test_per_tensor_adamw():
    p = torch.zeros(16, device=DEV)
    with pytest.raises(ValueError, match="NULL array"):
        _call("nt_adamw_f32", p.data_ptr(), None, p.data_ptr(), p.data_ptr(), *([1.0] * 10), 0, 1, 16, _stream())
    with pytest.raises(ValueError, match="NULL array"):          # parameter needed when it is updated
        _call("nt_adamw_f32", None, p.data_ptr(), p.data_ptr(), p.data_ptr(), *([1.0] * 10), 0, 1, 16, _stream())
    _call("nt_adamw_f32", None, None, None, None, *([1.0] * 10), 0, 1, 0, _stream())   # empty tensor


def test_plan_create(plans):
    keep = []
    rows, _ = _rows((F32, F32, F32, NONE), [64], keep=keep)
    table = (_native.MtTensor * 1)(*rows)
    layout = _native.MtLayout(F32, F32, F32, NONE)
    handle = ctypes.c_void_p()
    with pytest.raises(ValueError, match="output pointer is NULL"):
        _call("nt_plan_create", 0, table, 1, ctypes.byref(layout), 0, _stream(), None)
    with pytest.raises(ValueError, match="layout is NULL"):
        _call("nt_plan_create", 0, table, 1, None, 0, _stream(), ctypes.byref(handle))
    with pytest.raises(ValueError, match="tensor table is invalid"):
        _call("nt_plan_create", 0, table, -1, ctypes.byref(layout), 0, _stream(), ctypes.byref(handle))
    with pytest.raises(TypeError, match="unsupported dtype code"):
        _call("nt_plan_create", 0, table, 1, ctypes.byref(_native.MtLayout(F32, 7, F32, NONE)), 0, _stream(),
              ctypes.byref(handle))
    with pytest.raises(ValueError, match="multiple of 2048"):
        _call("nt_plan_create", 0, table, 1, ctypes.byref(layout), 1000, _stream(), ctypes.byref(handle))
    bad = _native.MtTensor(rows[0].param, None, rows[0].exp_avg, rows[0].exp_avg_sq, None, 64, 0, 0)
    with pytest.raises(ValueError, match="has no gradient"):
        _call("nt_plan_create", 0, (_native.MtTensor * 1)(bad), 1, ctypes.byref(layout), 0, _stream(),
              ctypes.byref(handle))
    bad = _native.MtTensor(rows[0].param, rows[0].grad, rows[0].exp_avg, rows[0].exp_avg_sq, None, 64, 16, 0)
    with pytest.raises(ValueError, match="slot >= 16"):
        _call("nt_plan_create", 0, (_native.MtTensor * 1)(bad), 1, ctypes.byref(layout), 0, _stream(),
              ctypes.byref(handle))
    bad = _native.MtTensor(rows[0].param + 2, rows[0].grad, rows[0].exp_avg, rows[0].exp_avg_sq, None, 60, 0, 0)
    with pytest.raises(ValueError, match="not aligned to its dtype"):
        _call("nt_plan_create", 0, (_native.MtTensor * 1)(bad), 1, ctypes.byref(layout), 0, _stream(),
              ctypes.byref(handle))
    assert handle.value is None
    _call("nt_plan_destroy", None)
    with pytest.raises(ValueError, match="plan is NULL"):
        _call("nt_plan_info", None, None, None, None)
    plan = plans((F32, F32, F32, NONE), [10000, 1])
    numel, tensors, tasks = _native.c_uint64(), _native.c_int32(), _native.c_int64()
    _call("nt_plan_info", plan, ctypes.byref(numel), ctypes.byref(tensors), ctypes.byref(tasks))
    assert (numel.value, tensors.value, tasks.value) == (10001, 2, 4)


def test_multi_tensor_adamw(plans):
    plan = plans((F32, F32, F32, NONE), [64, 64], slots=[0, 3])
    with pytest.raises(ValueError, match="plan is NULL"):
        _call("nt_adamw_mt", None, _coefs(), 1, None, _stream())
    for count in (0, 17):
        with pytest.raises(ValueError, match="1..16 coefficient slots"):
            _call("nt_adamw_mt", plan, _coefs(16), count, None, _stream())
    with pytest.raises(ValueError, match="1..16 coefficient slots"):
        _call("nt_adamw_mt", plan, None, 4, None, _stream())
    with pytest.raises(ValueError, match="selects coefficient slot 3 but only 2"):
        _call("nt_adamw_mt", plan, _coefs(2), 2, None, _stream())
    grads_only = plans((NONE, F32, NONE, NONE), [64])
    with pytest.raises(ValueError, match="plan has no parameters"):
        _call("nt_adamw_mt", grads_only, _coefs(), 1, None, _stream())
    mixed64 = plans((F64, F32, F64, NONE), [64])
    with pytest.raises(TypeError, match="float64 AdamW requires float64"):
        _call("nt_adamw_mt", mixed64, _coefs(), 1, None, _stream())
    mixed16 = plans((F16, F16, F32, NONE), [64])
    with pytest.raises(TypeError, match="float16 AdamW requires float16"):
        _call("nt_adamw_mt", mixed16, _coefs(), 1, None, _stream())
    f16_state = plans((F32, F32, F16, NONE), [64])
    with pytest.raises(TypeError, match="optimizer-state dtype"):
        _call("nt_adamw_mt", f16_state, _coefs(), 1, None, _stream())
    f64_copy = plans((F32, F32, F32, F64), [64])
    with pytest.raises(TypeError, match="model-copy dtype"):
        _call("nt_adamw_mt", f64_copy, _coefs(), 1, None, _stream())
    # An empty plan with a bad layout fails like a non-empty one.
    empty = plans((F32, F64, F32, NONE), [0])
    with pytest.raises(TypeError, match="gradient dtype"):
        _call("nt_adamw_mt", empty, _coefs(), 1, None, _stream())
    _call("nt_adamw_mt", plans((F32, F32, F32, NONE), [0]), _coefs(), 1, None, _stream())
    assert _lib().nt_last_error() == b""


def test_prepass_finalize_norm_and_apply(plans):
    plan = plans((NONE, F32, NONE, NONE), [5000])
    ctrl = torch.zeros(ctypes.sizeof(_native.AmpCtrl), dtype=torch.uint8, device=DEV)
    c = ctrl.data_ptr()
    for scale in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(ValueError, match="loss scale must be finite and positive"):
            _call("nt_amp_prepass", plan, scale, 1, None, _stream())
    with pytest.raises(ValueError, match="plan is NULL"):
        _call("nt_amp_prepass", None, 1.0, 0, None, _stream())
    with pytest.raises(ValueError, match="control block is NULL"):
        _call("nt_amp_finalize", plan, None, None, 2.0, -1.0, 0, 2.0, 0.5, 2000, None, _stream())
    with pytest.raises(ValueError, match="carry and ctrl must be different"):
        _call("nt_amp_finalize", plan, c, c, 2.0, -1.0, 0, 2.0, 0.5, 2000, None, _stream())
    for norm_type in (0.0, -2.0, float("nan")):
        with pytest.raises(ValueError, match="norm_type must be positive"):
            _call("nt_amp_finalize", plan, c, None, norm_type, -1.0, 0, 2.0, 0.5, 2000, None, _stream())
    with pytest.raises(ValueError, match="unknown flags"):
        _call("nt_amp_finalize", plan, c, None, 2.0, -1.0, 8, 2.0, 0.5, 2000, None, _stream())
    update = _native.NT_FINALIZE_SCALER_UPDATE
    for growth, backoff, interval in ((2.0, 0.5, 0), (1.0, 0.5, 10), (2.0, 1.0, 10), (2.0, 0.0, 10)):
        with pytest.raises(ValueError, match="growth/backoff"):
            _call("nt_amp_finalize", plan, c, None, 2.0, -1.0, update, growth, backoff, interval, None, _stream())
    with pytest.raises(ValueError, match="control block is NULL"):
        _call("nt_grad_norm_pow", plan, None, 3.0, -1.0, 1.0, 0, 0, 0, _stream())
    for norm_type in (float("inf"), 0.0):
        with pytest.raises(ValueError, match="finite positive norm_type"):
            _call("nt_grad_norm_pow", plan, c, norm_type, -1.0, 1.0, 0, 0, 0, _stream())
    with pytest.raises(ValueError, match="unknown flags"):
        _call("nt_grad_norm_pow", plan, c, 2.0, -1.0, 1.0, 0, 0, 4, _stream())
    with pytest.raises(ValueError, match="norm_type 2 only"):
        _call("nt_grad_norm_pow", plan, c, 3.0, -1.0, 1.0, 0, 0, _native.NT_NORM_POW_GUARD, _stream())
    with pytest.raises(ValueError, match="plan is NULL"):
        _call("nt_grad_apply", None, None, _stream())
    _call("nt_grad_apply", plan, None, _stream())                         # no transform: nothing to do
    assert _lib().nt_last_error() == b""


def test_control_blocks_and_small_kernels():
    ctrl = torch.zeros(ctypes.sizeof(_native.AmpCtrl), dtype=torch.uint8, device=DEV)
    with pytest.raises(ValueError, match="control block is NULL"):
        _call("nt_ctrl_reset", None, 1.0, 0, _stream())
    with pytest.raises(ValueError, match="control block is NULL"):
        _call("nt_ctrl_carry", None, ctrl.data_ptr(), _stream())
    with pytest.raises(ValueError, match="alias"):
        _call("nt_ctrl_carry", ctrl.data_ptr(), ctrl.data_ptr(), _stream())
    x = torch.ones(8, device=DEV)
    mul, div = _native.NT_OP_MUL, _native.NT_OP_DIV
    with pytest.raises(ValueError, match="NULL array"):
        _call("nt_tensor_scalar", None, F32, x.data_ptr(), F32, 2.0, mul, None, 8, _stream())
    with pytest.raises(TypeError, match="unsupported input dtype"):
        _call("nt_tensor_scalar", x.data_ptr(), 9, x.data_ptr(), F32, 2.0, mul, None, 8, _stream())
    with pytest.raises(TypeError, match="unsupported output dtype"):
        _call("nt_tensor_scalar", x.data_ptr(), F32, x.data_ptr(), 9, 2.0, div, None, 8, _stream())
    with pytest.raises(ValueError, match="unknown operation"):
        _call("nt_tensor_scalar", x.data_ptr(), F32, x.data_ptr(), F32, 2.0, 7, None, 8, _stream())
    _call("nt_tensor_scalar", None, F32, None, F32, 2.0, mul, None, 0, _stream())      # empty loss
    flag = torch.ones(1, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="NULL flag"):
        _call("nt_any_negative", x.data_ptr(), F32, 8, None, _stream())
    with pytest.raises(ValueError, match="NULL array"):
        _call("nt_any_negative", None, F32, 8, flag.data_ptr(), _stream())
    with pytest.raises(TypeError, match="unsupported dtype"):
        _call("nt_any_negative", x.data_ptr(), 9, 8, flag.data_ptr(), _stream())
    torch.cuda.synchronize()
    assert int(flag.item()) == 0                                          # cleared before the checks failed


def test_combine_arguments():
    size = ctypes.sizeof(_native.AmpCtrl)
    blocks = [torch.zeros(size, dtype=torch.uint8, device=DEV) for _ in range(_native.NT_MAX_COMBINE + 2)]
    carry = blocks[-1].data_ptr()

    def table(*tensors):
        return (ctypes.c_void_p * max(1, len(tensors)))(*[t if isinstance(t, int) or t is None else t.data_ptr()
                                                          for t in tensors])

    def combine(pointers, n, carry_ptr=carry, norm_type=2.0, flags=0, growth=2.0, backoff=0.5, interval=2000):
        _call("nt_amp_combine", pointers, n, carry_ptr, norm_type, 1.0, flags, growth, backoff, interval, None, _stream())

    two = table(blocks[0], blocks[1])
    for n in (0, -1, _native.NT_MAX_COMBINE + 1):
        with pytest.raises(ValueError, match="control blocks required"):
            combine(table(*blocks[:max(n, 1)]), n)
    with pytest.raises(ValueError, match="control blocks required"):
        combine(None, 2)
    with pytest.raises(ValueError, match="carry block is NULL"):
        combine(two, 2, carry_ptr=None)
    with pytest.raises(ValueError, match="control block is NULL"):
        combine(table(blocks[0], None), 2)
    with pytest.raises(ValueError, match="carry and a combined block"):
        combine(table(blocks[0], carry), 2)
    with pytest.raises(ValueError, match="listed twice"):
        combine(table(blocks[0], blocks[1], blocks[0]), 3)
    for norm_type in (1.0, 3.0, float("-inf"), float("nan")):
        with pytest.raises(ValueError, match="norm_type must be 2 or positive infinity"):
            combine(two, 2, norm_type=norm_type)
    with pytest.raises(ValueError, match="unknown flags"):
        combine(two, 2, flags=4)
    update = _native.NT_FINALIZE_SCALER_UPDATE
    for growth, backoff, interval in ((1.0, 0.5, 10), (2.0, 1.0, 10), (2.0, 0.5, 0)):
        with pytest.raises(ValueError, match="growth/backoff"):
            combine(two, 2, flags=update, growth=growth, backoff=backoff, interval=interval)
    torch.cuda.synchronize()
    assert all(int(b.sum().item()) == 0 for b in blocks)                  # nothing was launched


def test_gradient_edges_and_pointer_columns(plans):
    grads = plans((NONE, BF16, NONE, NONE), [4096, 100])
    with pytest.raises(ValueError, match="plan is NULL"):
        _call("nt_grad_zero", None, _stream())
    with pytest.raises(ValueError, match="no incoming gradients"):
        _call("nt_grad_accumulate", grads, 0, _stream())
    fresh = [torch.zeros(4096, dtype=torch.bfloat16, device=DEV), torch.zeros(100, dtype=torch.bfloat16, device=DEV)]
    pointers = (ctypes.c_void_p * 2)(*[t.data_ptr() for t in fresh])
    for column in (-1, 6):
        with pytest.raises(ValueError, match="column must be 0..5"):
            _call("nt_plan_set_pointers", grads, column, pointers, 2, _stream())
    with pytest.raises(ValueError, match="no such column"):
        _call("nt_plan_set_pointers", grads, 2, pointers, 2, _stream())
    with pytest.raises(ValueError, match="one pointer per plan tensor"):
        _call("nt_plan_set_pointers", grads, 1, pointers, 1, _stream())
    with pytest.raises(ValueError, match="pointer 1 is NULL"):
        _call("nt_plan_set_pointers", grads, 1, (ctypes.c_void_p * 2)(fresh[0].data_ptr(), None), 2, _stream())
    with pytest.raises(ValueError, match="breaks the alignment"):       # 16-byte aligned plan, 2-byte aligned pointer
        _call("nt_plan_set_pointers", grads, 1, (ctypes.c_void_p * 2)(fresh[0].data_ptr() + 2, fresh[1].data_ptr()),
              2, _stream())
    with pytest.raises(ValueError, match="breaks the alignment"):       # not even aligned to the dtype
        _call("nt_plan_set_pointers", grads, 1, (ctypes.c_void_p * 2)(fresh[0].data_ptr(), fresh[1].data_ptr() + 1),
              2, _stream())
    _call("nt_plan_set_pointers", grads, 1, pointers, 2, _stream())
    _call("nt_grad_zero", grads, _stream())
    torch.cuda.synchronize()
    assert _lib().nt_last_error() == b""
