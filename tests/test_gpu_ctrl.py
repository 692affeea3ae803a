"""The finalize's carry argument: finalizing into an unwritten block while
carrying the scaler state of the previous one gives, byte for byte, the
block that nt_ctrl_carry followed by a plain finalize gives (fused_step
relies on it to skip the carry launch), for finite and non-finite gradients,
with and without the clip and the scaler update, including a growth step and
a backoff."""

from __future__ import annotations

import ctypes

import pytest
import torch

from namitorch_amd import _native, runtime

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
NONE, BF16, F16 = _native.NT_DTYPE_NONE, _native.NT_BF16, _native.NT_F16
SIZE = ctypes.sizeof(_native.AmpCtrl)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _block(scale, tracker, iterations, skipped):
    ctrl = _native.AmpCtrl()
    ctrl.scale, ctrl.scale_used, ctrl.growth_tracker = scale, scale, tracker
    ctrl.iterations, ctrl.skipped, ctrl.clip_coef = iterations, skipped, 1.0
    ctrl.sumsq, ctrl.norm, ctrl.found_inf, ctrl.skip = 123.0, 4.5, 1, 1     # stale per-iteration fields
    host = torch.frombuffer(bytearray(bytes(ctrl)), dtype=torch.uint8)
    return host.to(DEV)


@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("poison", [False, True])
@pytest.mark.parametrize("flags,max_norm", [(0, -1.0), (3, 1e-3), (1, -1.0), (2, 0.05)])
@pytest.mark.parametrize("tracker", [0, 4])
def test_finalize_with_carry_equals_carry_then_finalize(dtype, poison, flags, max_norm, tracker):
    torch_dtype = torch.bfloat16 if dtype == BF16 else torch.float16
    gen = torch.Generator(device=DEV).manual_seed(9)
    grads = [(torch.randn(n, generator=gen, device=DEV) * 64.0).to(torch_dtype) for n in (1, 300, 5000, 70000)]
    if poison:
        grads[2][17] = float("inf")
    rows = [_native.MtTensor(None, g.data_ptr(), None, None, None, g.numel(), 0, 0) for g in grads]
    plan = ctypes.c_void_p()
    _native.call("nt_plan_create", 0, (_native.MtTensor * len(rows))(*rows), len(rows),
                 ctypes.byref(_native.MtLayout(NONE, dtype, NONE, NONE)), 0, _stream(), ctypes.byref(plan))
    try:
        previous = _block(1024.0, tracker, 7, 2)
        carried = torch.zeros(SIZE, dtype=torch.uint8, device=DEV)
        direct = torch.full((SIZE,), 0xA5, dtype=torch.uint8, device=DEV)       # unwritten block
        args = (2.0, max_norm, flags, 2.0, 0.5, 5)
        _native.call("nt_ctrl_carry", carried.data_ptr(), previous.data_ptr(), _stream())
        _native.call("nt_amp_prepass", plan, 1.0, 1, carried.data_ptr(), _stream())
        _native.call("nt_amp_finalize", plan, carried.data_ptr(), None, *args, None, _stream())
        _native.call("nt_amp_prepass", plan, 1.0, 1, previous.data_ptr(), _stream())
        mirror = runtime.take_mirror()
        _native.call("nt_amp_finalize", plan, direct.data_ptr(), previous.data_ptr(), *args, ctypes.addressof(mirror),
                     _stream())
        torch.cuda.synchronize()
    finally:
        _native.call("nt_plan_destroy", plan)
    assert torch.equal(carried.cpu(), direct.cpu())
    # the finalize's host mirror holds the finished block, flagged ready
    assert mirror.ready == 1
    assert bytes(mirror.ctrl) == bytes(direct.cpu().numpy())
    runtime.give_mirror(mirror)
    ctrl = _native.AmpCtrl.from_buffer_copy(bytes(direct.cpu().numpy()))
    assert ctrl.found_inf == int(poison) and ctrl.iterations == 8 and ctrl.skipped == 2 + int(poison)
    if flags & _native.NT_FINALIZE_SCALER_UPDATE:
        expected = 512.0 if poison else (2048.0 if tracker == 4 else 1024.0)
        assert ctrl.scale == expected and ctrl.scale_used == 1024.0
