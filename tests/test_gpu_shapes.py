"""Launch shapes: every plan task size gives the same bits.

The multi-tensor kernels split a task over several workgroups when its size
is a power-of-two multiple of their slice (2048-16384 elements here) and
run whole tasks otherwise (6144: not a power-of-two multiple; 32768 and
65536: more than 64 slices).  For ragged tensor sizes around the slice and
task boundaries, the AdamW pass (fp32 and the AMP/clip bf16 layout), the
gradient zero/accumulate kernels and the in-place grad transform give
bit-identical results for every task size, equal to those of the default
4096-element plan, which the parity tests pin against the oracle."""

from __future__ import annotations

import ctypes

import pytest
import torch

from namitorch_amd import _native

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
F32, F16, BF16, NONE = _native.NT_F32, _native.NT_F16, _native.NT_BF16, _native.NT_DTYPE_NONE
TORCH = {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}
SIZES = (1, 255, 256, 257, 1000, 2047, 2048, 2049, 4095, 4096, 4097, 6143, 6145, 16385, 70001)
CHUNKS = (0, 2048, 6144, 8192, 16384, 32768, 65536)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _plan(layout, rows, chunk):
    handle = ctypes.c_void_p()
    _native.call("nt_plan_create", 0, (_native.MtTensor * len(rows))(*rows), len(rows),
                 ctypes.byref(_native.MtLayout(*layout)), chunk, _stream(), ctypes.byref(handle))
    return handle


def _buffers(layout, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    p_code, g_code, s_code, c_code = layout
    tensors = []
    for n in SIZES:
        p = (torch.randn(n, generator=gen, device=DEV) * 0.02).to(TORCH[p_code])
        g = (torch.randn(n, generator=gen, device=DEV) * 1e-3).to(TORCH[g_code])
        m = (torch.randn(n, generator=gen, device=DEV) * 1e-4).to(TORCH[s_code])
        v = (torch.rand(n, generator=gen, device=DEV) * 1e-6).to(TORCH[s_code])
        c = torch.zeros(n, dtype=TORCH[c_code], device=DEV) if c_code != NONE else None
        tensors.append([p, g, m, v, c])
    return tensors


def _rows(tensors):
    return [_native.MtTensor(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(),
                             None if c is None else c.data_ptr(), p.numel(), index % 2, 0)
            for index, (p, g, m, v, c) in enumerate(tensors)]


def _bits(t):
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).cpu()


@pytest.mark.parametrize("layout,xform", [
    ((F32, F32, F32, NONE), None),
    ((F32, BF16, F32, BF16), dict(scale=65536.0, unscale=1, clip_coef=0.37, clip=1)),
    ((F32, BF16, BF16, BF16), dict(scale=1.0, unscale=0, clip_coef=0.5, clip=1)),
], ids=["fp32", "c5-layout-amp-clip", "c4-layout-clip"])
def test_adamw_pass_is_identical_for_every_task_size(layout, xform):
    records = [_native.AdamWCoefs(1e-3, 0.9, 0.999, 0.1, 0.001, 1e-8, 0.1, 1 - 1e-4, 0.1, 0.001, 0, 1, 0, 0),
               _native.AdamWCoefs(2e-3, 0.8, 0.99, 0.2, 0.01, 1e-6, 0.0, 1.0, 0.2, 0.01, 0, 1, 0, 0)]
    slots = (_native.AdamWCoefs * 2)(*records)
    xf = None if xform is None else ctypes.byref(_native.GradXform(**xform))
    expected = None
    for chunk in CHUNKS:
        print(f"adamw layout={layout} chunk={chunk}", flush=True)
        tensors = _buffers(layout, seed=11)
        if layout[1] == BF16 and xform is not None and xform["unscale"]:
            for t in tensors:
                t[1].mul_(65536.0)
        plan = _plan(layout, _rows(tensors), chunk)
        try:
            for _ in range(2):
                _native.call("nt_adamw_mt", plan, slots, 2, xf, _stream())
            torch.cuda.synchronize()
        finally:
            _native.call("nt_plan_destroy", plan)
        got = [[_bits(x) for x in (p, m, v) + ((c,) if c is not None else ())] for p, g, m, v, c in tensors]
        if expected is None:
            expected = got
            continue
        for index, (a, b) in enumerate(zip(got, expected)):
            for x, y in zip(a, b):
                assert torch.equal(x, y), (chunk, SIZES[index])


@pytest.mark.parametrize("dtype", [F32, BF16, F16])
def test_gradient_edges_are_identical_for_every_task_size(dtype):
    expected = None
    xf = _native.GradXform(scale=8.0, unscale=1, clip_coef=0.75, clip=1, honor_skip=0, ctrl=None)
    for chunk in CHUNKS:
        print(f"edges dtype={dtype} chunk={chunk}", flush=True)
        gen = torch.Generator(device=DEV).manual_seed(3)
        stored = [torch.randn(n, generator=gen, device=DEV).to(TORCH[dtype]) for n in SIZES]
        incoming = [torch.randn(n, generator=gen, device=DEV).to(TORCH[dtype]) for n in SIZES]
        zeroed = [torch.randn(n, generator=gen, device=DEV).to(TORCH[dtype]) for n in SIZES]
        layout = (dtype, dtype, NONE, NONE)
        rows = [_native.MtTensor(i.data_ptr(), s.data_ptr(), None, None, None, s.numel(), 0, 0)
                for s, i in zip(stored, incoming)]
        zero_rows = [_native.MtTensor(None, z.data_ptr(), None, None, None, z.numel(), 0, 0) for z in zeroed]
        plan = _plan(layout, rows, chunk)
        zero_plan = _plan((NONE, dtype, NONE, NONE), zero_rows, chunk)
        try:
            _native.call("nt_grad_accumulate", plan, 0, _stream())
            _native.call("nt_grad_apply", plan, ctypes.byref(xf), _stream())
            _native.call("nt_grad_zero", zero_plan, _stream())
            torch.cuda.synchronize()
        finally:
            _native.call("nt_plan_destroy", plan)
            _native.call("nt_plan_destroy", zero_plan)
        assert all(int(torch.count_nonzero(z)) == 0 for z in zeroed), chunk
        got = [_bits(s) for s in stored]
        if expected is None:
            expected = got
            continue
        for n, a, b in zip(SIZES, got, expected):
            assert torch.equal(a, b), (chunk, n)
