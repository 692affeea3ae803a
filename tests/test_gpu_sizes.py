"""Tensors past 2**31 and 2**32 elements: every kernel indexes elements
with 64-bit offsets, and a flat buffer of that size (a ZeRO/FSDP-style flat
parameter) updates exactly like a small one.

One tensor of n = 2**32 + 12293 elements (a ragged tail after the last
whole 4096-element task), filled with a block of B seeded values repeated
(B prime to 2, so the windows below see different block offsets).  The
update is elementwise, so the oracle on a window's inputs gives that
window's exact results; the windows sit at the start, across 2**31, across
2**32 and at the end.  The global norm is checked against the closed form
of the repeated block (fsum of the block's exact squares), 1e-12 relative.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import namitorch_amd as nt
from namitorch_amd.array import DeviceArray
from oracle import adam as oadam
from oracle import clip as oclip
from oracle import lowp
from oracle import scaler as oscaler

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
N = 2 ** 32 + 3 * 4096 + 5
BLOCK = 1_048_583
WINDOWS = [(0, 4096), (2 ** 31 - 2500, 2 ** 31 + 2500), (2 ** 32 - 2500, 2 ** 32 + 2500), (N - 9000, N)]


def _tiled(block: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    """Device tensor of N elements: `block` repeated, without a temporary."""
    source = torch.from_numpy(block).to(DEV, dtype)
    out = torch.empty(N, dtype=dtype, device=DEV)
    full, rest = divmod(N, BLOCK)
    out[:full * BLOCK].view(full, BLOCK).copy_(source.expand(full, BLOCK))
    out[full * BLOCK:].copy_(source[:rest])
    return out


def _window(block: np.ndarray, lo: int, hi: int) -> np.ndarray:
    return block[np.arange(lo, hi, dtype=np.int64) % BLOCK]


def _host(tensor, lo: int, hi: int) -> np.ndarray:
    if isinstance(tensor, DeviceArray):
        return tensor.narrow(lo, hi - lo).download()      # bfloat16 as uint16 bits
    values = tensor[lo:hi].cpu()
    return values.view(torch.int16).numpy().view(np.uint16) if values.dtype == torch.bfloat16 else values.numpy()


def _same(a, b) -> bool:
    return a.shape == b.shape and a.dtype == b.dtype and bool(np.all(a.view(f"u{a.itemsize}") == b.view(f"u{b.itemsize}")))


@pytest.fixture(autouse=True)
def _release():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    nt.runtime.empty_cache(0)


@pytest.mark.parametrize("path", ["optimizer", "per_tensor_hook"])
def test_fp32_step_past_2_32_elements(path):
    rng = np.random.Generator(np.random.PCG64(4242))
    p_block = (rng.standard_normal(BLOCK, dtype=np.float32) * np.float32(0.05))
    g_block = (rng.standard_normal(BLOCK, dtype=np.float32) * np.float32(1e-3))
    p = _tiled(p_block, torch.float32)
    g = _tiled(g_block, torch.float32)
    options = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
    if path == "optimizer":
        param = nt.Parameter.__new__(nt.Parameter)
        nt.Tensor._initialize(param, p, True)
        param.grad = nt.Tensor._from_storage(g)
        optimizer = nt.optim.AdamW([param], **options)
        optimizer.step()
        optimizer.step()
        state = optimizer.state[id(param)]
        m, v = state["exp_avg"]._storage, state["exp_avg_sq"]._storage
        assert state["step"] == 2
    else:
        backend = nt.get_backend(DEV)
        m = torch.zeros_like(p)
        v = torch.zeros_like(p)
        for step in (1, 2):
            coefficients = oadam.coefficients(np.float32, options["lr"], options["betas"], options["eps"],
                                              options["weight_decay"], step)
            assert backend.adamw.run(p, g, m, v, coefficients=coefficients, maximize=False, update_parameter=True)
    torch.cuda.synchronize()
    for lo, hi in WINDOWS:
        rp, rg = _window(p_block, lo, hi), _window(g_block, lo, hi)
        rm, rv = np.zeros_like(rp), np.zeros_like(rp)
        for step in (1, 2):
            oadam.adam_step(rp, rg, rm, rv, step, **options)
        assert _same(_host(p, lo, hi), rp), (path, lo)
        assert _same(_host(m, lo, hi), rm), (path, lo)
        assert _same(_host(v, lo, hi), rv), (path, lo)


def test_amp_fused_step_past_2_32_elements():
    """bf16 model + fp32 master, bf16 grads scaled by 65536, clip at 1.0:
    an inf in the very last element skips the step and halves the scale;
    the next step (fresh gradients) unscales, clips and updates every element."""
    rng = np.random.Generator(np.random.PCG64(4343))
    p_block = lowp.round_bf16(rng.standard_normal(BLOCK, dtype=np.float32) * np.float32(0.05))
    g_block = lowp.round_bf16(rng.standard_normal(BLOCK, dtype=np.float32) * np.float32(1e-3 * 65536))
    p = _tiled(p_block, torch.bfloat16)
    g = _tiled(g_block, torch.bfloat16)
    param = nt.Parameter.__new__(nt.Parameter)
    nt.Tensor._initialize(param, p, True)
    param.grad = nt.Tensor._from_storage(g)
    optimizer = nt.optim.AdamW([param], lr=1e-3, weight_decay=0.1, master_weights=True)
    scaler = nt.GradScaler(init_scale=65536.0)
    loss = nt.Tensor._from_storage(torch.ones((), device=DEV))

    g[N - 1] = float("inf")
    scaler.scale(loss)
    skipped = nt.amp.fused_step(optimizer, scaler, max_norm=1.0)
    assert not skipped.finite and not skipped.updated
    assert scaler.get_scale() == 32768.0
    for lo, hi in WINDOWS:
        assert _same(_host(p, lo, hi), lowp.f32_to_bf16(_window(p_block, lo, hi))), lo

    # The skipped step left the gradients unscaled in place (as unscale_
    # does); the next backward produces fresh ones.
    param.grad = None
    del g
    g = _tiled(g_block, torch.bfloat16)
    param.grad = nt.Tensor._from_storage(g)
    scaler.scale(loss)
    result = nt.amp.fused_step(optimizer, scaler, max_norm=1.0)
    assert result.finite and result.updated
    unscaled = oscaler.unscale(g_block, 32768.0, "bfloat16").astype(np.float64)
    full, rest = divmod(N, BLOCK)
    squares = unscaled * unscaled                    # exact: 8-bit significands
    expected = math.sqrt(math.fsum([full * math.fsum(squares), math.fsum(squares[:rest])]))
    assert abs(result.norm - expected) <= 1e-12 * expected, (result.norm, expected)
    coefficient = oclip.clip_coefficient(1.0, result.norm)
    assert coefficient < 1.0
    state = optimizer.state[id(param)]
    assert state["step"] == 1 and scaler.get_scale() == 32768.0
    for lo, hi in WINDOWS:
        grad = oclip.clip_apply(oscaler.unscale(_window(g_block, lo, hi), 32768.0, "bfloat16"), coefficient, "bfloat16")
        master = _window(p_block, lo, hi).copy()
        m, v = np.zeros_like(master), np.zeros_like(master)
        oadam.master_step(master, grad, m, v, 1, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
        assert _same(_host(state["master"]._storage, lo, hi), master), lo
        assert _same(_host(state["exp_avg"]._storage, lo, hi), m), lo
        assert _same(_host(state["exp_avg_sq"]._storage, lo, hi), v), lo
        assert _same(_host(p, lo, hi), lowp.f32_to_bf16(master)), lo
