"""Graph capture on the device: inside a real HIP stream capture
(torch.cuda.graph) the optimizer path raises the reference's capture
errors (optim/_common.py:134, amp.py:128,170, tensor.py:471-481,1253)
before queuing anything, so the capture ends empty and valid, the state is
untouched, and the same optimizer steps normally afterwards."""

from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

import namitorch_amd as nt

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
SUFFIX = " is not supported in CUDA graph preparation or capture; only deterministic FP32 inference is supported."


def test_stream_capture_rejects_the_optimizer_path():
    rng = np.random.Generator(np.random.PCG64(5))
    p = nt.Parameter((rng.standard_normal((64, 8)) * 0.05).astype(np.float32), device=DEV)
    p.grad = nt.Tensor((rng.standard_normal((64, 8)) * 1e-3).astype(np.float32), device=DEV)
    optimizer = nt.optim.AdamW([p], lr=1e-3)
    optimizer.step()
    optimizer.step()                                     # the step memo is in place
    scaler = nt.GradScaler()
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    torch.cuda.synchronize()
    before = p.numpy()
    calls = {
        "optimizer.step": ("Optimizer steps", optimizer.step),
        "fused_step": ("Optimizer steps", lambda: nt.amp.fused_step(optimizer, None, max_norm=1.0)),
        "scaler.scale": ("GradScaler", lambda: scaler.scale(loss)),
        "scaler.unscale_": ("GradScaler", lambda: scaler.unscale_(optimizer)),
        "clip_grad_norm_": ("Host Tensor reads", lambda: nt.optim.clip_grad_norm_([p], 1.0)),
        "Tensor.numpy": ("Host Tensor reads", p.numpy),
        "Tensor.copy_": ("In-place Tensor updates", lambda: p.grad.copy_(np.zeros((64, 8), np.float32))),
        "zero_grad": ("In-place Tensor updates", lambda: optimizer.zero_grad(set_to_none=False)),
    }
    raised = {}
    graph = torch.cuda.CUDAGraph()
    gc.disable()                                         # no finalizer may run HIP calls mid-capture
    try:
        with pytest.warns(UserWarning, match="CUDA Graph is empty"):       # nothing was queued
            with torch.cuda.graph(graph):
                for name, (_, call) in calls.items():
                    try:
                        call()
                        raised[name] = None
                    except RuntimeError as error:
                        raised[name] = str(error)
    finally:
        gc.enable()
    torch.cuda.synchronize()
    for name, (operation, _) in calls.items():
        assert raised[name] == operation + SUFFIX, (name, raised[name])
    assert np.array_equal(p.numpy(), before)
    assert optimizer.state[id(p)]["step"] == 2
    optimizer.step()
    torch.cuda.synchronize()
    assert optimizer.state[id(p)]["step"] == 3
    assert not np.array_equal(p.numpy(), before)
