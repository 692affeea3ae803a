"""Gradient producer edges on the device: multi-tensor accumulation
(Tensor._accumulate_grad / autograd.accumulate_gradient) and
zero_grad(set_to_none=False), bit-exact against the reference's outputs
(tests/golden/accumulate.npz) and the oracle."""

from __future__ import annotations

import numpy as np
import pytest

import namitorch_amd as nt
from oracle import grads as ograds
from oracle import lowp

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
KEYS = [f"{leaf}_{incoming}" for leaf in ("float32", "float16", "float64") for incoming in ("float16", "float32", "float64")]


def _bits(tensor):
    return tensor.bits().tobytes()


def test_accumulate_matches_reference_golden(golden_dir):
    """All nine (leaf, incoming) dtype pairs in one call: stored gradients
    get the incoming ones added, fresh leaves get a cast copy."""
    data = np.load(golden_dir / "accumulate.npz")
    stored_leaves, fresh_leaves, incoming_stored, incoming_fresh = [], [], [], []
    for key in KEYS:
        leaf = key.split("_")[0]
        p = nt.Parameter(np.zeros_like(data[f"{key}_existing"]), device=DEV)
        p.grad = nt.Tensor(data[f"{key}_existing"], device=DEV)
        stored_leaves.append(p)
        incoming_stored.append(nt.Tensor(data[f"{key}_incoming"], device=DEV))
        q = nt.Parameter(np.zeros(data[f"{key}_existing"].shape, dtype=leaf), device=DEV)
        fresh_leaves.append(q)
        incoming_fresh.append(nt.Tensor(data[f"{key}_incoming"], device=DEV))
    versions = [p.grad._version for p in stored_leaves]
    nt.accumulate_grads(stored_leaves + fresh_leaves, incoming_stored + incoming_fresh)
    for key, p, q, version in zip(KEYS, stored_leaves, fresh_leaves, versions):
        assert p.grad.numpy().tobytes() == data[f"{key}_added"].tobytes(), key
        assert p.grad._version == version + 1
        assert q.grad is not None and q.grad.dtype is q.dtype
        assert q.grad.numpy().tobytes() == data[f"{key}_fresh"].tobytes(), key


@pytest.mark.parametrize("n", [1, 3, 4, 4095, 4096, 4097, 70001])
@pytest.mark.parametrize("pair", [("float32", "float32"), ("float16", "float16"), ("bfloat16", "float32"),
                                  ("bfloat16", "bfloat16"), ("float32", "bfloat16"), ("float16", "float32")])
def test_accumulate_sizes_and_tails(n, pair):
    leaf, incoming = pair
    rng = np.random.default_rng(n)
    existing = (rng.standard_normal(n) * 2.0).astype(np.float32)
    values = (rng.standard_normal(n) * 2.0).astype(np.float32)
    if leaf == "bfloat16":
        existing = lowp.round_bf16(existing)
    if incoming == "bfloat16":
        values = lowp.round_bf16(values)
    p = nt.Parameter(np.zeros(n, np.float32), dtype=leaf, device=DEV)
    p.grad = nt.Tensor(existing, dtype=leaf, device=DEV)
    nt.accumulate_grads([p], [nt.Tensor(values, dtype=incoming, device=DEV)])
    stored = existing if leaf == "bfloat16" else existing.astype(leaf)
    want = ograds.accumulate(stored, values, leaf)
    got = p.grad.numpy()
    assert got.tobytes() == np.asarray(want, dtype=got.dtype).tobytes()


def test_accumulate_unaligned_views_and_repeats():
    """Storage offsets that break 16-byte alignment take the scalar path; a
    leaf listed twice accumulates twice, in order."""
    import torch
    base = torch.zeros(4099, dtype=torch.float32, device=DEV)
    p = nt.Parameter(np.zeros(4097, np.float32), device=DEV)
    p.grad = nt.Tensor._from_storage(base[1:4098])       # 4-byte aligned only
    p.grad.copy_(nt.Tensor(np.full(4097, 0.5, np.float32), device=DEV))
    g1 = nt.Tensor(np.full(4097, 0.25, np.float32), device=DEV)
    g2 = nt.Tensor(np.full(4097, 2.0, np.float32), device=DEV)
    version = p.grad._version
    nt.accumulate_grads([p, p], [g1, g2])
    assert np.all(p.grad.numpy() == np.float32(2.75))
    assert p.grad._version == version + 2
    assert base[0].item() == 0.0 and base[4098].item() == 0.0     # neighbours untouched


def test_accumulate_then_step_equals_summed_gradient():
    """Micro-batch accumulation feeding AdamW gives the step on the sum."""
    rng = np.random.default_rng(5)
    p0 = (rng.standard_normal(5000) * 0.02).astype(np.float32)
    micro = [(rng.standard_normal(5000) * 1e-3).astype(np.float32) for _ in range(3)]
    a = nt.Parameter(p0, device=DEV)
    for g in micro:
        a._accumulate_grad(nt.Tensor(g, device=DEV))
    b = nt.Parameter(p0, device=DEV)
    b.grad = nt.Tensor(ograds.accumulate(ograds.accumulate(ograds.accumulate(None, micro[0], "float32"),
                                                           micro[1], "float32"), micro[2], "float32"), device=DEV)
    assert _bits(a.grad) == _bits(b.grad)
    for p in (a, b):
        nt.optim.AdamW([p], lr=1e-3).step()
    assert _bits(a) == _bits(b)


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16", "float64"])
def test_zero_grad_keep_buffers(dtype):
    rng = np.random.default_rng(9)
    shapes = [(17,), (64, 33), (4096,), (3, 5, 7)]
    params = [nt.Parameter(np.zeros(s, np.float32), dtype=dtype, device=DEV) for s in shapes]
    for p in params:
        p.grad = nt.Tensor(rng.standard_normal(p.shape).astype(np.float32) + 1.0, dtype=dtype, device=DEV)
    grads = [p.grad for p in params]
    versions = [g._version for g in grads]
    optimizer = nt.optim.AdamW(params) if dtype in ("float32", "float64") else nt.optim.AdamW(params, master_weights=True)
    optimizer.zero_grad(set_to_none=False)
    for p, g, version in zip(params, grads, versions):
        assert p.grad is g and g._version == version + 1
        assert not np.any(g.bits())                         # +0.0 everywhere
    optimizer.zero_grad()
    assert all(p.grad is None for p in params)
