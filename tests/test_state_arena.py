"""Optimizer state buffers created or loaded together are ranges of one flat
allocation per (buffer, device, dtype).  Values, dtypes, shapes, aliasing
and the state_dict round trip are the same as with one allocation per
buffer (the reference's ``_buffer``, _common.py:50-54, which the tests
force by turning the bulk creation off)."""

from __future__ import annotations

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd.optim import _common
from namitorch_amd.optim.adam import AdamW

SHAPES = ((3, 5), (7,), (0, 4), (2, 2, 3), (300,), (1,))


DEV = "cuda:0"


def _model(rng, dtype="float32", device=None):
    return [nt.Parameter(rng.standard_normal(shape).astype(np.float32), dtype=dtype, device=device) for shape in SHAPES]


def _base(tensor):
    """Identity of the allocation behind a Tensor's storage."""
    storage = tensor._storage
    if isinstance(storage, np.ndarray):
        return id(storage.base if storage.base is not None else storage)
    return storage._base.ptr


def _offset(tensor):
    """Elements between the allocation's start and the Tensor's first element."""
    storage = tensor._storage
    if isinstance(storage, np.ndarray):
        owner = storage.base if storage.base is not None else storage
        start = owner.__array_interface__["data"][0]
        return (storage.__array_interface__["data"][0] - start) // storage.itemsize
    return (storage.data_ptr() - storage._base.ptr) // tensor.dtype.itemsize


def _write(tensor, source):
    """Store `source`'s storage into `tensor`'s without a version bump."""
    if isinstance(tensor._storage, np.ndarray):
        np.copyto(tensor._storage, source._storage)
    else:
        tensor._storage.copy_from(source._storage)


def _run(master, per_buffer, monkeypatch, steps=3):
    rng = np.random.default_rng(4)
    dtype = "bfloat16" if master else "float32"
    params = _model(rng, dtype, DEV)
    optimizer = AdamW([{"params": params[:3], "weight_decay": 0.1}, {"params": params[3:]}], lr=1e-2,
                      master_weights=master)
    if per_buffer:
        monkeypatch.setattr(AdamW, "_create_buffers", lambda self, parameters: None)
    for _ in range(steps):
        for parameter in params:
            parameter.grad = nt.Tensor(rng.standard_normal(parameter.shape).astype(np.float32), dtype=dtype,
                                       device=DEV)
        optimizer.step()
    monkeypatch.undo()
    return optimizer, params


@pytest.mark.gpu
@pytest.mark.parametrize("master", [False, True])
def test_bulk_buffers_share_one_allocation_and_match_per_buffer_creation(master, monkeypatch):
    packed, packed_params = _run(master, False, monkeypatch)
    single, single_params = _run(master, True, monkeypatch)
    names = ("exp_avg", "exp_avg_sq") + (("master",) if master else ())
    for name in names:
        bases = {_base(packed.state[id(parameter)][name]) for parameter in packed_params}
        assert len(bases) == 1, name
        singles = {_base(single.state[id(parameter)][name]) for parameter in single_params if parameter.numel()}
        assert len(singles) == sum(1 for parameter in single_params if parameter.numel()), name
    for a, b in zip(packed_params, single_params):
        assert np.array_equal(a.numpy().view(np.uint8), b.numpy().view(np.uint8))
        for name in names:
            x, y = packed.state[id(a)][name], single.state[id(b)][name]
            assert x.dtype is y.dtype and x.shape == y.shape
            assert np.array_equal(x.numpy().view(np.uint8), y.numpy().view(np.uint8)), name
        assert packed.state[id(a)]["step"] == single.state[id(b)]["step"] == 3


@pytest.mark.parametrize("master", [False, True])
def test_bulk_creation_matches_one_at_a_time(master):
    """Host-side: ``_create_buffers`` against ``_buffers`` for the same parameters."""
    rng = np.random.default_rng(2)
    dtype = "bfloat16" if master else "float32"
    params = _model(rng, dtype)
    bulk = AdamW(params, lr=1e-2, master_weights=master)
    bulk._create_buffers(params)
    single = AdamW(params, lr=1e-2, master_weights=master)
    for parameter in params:
        single._buffers(parameter, single.state[id(parameter)])
    names = ("exp_avg", "exp_avg_sq") + (("master",) if master else ())
    for name in names:
        assert len({_base(bulk.state[id(parameter)][name]) for parameter in params}) == 1
        for parameter in params:
            x, y = bulk.state[id(parameter)][name], single.state[id(parameter)][name]
            assert x.dtype is y.dtype and x.shape == y.shape and x.device == y.device
            assert np.array_equal(x.numpy().view(np.uint8), y.numpy().view(np.uint8)), name
    bulk._create_buffers(params)                                  # nothing missing: nothing replaced
    assert all(bulk.state[id(parameter)]["exp_avg"] is not None for parameter in params)


def test_bulk_buffers_start_aligned_and_do_not_overlap():
    rng = np.random.default_rng(3)
    params = _model(rng)
    optimizer = AdamW(params, lr=1e-2)
    optimizer._create_buffers(params)
    for name in ("exp_avg", "exp_avg_sq"):
        spans = []
        for parameter in params:
            buffer = optimizer.state[id(parameter)][name]
            offset = _offset(buffer)
            assert offset % _common._ARENA_ALIGN == 0
            spans.append((offset, offset + buffer.numel()))
        spans.sort()
        assert all(end <= start for (_, end), (start, _) in zip(spans, spans[1:]))


def test_loaded_state_is_packed_with_values_kept():
    rng = np.random.default_rng(5)
    params = _model(rng, "bfloat16")
    optimizer = AdamW([{"params": params[:3], "weight_decay": 0.1}, {"params": params[3:]}], lr=1e-2,
                      master_weights=True)
    for index, parameter in enumerate(params):                   # one allocation per buffer
        state = optimizer.state[id(parameter)]
        optimizer._buffers(parameter, state)
        _write(state["exp_avg"], nt.Tensor(rng.standard_normal(parameter.shape).astype(np.float32)))
        _write(state["exp_avg_sq"], nt.Tensor(rng.random(parameter.shape).astype(np.float32)))
        state["step"] = index + 1
    saved = optimizer.state_dict()
    fresh = _model(rng, "bfloat16")
    for parameter, source in zip(fresh, params):
        _write(parameter, source)
    restored = AdamW([{"params": fresh[:3], "weight_decay": 0.1}, {"params": fresh[3:]}], lr=1e-2,
                     master_weights=True)
    restored.load_state_dict(saved)
    for name in ("exp_avg", "exp_avg_sq", "master"):
        assert len({_base(restored.state[id(parameter)][name]) for parameter in fresh}) == 1
        for parameter, source in zip(fresh, params):
            got, want = restored.state[id(parameter)][name], optimizer.state[id(source)][name]
            assert np.array_equal(got.numpy().view(np.uint8), want.numpy().view(np.uint8))
    again = restored.state_dict()
    for index in saved["state"]:
        for name in ("exp_avg", "exp_avg_sq", "master"):
            assert np.array_equal(np.asarray(again["state"][index][name].numpy()).view(np.uint8),
                                  np.asarray(saved["state"][index][name].numpy()).view(np.uint8))


def test_packing_keeps_one_object_for_an_aliased_buffer():
    rng = np.random.default_rng(1)
    shared = nt.Tensor(rng.standard_normal((4,)).astype(np.float32))
    other = nt.Tensor(rng.standard_normal((4,)).astype(np.float32))
    states = [{"exp_avg": shared, "exp_avg_sq": shared}, {"exp_avg": other, "exp_avg_sq": shared}]
    before = [shared.numpy().copy(), other.numpy().copy()]
    _common._pack_state_buffers(states, ("exp_avg", "exp_avg_sq"))
    assert states[0]["exp_avg"] is states[0]["exp_avg_sq"] is states[1]["exp_avg_sq"]
    assert states[1]["exp_avg"] is not states[0]["exp_avg"]
    assert _base(states[0]["exp_avg"]) == _base(states[1]["exp_avg"])
    assert np.array_equal(states[0]["exp_avg"].numpy(), before[0])
    assert np.array_equal(states[1]["exp_avg"].numpy(), before[1])


@pytest.mark.gpu
def test_a_single_fresh_parameter_keeps_its_own_allocation():
    rng = np.random.default_rng(6)
    params = _model(rng, device=DEV)
    optimizer = AdamW(params, lr=1e-2)
    params[4].grad = nt.Tensor(rng.standard_normal(params[4].shape).astype(np.float32), device=DEV)
    optimizer.step()
    assert set(optimizer.state[id(params[4])]) == {"exp_avg", "exp_avg_sq", "step"}
    assert _offset(optimizer.state[id(params[4])]["exp_avg"]) == 0


def test_moving_to_the_same_device_keeps_every_buffer_object():
    rng = np.random.default_rng(7)
    params = _model(rng)
    optimizer = AdamW(params, lr=1e-2)
    for parameter in params:                                     # one allocation per buffer
        optimizer._buffers(parameter, optimizer.state[id(parameter)])
        optimizer.state[id(parameter)]["step"] = 1
    before = {id(parameter): dict(optimizer.state[id(parameter)]) for parameter in params}
    optimizer.to("cpu")
    for parameter in params:
        for name in ("exp_avg", "exp_avg_sq"):
            assert optimizer.state[id(parameter)][name] is before[id(parameter)][name]


@pytest.mark.gpu
def test_state_moved_to_the_device_is_packed_with_values_kept():
    rng = np.random.default_rng(8)
    params = _model(rng, device=DEV)
    optimizer = AdamW(params, lr=1e-2)
    host = {}
    for parameter in params:
        values = {name: nt.Tensor(rng.standard_normal(parameter.shape).astype(np.float32))
                  for name in ("exp_avg", "exp_avg_sq")}
        values["exp_avg_sq"] = nt.Tensor(np.abs(values["exp_avg_sq"].numpy()))
        values["step"] = 2
        optimizer.state[id(parameter)] = values
        host[id(parameter)] = {name: values[name].numpy().copy() for name in ("exp_avg", "exp_avg_sq")}
    optimizer.to(DEV)
    for name in ("exp_avg", "exp_avg_sq"):
        assert len({_base(optimizer.state[id(parameter)][name]) for parameter in params}) == 1
        for parameter in params:
            moved = optimizer.state[id(parameter)][name]
            assert moved.device == nt.Device(DEV)
            assert np.array_equal(moved.numpy(), host[id(parameter)][name])


def test_bulk_creation_groups_by_dtype():
    rng = np.random.default_rng(12)
    params = [nt.Parameter(rng.standard_normal(shape).astype(np.float32), dtype=dtype)
              for shape, dtype in zip(SHAPES, ("float32", "float16", "float64", "float32", "float16", "float64"))]
    bulk = AdamW(params, lr=1e-2)
    bulk._create_buffers(params)
    single = AdamW(params, lr=1e-2)
    for parameter in params:
        single._buffers(parameter, single.state[id(parameter)])
    for name in ("exp_avg", "exp_avg_sq"):
        for dtype in ("float32", "float16", "float64"):
            members = [parameter for parameter in params if parameter.dtype.name == dtype]
            assert len({_base(bulk.state[id(parameter)][name]) for parameter in members}) == 1
        for parameter in params:
            x, y = bulk.state[id(parameter)][name], single.state[id(parameter)][name]
            assert x.dtype is y.dtype is parameter.dtype and x.shape == y.shape
            assert np.array_equal(x.numpy().view(np.uint8), y.numpy().view(np.uint8))
