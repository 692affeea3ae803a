"""The optimizer's (group, parameter, gradient) entries: the memoized and
bulk-checked ``Optimizer._grad_entries`` returns exactly what the per-item
iterator ``_parameters_with_grad`` yields (the reference's loop,
optimizer.py:186-196), and raises the iterator's first error."""

from __future__ import annotations

import numpy as np
import pytest

import namitorch_amd as nt

SHAPES = ((3, 4), (5,), (2, 2, 2), (7,), (4, 3), (1,), (6,))


def _optimizer(rng, master=False, dtype="float32"):
    params = [nt.Parameter(rng.standard_normal(shape).astype(np.float32), dtype=dtype) for shape in SHAPES]
    groups = [{"params": params[:3], "weight_decay": 0.1}, {"params": params[3:5]}, {"params": params[5:]}]
    return nt.optim.AdamW(groups, lr=1e-3, master_weights=master), params


def _gradient(rng, parameter, dtype=None, shape=None):
    shape = parameter.shape if shape is None else shape
    return nt.Tensor(rng.standard_normal(shape).astype(np.float32), dtype=dtype or parameter.dtype.name)


def _same(first, second):
    assert len(first) == len(second)
    for a, b in zip(first, second):
        assert len(a) == 3 and all(x is y for x, y in zip(a, b))


def _outcome(call):
    try:
        return call(), None
    except (TypeError, ValueError, RuntimeError) as error:
        return None, (type(error), str(error))


@pytest.mark.parametrize("master", [False, True])
def test_entries_match_the_iterator_over_random_patterns(master):
    rng = np.random.default_rng(11 + master)
    optimizer, params = _optimizer(rng, master=master, dtype="bfloat16" if master else "float32")
    kept = [None] * len(params)
    for step in range(60):
        for index, parameter in enumerate(params):
            roll = rng.integers(6)
            if roll == 0:
                parameter.grad = None
            elif roll == 1:
                parameter.grad = kept[index] = _gradient(rng, parameter)
            elif roll == 2 and kept[index] is not None:
                parameter.grad = kept[index]                     # an older gradient object again
            elif roll == 3:
                parameter.requires_grad = not parameter.requires_grad
        for _ in range(2):                                       # a miss, then the memo
            entries = optimizer._grad_entries()
            _same(entries, tuple(optimizer._parameters_with_grad()))
        for group, parameter, gradient in entries:
            assert any(parameter is member for member in group["params"])
            assert parameter.grad is gradient and parameter.requires_grad


@pytest.mark.parametrize("master", [False, True])
def test_entries_raise_the_iterators_first_error(master):
    rng = np.random.default_rng(5)
    dtype = "bfloat16" if master else "float32"
    wrong_dtype = "float64"
    cases = [
        {1: dict(shape=(9,)), 4: dict(dtype=wrong_dtype)},
        {1: dict(dtype=wrong_dtype), 4: dict(shape=(9,))},
        {6: dict(shape=(2,))},
        {0: dict(dtype=wrong_dtype)},
    ]
    for bad in cases:
        optimizer, params = _optimizer(rng, master=master, dtype=dtype)
        for index, parameter in enumerate(params):
            parameter.grad = _gradient(rng, parameter, **bad.get(index, {}))
        got = _outcome(optimizer._grad_entries)
        expected = _outcome(lambda: tuple(optimizer._parameters_with_grad()))
        assert got[0] is None and got[1] == expected[1], bad
        # A parameter that does not require gradients is skipped with its gradient.
        for index in bad:
            params[index].requires_grad = False
        _same(optimizer._grad_entries(), tuple(optimizer._parameters_with_grad()))


def test_entries_report_a_device_mismatch_like_the_iterator():
    rng = np.random.default_rng(3)
    optimizer, params = _optimizer(rng)
    for parameter in params:
        parameter.grad = _gradient(rng, parameter)
    params[2].grad._device = nt.Device("cuda", 0)               # a gradient that claims another device
    got = _outcome(optimizer._grad_entries)
    expected = _outcome(lambda: tuple(optimizer._parameters_with_grad()))
    assert got[0] is None and got[1] == expected[1]


def test_master_weights_accept_mixed_low_precision_gradients():
    rng = np.random.default_rng(8)
    optimizer, params = _optimizer(rng, master=True, dtype="bfloat16")
    for index, parameter in enumerate(params):
        parameter.grad = _gradient(rng, parameter, dtype=("float16", "bfloat16", "float32")[index % 3])
    _same(optimizer._grad_entries(), tuple(optimizer._parameters_with_grad()))
    params[3].grad = _gradient(rng, params[3], dtype="float64")
    got = _outcome(optimizer._grad_entries)
    assert got[1] == _outcome(lambda: tuple(optimizer._parameters_with_grad()))[1]
    assert got[1][0] is TypeError


def test_memo_keeps_no_gradient_alive():
    import gc
    import weakref

    rng = np.random.default_rng(2)
    optimizer, params = _optimizer(rng)
    for parameter in params:
        parameter.grad = _gradient(rng, parameter)
    optimizer._grad_entries()
    watched = weakref.ref(params[0].grad)
    params[0].grad = None
    gc.collect()
    assert watched() is None
    _same(optimizer._grad_entries(), tuple(optimizer._parameters_with_grad()))
