"""The array namespace of the backend protocol (backends/__init__.py:79-80):
NumPy for host arrays; for HIP devices the constructors and copies the
optimizer path's callers use, with every other name an error rather than a
CPU fallback."""

from __future__ import annotations

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd import backends
from namitorch_amd.array import DeviceArray

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def test_namespace_of_device_and_array():
    xp = backends.namespace(DEV)
    assert xp is nt.get_backend(DEV).namespace
    assert backends.namespace(DeviceArray.zeros((3,), nt.float32, DEV)) is xp
    assert backends.namespace("cpu") is np and backends.namespace(np.zeros(2)) is np


def test_constructors():
    xp = backends.namespace(DEV)
    zeros = xp.zeros((2, 3), "bfloat16")
    assert isinstance(zeros, DeviceArray) and zeros.shape == (2, 3) and zeros.dtype is nt.bfloat16
    assert not np.any(zeros.raw_bits())
    empty = xp.empty(5)
    assert empty.shape == (5,) and empty.dtype is nt.float32
    values = np.linspace(-1, 1, 6, dtype=np.float32).reshape(2, 3)
    source = xp.asarray(values)
    assert source.download().tobytes() == values.tobytes()
    assert xp.asarray(source) is source
    assert xp.array(source) is not source and xp.array(source).download().tobytes() == values.tobytes()
    wide = xp.zeros_like(source, dtype="float64")
    assert wide.dtype is nt.float64 and wide.shape == (2, 3) and not np.any(wide.download())
    assert xp.empty_like(source).shape == (2, 3)


def test_copyto_from_arrays_and_scalars():
    xp = backends.namespace(DEV)
    values = np.arange(6, dtype=np.float32).reshape(2, 3)
    source = xp.asarray(values)
    target = xp.empty_like(source)
    xp.copyto(target, source)
    assert target.download().tobytes() == values.tobytes()
    xp.copyto(target, values[::-1].copy())
    assert target.download().tobytes() == values[::-1].tobytes()
    xp.copyto(target, 0.5)
    assert np.all(target.download() == np.float32(0.5))
    with pytest.raises(ValueError):
        xp.copyto(target, xp.zeros((4,)))


def test_other_names_are_errors_not_fallbacks():
    xp = backends.namespace(DEV)
    source = xp.zeros((3,))
    with pytest.raises(RuntimeError, match="'sqrt' is not available"):
        xp.sqrt(source)
    with pytest.raises(RuntimeError, match="'sum' is not available"):
        xp.sum
