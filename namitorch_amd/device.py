"""Devices: ``cpu`` and ``cuda[:N]``.

HIP devices keep the reference's ``cuda`` name, as PyTorch-ROCm does.  The
accepted spellings and the errors for everything else are those of
``namitorch/device.py``: ``"cpu"``, ``"cuda"`` (device 0), ``"cuda:N"`` with
N written without leading zeros, ``Device(...)`` copies, and an ``index``
argument for a bare ``"cuda"``.

Devices are immutable and interned: every spelling of one device yields the
same object, so device comparisons on the hot path are identity checks.
"""

from __future__ import annotations

import operator
from numbers import Integral
from threading import Lock

_KINDS = ("cpu", "cuda")
_ASCII_DIGITS = frozenset("0123456789")


def _split(spec: str):
    """(kind, index written in the string or None) of a device string."""
    kind, colon, written = spec.partition(":")
    if kind not in _KINDS:
        return None
    if not colon:
        return kind, None
    if not written or not set(written) <= _ASCII_DIGITS or (written[0] == "0" and written != "0"):
        return None
    return kind, int(written)


def _ordinal(kind: str, index):
    """The index a device of `kind` ends up with, checked."""
    if kind == "cpu":
        if index is not None:
            raise ValueError("CPU devices do not have an index.")
        return None
    if index is None:
        return 0
    if isinstance(index, bool) or not isinstance(index, Integral):
        raise TypeError("Device index must be a nonnegative integer.")
    try:
        index = operator.index(index)
    except TypeError:
        raise TypeError("Device index must be a nonnegative integer.") from None
    if index < 0:
        raise ValueError("Device index must be nonnegative.")
    return index


class Device:
    __slots__ = ("type", "index", "_hash")

    _interned: dict = {}
    _intern_lock = Lock()

    def __new__(cls, value="cpu", index=None):
        if isinstance(value, Device):
            if index is not None:
                raise ValueError("A Device cannot be combined with an index override.")
            return value
        if not isinstance(value, str):
            raise TypeError("Device expects a device string or another Device.")
        parsed = _split(value)
        if parsed is None:
            raise ValueError(f"Unsupported device {value!r}; expected cpu, cuda or cuda:N.")
        kind, written = parsed
        if written is not None and index is not None:
            raise ValueError("Specify the device index only once.")
        key = (kind, _ordinal(kind, written if written is not None else index))
        found = cls._interned.get(key)
        if found is None:
            with cls._intern_lock:
                found = cls._interned.get(key)
                if found is None:
                    found = object.__new__(cls)
                    object.__setattr__(found, "type", key[0])
                    object.__setattr__(found, "index", key[1])
                    object.__setattr__(found, "_hash", hash(key))
                    cls._interned[key] = found
        return found

    def __setattr__(self, name, value):
        raise AttributeError("Device is immutable.")

    def __reduce__(self):
        return (Device, (str(self),))

    def __eq__(self, other):
        return self is other or (isinstance(other, Device) and self.type == other.type and self.index == other.index)

    def __hash__(self):
        return self._hash

    def __str__(self):
        return self.type if self.index is None else f"{self.type}:{self.index}"

    def __repr__(self):
        return f"Device({str(self)!r})"

    @property
    def torch(self):
        import torch
        return torch.device(str(self))


def device(value="cpu", index=None) -> Device:
    return Device(value, index)


__all__ = ["Device", "device"]
