"""Devices: ``cpu`` and ``cuda[:N]`` (HIP devices keep the reference's
``cuda`` name, as PyTorch-ROCm does).  Mirrors ``namitorch/device.py``:
the same accepted spellings and the same errors."""

from __future__ import annotations

import operator
import re
from numbers import Integral


class Device:
    __slots__ = ("type", "index", "_hash")

    def __init__(self, value="cpu", index=None):
        if isinstance(value, Device):
            if index is not None:
                raise ValueError("A Device cannot be combined with an index override.")
            kind, ordinal = value.type, value.index
        elif isinstance(value, str):
            match = re.fullmatch(r"(cpu|cuda)(?::(0|[1-9][0-9]*))?", value)
            if match is None:
                raise ValueError(f"Unsupported device {value!r}; expected cpu, cuda or cuda:N.")
            kind, embedded = match.groups()
            if embedded is not None and index is not None:
                raise ValueError("Specify the device index only once.")
            ordinal = int(embedded) if embedded is not None else index
            if kind == "cpu":
                if ordinal is not None:
                    raise ValueError("CPU devices do not have an index.")
            else:
                if ordinal is None:
                    ordinal = 0
                if isinstance(ordinal, bool) or not isinstance(ordinal, Integral):
                    raise TypeError("Device index must be a nonnegative integer.")
                ordinal = operator.index(ordinal)
                if ordinal < 0:
                    raise ValueError("Device index must be nonnegative.")
        else:
            raise TypeError("Device expects a device string or another Device.")
        object.__setattr__(self, "type", kind)
        object.__setattr__(self, "index", ordinal)
        object.__setattr__(self, "_hash", hash((kind, ordinal)))

    def __setattr__(self, name, value):
        raise AttributeError("Device is immutable.")

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
