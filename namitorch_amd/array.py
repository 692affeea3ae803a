"""Device arrays over the library's caching allocator.

A :class:`DeviceArray` is a contiguous, typed view of device memory: either
a block from ``nt_malloc`` (returned to the pool when the last view of it is
gone) or memory owned by another framework, wrapped without a copy (anything
exposing ``__cuda_array_interface__``, or PyTorch-style ``data_ptr()`` /
``dtype`` / ``shape`` / ``device`` attributes, which also covers bfloat16).
It is the storage of device Tensors (``namitorch_amd.tensor``) and the array
type of the HIP backend, as CuPy arrays are the reference's
(``backends/cuda/__init__.py:30-32``).

Every operation is queued on the calling thread's current stream of the
array's device (``namitorch_amd.runtime``); host copies wait for it.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np

from . import _native, runtime
from .device import Device
from .dtype import DType, normalize_dtype

# bfloat16 has no type string of its own: like ml_dtypes and PyTorch, it is
# exported as a 2-byte opaque type ("<V2"), and "<V2" is read back as bfloat16.
_TYPESTR = {"float32": "<f4", "float16": "<f2", "float64": "<f8", "bfloat16": "<V2", "int8": "|i1", "int16": "<i2",
            "int32": "<i4", "int64": "<i8", "uint8": "|u1", "bool": "|b1"}
_FROM_TYPESTR = {value: key for key, value in _TYPESTR.items()}
_HOST_VIEW = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}


class _Block:
    """One ``nt_malloc`` allocation; freed (returned to the pool) with this object."""

    __slots__ = ("ptr", "nbytes", "device", "__weakref__")

    def __init__(self, device: int, nbytes: int):
        address = ctypes.c_void_p()
        _native.call("nt_malloc", device, nbytes, runtime.current_stream(device), ctypes.byref(address))
        self.ptr = address.value
        self.nbytes = nbytes
        self.device = device

    def __del__(self):
        try:                           # module globals may already be gone at interpreter exit
            if self.ptr and not _native.shutting_down():
                _native.load().nt_free(self.ptr)
        except Exception:
            pass


def _numel(shape) -> int:
    return math.prod(shape)


def _external_layout(obj):
    """(pointer, shape, DType, device index) of a contiguous device array
    owned elsewhere, or None when `obj` is not one."""
    interface = None
    try:
        interface = obj.__cuda_array_interface__
    except (AttributeError, TypeError, RuntimeError):
        interface = None
    if interface is not None:
        strides = interface.get("strides")
        shape = tuple(int(size) for size in interface["shape"])
        kind = _FROM_TYPESTR.get(interface["typestr"])
        if kind is None:
            raise TypeError(f"Unsupported device array type {interface['typestr']!r}.")
        dtype = DType(kind)
        if strides is not None:
            expected, step = [], dtype.itemsize
            for size in reversed(shape):
                expected.append(step)
                step *= size
            if tuple(reversed(expected)) != tuple(strides) and _numel(shape) > 1:
                raise ValueError("Device arrays must be C-contiguous.")
        pointer = int(interface["data"][0])
        device = _pointer_device(pointer) if pointer else 0
        return pointer, shape, dtype, device
    data_ptr, place = getattr(obj, "data_ptr", None), getattr(obj, "device", None)
    if callable(data_ptr) and getattr(place, "type", None) == "cuda":
        if callable(getattr(obj, "is_contiguous", None)) and not obj.is_contiguous():
            raise ValueError("Device arrays must be contiguous.")
        dtype = normalize_dtype(str(obj.dtype).rsplit(".", 1)[-1])
        return int(data_ptr()), tuple(int(size) for size in obj.shape), dtype, int(place.index or 0)
    return None


def _pointer_device(pointer: int) -> int:
    device = ctypes.c_int32()
    _native.call("nt_pointer_device", pointer, ctypes.byref(device))
    return device.value


def is_device_array(obj) -> bool:
    """A DeviceArray, or a device array of another framework (one exposing
    ``__cuda_array_interface__`` or PyTorch-style ``data_ptr()`` on a
    ``cuda`` device).  Whether its layout can be wrapped (contiguous, of a
    supported dtype) is checked by :meth:`DeviceArray.wrap`, which raises."""
    if isinstance(obj, DeviceArray):
        return True
    if isinstance(obj, (np.ndarray, np.generic, str, bytes, int, float, bool)) or obj is None:
        return False
    try:
        if getattr(obj, "__cuda_array_interface__", None) is not None:
            return True
    except Exception:
        pass
    return callable(getattr(obj, "data_ptr", None)) and getattr(getattr(obj, "device", None), "type", None) == "cuda"


class DeviceArray:
    __slots__ = ("_base", "_ptr", "_shape", "_dtype", "_device", "_numel", "__weakref__")

    # ---- construction -----------------------------------------------------------------------
    @classmethod
    def _make(cls, base, ptr: int, shape, dtype: DType, device: Device) -> "DeviceArray":
        array = cls.__new__(cls)
        array._base = base
        array._ptr = ptr
        array._shape = tuple(shape)
        array._dtype = dtype
        array._device = device
        array._numel = _numel(array._shape)
        return array

    @classmethod
    def empty(cls, shape, dtype, device) -> "DeviceArray":
        dtype = normalize_dtype(dtype)
        device = Device(device)
        shape = tuple(int(size) for size in shape)
        block = _Block(device.index, _numel(shape) * dtype.itemsize)
        return cls._make(block, block.ptr, shape, dtype, device)

    @classmethod
    def zeros(cls, shape, dtype, device) -> "DeviceArray":
        array = cls.empty(shape, dtype, device)
        array.fill_bits(0)
        return array

    @classmethod
    def wrap(cls, obj) -> "DeviceArray":
        """A view of another framework's device array (kept alive by the view)."""
        if isinstance(obj, DeviceArray):
            return obj
        layout = _external_layout(obj)
        if layout is None:
            raise TypeError(f"{type(obj).__name__} is not a device array.")
        pointer, shape, dtype, index = layout
        return cls._make(obj, pointer, shape, dtype, Device("cuda", index))

    # ---- description ------------------------------------------------------------------------
    @property
    def shape(self) -> tuple:
        return self._shape

    @property
    def dtype(self) -> DType:
        return self._dtype

    @property
    def device(self) -> Device:
        return self._device

    @property
    def ndim(self) -> int:
        return len(self._shape)

    @property
    def nbytes(self) -> int:
        return self._numel * self._dtype.itemsize

    def numel(self) -> int:
        return self._numel

    def dim(self) -> int:
        return len(self._shape)

    def data_ptr(self) -> int:
        return self._ptr

    def is_contiguous(self) -> bool:
        return True

    @property
    def __cuda_array_interface__(self) -> dict:
        typestr = _TYPESTR.get(self._dtype.value)
        if typestr is None:
            raise TypeError(f"{self._dtype.name} has no __cuda_array_interface__ type string.")
        return {"shape": self._shape, "typestr": typestr, "data": (self._ptr, False), "version": 3, "strides": None,
                "stream": runtime.current_stream(self._device.index) or 1}

    def __repr__(self) -> str:
        return f"DeviceArray(shape={self._shape}, dtype={self._dtype.name}, device='{self._device}')"

    # ---- views ------------------------------------------------------------------------------
    def reshape(self, shape) -> "DeviceArray":
        shape = tuple(int(size) for size in shape)
        if _numel(shape) != self._numel:
            raise ValueError(f"Cannot view {self._numel} elements as shape {shape}.")
        return DeviceArray._make(self._base, self._ptr, shape, self._dtype, self._device)

    def narrow(self, start: int, count: int, shape=None) -> "DeviceArray":
        """Elements [start, start + count) of the flat array, as `shape`."""
        if start < 0 or count < 0 or start + count > self._numel:
            raise ValueError("Range outside the array.")
        shape = (count,) if shape is None else tuple(shape)
        return DeviceArray._make(self._base, self._ptr + start * self._dtype.itemsize, shape, self._dtype,
                                 self._device)

    # ---- data movement ----------------------------------------------------------------------
    def _stream(self) -> int:
        return runtime.current_stream(self._device.index)

    def record_stream(self, stream_handle: int) -> None:
        """Keep the memory from reuse until work queued so far on
        `stream_handle` (a stream other than the allocating one) completes."""
        base = self._base
        if isinstance(base, _Block):
            _native.call("nt_record_stream", base.ptr, stream_handle)

    def fill_bits(self, pattern: int) -> "DeviceArray":
        with runtime.device_scope(self._device.index):
            _native.call("nt_fill", self._ptr, self._numel, self._dtype.itemsize, int(pattern) & ((1 << 64) - 1),
                         self._stream())
        return self

    def copy_from(self, source: "DeviceArray") -> "DeviceArray":
        """Copy `source` (same element count) into this array, converting the
        dtype on the device with one rounding to nearest even."""
        if source._numel != self._numel:
            raise ValueError(f"Cannot copy {source._numel} elements into {self._numel}.")
        if source._dtype is not self._dtype and (source._dtype.code == _native.NT_DTYPE_NONE
                                                 or self._dtype.code == _native.NT_DTYPE_NONE):
            raise TypeError(f"Device conversions exist between floating dtypes only, not "
                            f"{source._dtype.name} -> {self._dtype.name}.")
        with runtime.device_scope(self._device.index):
            if source._dtype is self._dtype:
                _native.call("nt_memcpy_async", self._ptr, source._ptr, self.nbytes, _native.NT_COPY_D2D,
                             self._stream())
            else:
                _native.call("nt_cast", source._ptr, source._dtype.code, self._ptr, self._dtype.code, self._numel,
                             self._stream())
        return self

    def upload(self, host: np.ndarray) -> "DeviceArray":
        """Copy host data already in this array's storage format (bfloat16 as
        uint16 bits) into the array; returns when the copy is done."""
        host = np.ascontiguousarray(host)
        if host.nbytes != self.nbytes:
            raise ValueError(f"Host data of {host.nbytes} bytes for a {self.nbytes}-byte array.")
        with runtime.device_scope(self._device.index):
            _native.call("nt_memcpy_h2d", self._ptr, host.ctypes.data, self.nbytes, self._stream())
        return self

    def download(self) -> np.ndarray:
        """Host copy in the storage format (bfloat16 as uint16 bits), after the
        work queued so far on the current stream."""
        if self._dtype.value == "bfloat16":
            out = np.empty(self._shape, dtype=np.uint16)
        else:
            out = np.empty(self._shape, dtype=self._dtype.numpy_dtype)
        with runtime.device_scope(self._device.index):
            _native.call("nt_memcpy_d2h", out.ctypes.data, self._ptr, self.nbytes, self._stream())
        return out

    def raw_bits(self) -> np.ndarray:
        """Host copy of the bit patterns as unsigned integers."""
        return self.download().view(_HOST_VIEW[self._dtype.itemsize])

    def clone(self) -> "DeviceArray":
        return DeviceArray.empty(self._shape, self._dtype, self._device).copy_from(self)


__all__ = ["DeviceArray", "is_device_array"]
