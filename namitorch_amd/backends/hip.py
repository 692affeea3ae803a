"""HIP (MI355X) device backend.

Protocol of the reference's CUDA backend object
(namitorch/backends/cuda/__init__.py:23-225) as far as the optimizer step
uses it: ``device``, ``array_type``, ``array``, ``to_numpy``, ``item``,
``context``, ``result``, ``ready_for_host``, ``writable``, ``readonly`` and
the optional kernel attribute ``adamw``.  Backend arrays are
:class:`namitorch_amd.array.DeviceArray` (memory of the library's caching
allocator, or another framework's device array wrapped without a copy);
every operation launches the gfx950 kernels of ``libnamitorch_amd.so`` on
the calling thread's current stream of the device
(``namitorch_amd.runtime.current_stream``).

Multi-tensor plans (descriptor table + workgroup task map, see
``include/namitorch_amd.h``) are cached per backend, keyed by the raw
pointers, sizes, dtypes and coefficient slots they were built from; a key
match means the cached device tables describe exactly the current buffers.
"""

from __future__ import annotations

import atexit
import ctypes
import math
import operator
import threading
import weakref
from collections import OrderedDict

import numpy as np

from .. import _native, runtime
from ..array import DeviceArray
from ..device import Device
from ..dtype import float32, float64, int32, normalize_dtype, uint8

PLAN_CACHE_SIZE = 16
INCOMING = 5          # plan pointer column of deferred incoming gradients
_backends_alive: "weakref.WeakSet[HIPBackend]" = weakref.WeakSet()
_shutting_down = False


@atexit.register
def _release_plans() -> None:
    """Free cached plans while the HIP runtime is still up (before interpreter teardown)."""
    global _shutting_down
    for backend in list(_backends_alive):
        with backend._lock:
            backend._plans.clear()
    _shutting_down = True


class Plan:
    """A multi-tensor plan owned by the library; destroyed with this object."""

    __slots__ = ("handle", "numel", "ntensors", "ntasks", "layout", "columns", "stream_owner", "__weakref__")

    def __init__(self, handle: int, layout: tuple, stream_owner=None):
        self.handle = handle
        self.layout = layout
        # Destroying the plan records events on the streams it was used on:
        # a stream object created here stays alive as long as the plan.
        self.stream_owner = stream_owner
        self.columns: dict = {}       # volatile column -> pointers it currently holds
        numel = ctypes.c_uint64()
        tensors = ctypes.c_int32()
        tasks = ctypes.c_int64()
        _native.call("nt_plan_info", handle, ctypes.byref(numel), ctypes.byref(tensors), ctypes.byref(tasks))
        self.numel = numel.value
        self.ntensors = tensors.value
        self.ntasks = tasks.value

    def __del__(self):
        handle, self.handle = self.handle, None
        if handle and not _shutting_down:
            try:
                _native.load().nt_plan_destroy(handle)
            except Exception:
                pass


class AdamWHIPKernel:
    """The reference's per-tensor fused AdamW hook (backends/cuda/adamw.py:32-73).

    Arguments are raw storage arrays (DeviceArrays, or device arrays of
    another framework, on this device), exactly as the reference passes
    ``._data``; the caller owns version counters and ``state['step']``.
    """

    def __init__(self, backend: "HIPBackend"):
        self._backend = backend

    def supports(self, parameter, gradient, first=None, second=None) -> bool:
        arrays = (parameter, gradient, first, second)
        if parameter is None or gradient is None:
            return False
        present = []
        for array in arrays:
            if array is None:
                continue
            try:
                array = DeviceArray.wrap(array)
            except (TypeError, ValueError):
                return False
            present.append(array)
        shape = present[0].shape
        for array in present:
            if array.device != self._backend.device or array.dtype is not float32:
                return False
            if array.data_ptr() % 4 or array.shape != shape:
                return False
        ranges = [(array.data_ptr(), array.data_ptr() + array.numel() * 4) for array in present if array.numel()]
        return not any(
            max(start, other_start) < min(end, other_end)
            for position, (start, end) in enumerate(ranges)
            for other_start, other_end in ranges[position + 1:]
        )

    def run(self, parameter, gradient, first, second, *, coefficients, maximize, update_parameter) -> bool:
        if first is None or second is None or not self.supports(parameter, gradient, first, second):
            raise RuntimeError("Fused AdamW requires non-overlapping contiguous float32 CUDA arrays with identical shapes and device.")
        if len(coefficients) != 10 or any(not isinstance(value, np.float32) or not np.isfinite(value) for value in coefficients):
            raise ValueError("Fused AdamW requires ten finite float32 coefficients.")
        if coefficients[5] <= 0 or coefficients[8] <= 0 or coefficients[9] <= 0:
            raise ValueError("Fused AdamW eps and bias corrections must be positive.")
        if type(maximize) is not bool or type(update_parameter) is not bool:
            raise TypeError("Fused AdamW flags must be Python bools.")
        parameter, gradient, first, second = (DeviceArray.wrap(array) for array in (parameter, gradient, first, second))
        count = parameter.numel()
        if count == 0:
            return False
        with self._backend.context():
            _native.call(
                "nt_adamw_f32",
                parameter.data_ptr(), gradient.data_ptr(), first.data_ptr(), second.data_ptr(),
                *(float(value) for value in coefficients),
                int(maximize), int(update_parameter), count, self._backend.stream(),
            )
        return True


class HIPNamespace:
    """The backend's array namespace (the reference's ``backend.namespace``,
    backends/_namespace.py), for the array constructors and copies a caller
    of this path needs: ``zeros``, ``zeros_like``, ``empty``, ``empty_like``,
    ``asarray``/``array``, ``copyto`` and ``errstate``.  Array arithmetic is
    not offered: the optimizer step's arithmetic runs in the library's
    kernels, and other names raise RuntimeError, as the reference's
    namespace does for a primitive CuPy lacks (there is no CPU fallback)."""

    def __init__(self, backend: "HIPBackend"):
        self._backend = backend

    def zeros(self, shape, dtype=float32):
        with self._backend.context():
            return DeviceArray.zeros(_shape(shape), dtype, self._backend.device)

    def empty(self, shape, dtype=float32):
        with self._backend.context():
            return DeviceArray.empty(_shape(shape), dtype, self._backend.device)

    def zeros_like(self, array, dtype=None):
        array = DeviceArray.wrap(array)
        return self.zeros(array.shape, array.dtype if dtype is None else normalize_dtype(dtype))

    def empty_like(self, array, dtype=None):
        array = DeviceArray.wrap(array)
        return self.empty(array.shape, array.dtype if dtype is None else normalize_dtype(dtype))

    def asarray(self, value, dtype=None):
        return self._backend.array(value, dtype=dtype, copy=False)

    def array(self, value, dtype=None, copy=True):
        return self._backend.array(value, dtype=dtype, copy=copy)

    def copyto(self, destination, source):
        destination = DeviceArray.wrap(destination)
        if isinstance(source, DeviceArray) or _is_device(source):
            source = DeviceArray.wrap(source)
            if source.device != destination.device:
                raise RuntimeError(f"Operands are on different devices: {destination.device}, {source.device}; "
                                   "use an explicit .to() transfer.")
            if source.shape != destination.shape:
                raise ValueError(f"copyto: shapes {source.shape} and {destination.shape} differ.")
            destination.copy_from(source)
        else:
            from ..tensor import _assign_device
            _assign_device(destination, source, destination.dtype)

    errstate = staticmethod(np.errstate)

    def __getattr__(self, name):
        if name.startswith("__"):              # protocol probes (copy, pickle, hasattr) see a plain absence
            raise AttributeError(name)
        raise RuntimeError(f"HIP primitive {name!r} is not available in namitorch_amd: the optimizer step's "
                           "arithmetic runs in the library's kernels, and no CPU fallback is used.")


def _shape(shape) -> tuple:
    return (int(shape),) if isinstance(shape, (int, np.integer)) else tuple(int(size) for size in shape)


class HIPBackend:
    array_type = DeviceArray

    def __init__(self, device: Device):
        lib = _native.load()
        count = ctypes.c_int32()
        _native.check(lib.nt_device_count(ctypes.byref(count)))
        if device.index >= count.value:
            raise RuntimeError(f"CUDA device {device} is unavailable; found {count.value} CUDA devices.")
        self.device = device
        self.namespace = HIPNamespace(self)
        self.adamw = AdamWHIPKernel(self)
        self._plans: OrderedDict = OrderedDict()
        self._lock = threading.RLock()
        self._neutral_ctrl = None
        _backends_alive.add(self)

    def __repr__(self):
        return f"HIPBackend({self.device})"

    # ---- reference protocol --------------------------------------------------------------
    def context(self, *operands):
        """Make this backend's device the calling thread's current device."""
        return runtime.device_scope(self.device.index)

    def result(self, value):
        return value

    def ready_for_host(self, array):
        return array

    def supports_float16(self) -> bool:
        """gfx950 computes float16 natively (backends/cuda/__init__.py:47-53)."""
        return True

    def array(self, value, dtype=None, copy=True, *, non_blocking=False):
        """`value` (host data, a DeviceArray or another framework's device
        array) as a DeviceArray of this device, converted to `dtype`."""
        from ..tensor import _host_array, _resolve_dtype, _values
        kind = _resolve_dtype(value, dtype)
        if isinstance(value, DeviceArray) or (not isinstance(value, np.ndarray) and _is_device(value)):
            source = DeviceArray.wrap(value)
            if source.device == self.device and (source.dtype is kind or (source.dtype._floating and kind._floating)):
                if not copy and source.dtype is kind:
                    return source
                with self.context():
                    return DeviceArray.empty(source.shape, kind, self.device).copy_from(source)
            value = _values(source.download(), source.dtype)
        host = _host_array(value, kind)
        with self.context():
            return DeviceArray.empty(host.shape, kind, self.device).upload(host)

    def item(self, array):
        return self.to_numpy(array).reshape(()).item()

    def to_numpy(self, array):
        """Host copy of the values (bfloat16 widened exactly to float32)."""
        from ..tensor import _values
        array = DeviceArray.wrap(array)
        with self.context():
            return _values(array.download(), array.dtype)

    def writable(self, array):
        return True

    def readonly(self, array):
        return array

    # ---- streams ---------------------------------------------------------------------------
    def stream(self) -> int:
        """Handle of the calling thread's current stream on this device (a hipStream_t)."""
        return runtime.current_stream(self.device.index)

    def synchronize(self) -> None:
        with self.context():
            _native.call("nt_stream_synchronize", self.stream())

    # ---- plans -----------------------------------------------------------------------------
    def plan(self, rows: list[tuple], layout: tuple, chunk: int = 0, pointers: dict | None = None) -> Plan:
        """Plan for rows of (param, grad, exp_avg, exp_avg_sq, copy, numel, slot).

        Columns listed in `pointers` ({column: per-row pointers}) are volatile:
        their entries in `rows` are ignored (pass 0), the cached plan is keyed
        without them, and a hit whose pointers differ rewrites that column on
        the device (``nt_plan_set_pointers``, stream-ordered) instead of
        building a new plan.  Gradients reallocated every step therefore reuse
        one plan.  Plans are per stream: a column rewrite is ordered only on
        the stream that queues it."""
        volatile = () if not pointers else tuple(sorted(pointers))
        stream = self.stream()
        key = (layout, chunk, stream, volatile, tuple(rows))
        with self._lock:
            plan = self._plans.get(key)
            if plan is not None:
                self._plans.move_to_end(key)
                if volatile and not self._refresh_locked(plan, pointers, stream):
                    plan = None
                if plan is not None:
                    return plan
            full = rows
            in_rows = {column: values for column, values in (pointers or {}).items() if column < INCOMING}
            if in_rows:
                full = [tuple(in_rows[c][i] if c in in_rows else value for c, value in enumerate(row))
                        for i, row in enumerate(rows)]
            table = (_native.MtTensor * max(1, len(full)))()
            for index, (param, grad, first, second, copy, numel, slot) in enumerate(full):
                table[index] = _native.MtTensor(param or None, grad or None, first or None, second or None, copy or None, numel, slot, 0)
            spec = _native.MtLayout(*layout)
            handle = ctypes.c_void_p()
            with self.context():
                _native.call("nt_plan_create", self.device.index, table, len(full), ctypes.byref(spec), chunk, stream, ctypes.byref(handle))
            plan = Plan(handle.value, layout, runtime.current_stream_owner(self.device.index))
            plan.columns = {column: tuple(values) for column, values in in_rows.items()}
            if INCOMING in (pointers or {}) and not self._refresh_locked(plan, {INCOMING: pointers[INCOMING]}, stream):
                raise ValueError("Incoming gradients must be 16-byte aligned.")
            self._plans[key] = plan
            self._plans.move_to_end(key)
            while len(self._plans) > PLAN_CACHE_SIZE:
                self._plans.popitem(last=False)
            return plan

    def _refresh(self, plan: Plan, pointers: dict, stream: int) -> bool:
        """Point the volatile columns of a cached plan at `pointers`; False when
        a pointer breaks the plan's alignment (the caller builds a new plan)."""
        with self._lock:
            return self._refresh_locked(plan, pointers, stream)

    def _refresh_locked(self, plan: Plan, pointers: dict, stream: int) -> bool:
        for column, values in pointers.items():
            values = tuple(values)
            if plan.columns.get(column) == values:
                continue
            array = (ctypes.c_void_p * max(1, len(values)))(*values)
            with self.context():
                status = _native.load().nt_plan_set_pointers(plan.handle, column, array, len(values), stream)
            if status == _native.NT_ERR_VALUE:
                return False
            _native.check(status)
            plan.columns[column] = values
        return True

    def grad_plan(self, tensors, dtype, incoming: bool = False) -> Plan:
        """Gradient-only plan (the `grad` column volatile).  With `incoming`
        (the pre-pass) the deferred accumulations of the gradients become the
        plan's incoming column; otherwise they are written back first."""
        pointers = {1: [tensor._ptr for tensor in tensors]}
        addends = incoming_pointers(tensors)
        if addends is not None:
            if incoming:
                pointers[INCOMING] = addends
            else:
                for tensor in tensors:
                    if tensor._incoming is not None:
                        tensor._materialize()
        layout = (_native.NT_DTYPE_NONE, dtype.code, _native.NT_DTYPE_NONE, _native.NT_DTYPE_NONE)
        rows = [(0, 0, 0, 0, 0, tensor._numel, 0) for tensor in tensors]
        return self.plan(rows, layout, pointers=pointers)

    # ---- multi-tensor kernels --------------------------------------------------------------
    def adamw_multi(self, plan: Plan, slots, xform: _native.GradXform | None) -> None:
        with self.context():
            _native.call("nt_adamw_mt", plan.handle, ctypes.byref(slots), len(slots),
                         None if xform is None else ctypes.byref(xform), self.stream())

    def grad_prepass(self, plan: Plan, scale: float | None, ctrl_ptr: int | None = None, unscale: bool = False) -> None:
        with self.context():
            _native.call("nt_amp_prepass", plan.handle, 1.0 if scale is None else scale,
                         int(unscale or scale is not None), ctrl_ptr, self.stream())

    def grad_finalize(self, plan: Plan, ctrl_ptr: int, norm_type: float = 2.0, max_norm: float = -1.0,
                      flags: int = 0, growth: float = 2.0, backoff: float = 0.5, interval: int = 2000,
                      carry_ptr: int | None = None, mirror=None) -> None:
        """Finalize into `ctrl_ptr`; with `carry_ptr` the block starts from
        that block's scaler state (no separate carry launch); `mirror` (a
        ``runtime.take_mirror()``) receives the finished block on the host."""
        with self.context():
            _native.call("nt_amp_finalize", plan.handle, ctrl_ptr, carry_ptr, norm_type, max_norm, int(flags),
                         growth, backoff, interval, None if mirror is None else ctypes.addressof(mirror),
                         self.stream())

    def grad_combine(self, blocks, carry, norm_type: float, max_norm: float, flags: int, growth: float,
                     backoff: float, interval: int, mirrors=None) -> None:
        """nt_amp_combine over the finalized blocks (DeviceArrays), all
        carried from `carry`; `mirrors` (None, or one mirror or None per
        block) receive the finished blocks on the host."""
        pointers = (ctypes.c_void_p * len(blocks))(*[block.data_ptr() for block in blocks])
        hosts = None if mirrors is None else (ctypes.c_void_p * len(blocks))(
            *[None if mirror is None else ctypes.addressof(mirror) for mirror in mirrors])
        with self.context():
            _native.call("nt_amp_combine", pointers, len(blocks), carry.data_ptr(), norm_type, max_norm, int(flags),
                         growth, backoff, interval, hosts, self.stream())

    def grad_norm_pow(self, plan: Plan, ctrl_ptr: int, norm_type: float, max_norm: float,
                      scale: float | None, scale_from_ctrl: bool = False, flags: int = 0) -> None:
        with self.context():
            _native.call("nt_grad_norm_pow", plan.handle, ctrl_ptr, norm_type, max_norm,
                         1.0 if scale is None else scale, int(scale is not None or scale_from_ctrl),
                         int(scale_from_ctrl), int(flags), self.stream())

    def grad_apply(self, plan: Plan, xform: _native.GradXform) -> None:
        with self.context():
            _native.call("nt_grad_apply", plan.handle, ctypes.byref(xform), self.stream())

    # ---- control blocks ----------------------------------------------------------------------
    def new_ctrl(self, scale: float = 1.0, growth_tracker: int = 0) -> DeviceArray:
        block = self.empty_ctrl()
        self.reset_ctrl(block, scale, growth_tracker)
        return block

    def reset_ctrl(self, block: DeviceArray, scale: float, growth_tracker: int = 0) -> None:
        with self.context():
            _native.call("nt_ctrl_reset", block.data_ptr(), scale, growth_tracker, self.stream())

    def empty_ctrl(self) -> DeviceArray:
        """Device memory for a control block that a finalize will write whole."""
        with self.context():
            return DeviceArray.empty((ctypes.sizeof(_native.AmpCtrl),), uint8, self.device)

    def neutral_ctrl(self) -> DeviceArray:
        """A block with scale 1 and no history, kept per backend: the carry
        source of steps without a GradScaler.  Nothing writes it after set-up."""
        with self._lock:
            if self._neutral_ctrl is None:
                block = self.new_ctrl()
                self.synchronize()   # readable from any stream
                self._neutral_ctrl = block
            return self._neutral_ctrl

    def ctrl_norm(self, block: DeviceArray) -> DeviceArray:
        """A 0-d float64 array holding the block's ``norm``, copied on the
        device after the work queued so far (the host does not wait)."""
        with self.context():
            out = DeviceArray.empty((), float64, self.device)
            _native.call("nt_memcpy_async", out.data_ptr(), block.data_ptr() + _native.AmpCtrl.norm.offset,
                         ctypes.sizeof(ctypes.c_double), _native.NT_COPY_D2D, self.stream())
        return out

    def read_ctrl(self, block: DeviceArray) -> _native.AmpCtrl:
        out = _native.AmpCtrl()
        with self.context():
            _native.call("nt_memcpy_d2h", ctypes.addressof(out), block.data_ptr(), ctypes.sizeof(out), self.stream())
        return out

    # ---- single-tensor helpers --------------------------------------------------------------
    def zero_tensors(self, tensors) -> None:
        """Zero every tensor (one launch per dtype)."""
        by_dtype: dict = {}
        for tensor in tensors:
            by_dtype.setdefault(tensor.dtype, []).append(tensor)
        for dtype, group in by_dtype.items():
            plan = self.grad_plan(group, dtype)
            with self.context():
                _native.call("nt_grad_zero", plan.handle, self.stream())

    def accumulate_tensors(self, stored, incoming, assign: bool) -> None:
        """stored[i] <- cast(incoming[i]) (+ stored[i] unless `assign`), one
        launch per (stored dtype, incoming dtype)."""
        by_dtypes: dict = {}
        for target, source in zip(stored, incoming):
            by_dtypes.setdefault((target.dtype, source.dtype), []).append((target, source))
        for (target_dtype, source_dtype), pairs in by_dtypes.items():
            layout = (source_dtype.code, target_dtype.code, _native.NT_DTYPE_NONE, _native.NT_DTYPE_NONE)
            rows = [(0, 0, 0, 0, 0, target._numel, 0) for target, _ in pairs]
            plan = self.plan(rows, layout, pointers={0: [source._ptr for _, source in pairs],
                                                     1: [target._ptr for target, _ in pairs]})
            with self.context():
                _native.call("nt_grad_accumulate", plan.handle, int(assign), self.stream())

    def apply_grad_transform(self, tensors, transform) -> None:
        """Write pending GradTransforms back in place (one launch per dtype)."""
        by_dtype: dict = {}
        for tensor in tensors:
            by_dtype.setdefault(tensor.dtype, []).append(tensor)
        for dtype, group in by_dtype.items():
            plan = self.grad_plan(group, dtype)
            self.grad_apply(plan, make_xform(transform))

    def scalar_arithmetic(self, tensor, operand: float, op: int, dtype, ctrl: DeviceArray | None = None):
        """``tensor * operand`` (NT_OP_MUL) or ``tensor / operand`` (NT_OP_DIV)
        computed in `dtype`, a new Tensor of that dtype; `operand` is already
        a value of `dtype`.  With `ctrl` the operand is the loss scale held in
        that control block."""
        from ..tensor import Tensor
        if tensor.dtype.code == _native.NT_DTYPE_NONE or dtype.code == _native.NT_DTYPE_NONE:
            raise TypeError("Only floating Tensors support scalar arithmetic on the device.")
        source = tensor._data
        with self.context():
            out = DeviceArray.empty(source.shape, dtype, self.device)
            _native.call("nt_tensor_scalar", source.data_ptr(), tensor.dtype.code, out.data_ptr(), dtype.code,
                         float(operand), int(op), None if ctrl is None else ctrl.data_ptr(), tensor.size,
                         self.stream())
        return Tensor._from_storage(out, tensor.requires_grad)

    def any_negative(self, array: DeviceArray, code: int) -> bool:
        with self.context():
            flag = DeviceArray.empty((1,), int32, self.device)
            _native.call("nt_any_negative", array.data_ptr(), code, array.numel(), flag.data_ptr(), self.stream())
            return bool(flag.download()[0])


_INCOMING_OF = operator.attrgetter("_incoming")


def incoming_pointers(gradients) -> list | None:
    """The incoming-gradient column for `gradients` (0 where nothing is
    deferred), or None when no gradient has a deferred accumulation.
    Raises if an incoming gradient changed since it was deferred."""
    if not any(map(_INCOMING_OF, gradients)):
        return None
    from ..tensor import check_addends
    check_addends(gradients)
    return [0 if gradient._incoming is None else gradient._incoming[0]._ptr for gradient in gradients]


def _is_device(value) -> bool:
    from ..array import is_device_array
    return is_device_array(value)


def make_xform(transform, ctrl_ptr: int | None = None, honor_skip: bool = False) -> _native.GradXform:
    """C-ABI grad transform from a GradTransform (or from a device ctrl block)."""
    xform = _native.GradXform()
    xform.scale = 1.0
    xform.clip_coef = 1.0
    device = getattr(transform, "device", None)
    if device is not None:
        xform.unscale = int(device.unscale)
        xform.honor_skip = int(device.honor_skip)
        # The caller launches on its current stream: another stream than the
        # one that wrote the block first waits for that step's finalize.
        xform.ctrl = device.block_for_current_stream().data_ptr()
        return xform
    if transform is not None:
        if transform.scale is not None:
            xform.scale = transform.scale
            xform.unscale = 1
        if transform.clip is not None:
            xform.clip = 1
            xform.clip_coef = transform.clip
    xform.honor_skip = int(honor_skip)
    xform.ctrl = ctrl_ptr
    return xform


def is_power_of_two(value: float) -> bool:
    mantissa, _ = math.frexp(value)
    return mantissa == 0.5


__all__ = ["HIPBackend", "HIPNamespace", "AdamWHIPKernel", "Plan", "make_xform"]
