"""Streams, events, the current stream and pinned host memory, over the
library's C ABI (``nt_stream_*``, ``nt_event_*``, ``nt_host_alloc``).

The reference takes these from CuPy (``backends/_cuda_execution.py``,
``cuda/streams.py``): every launch goes to the calling thread's current
stream (``backends/cuda/adamw.py:71``).  Here the current stream of a device
is, in order of precedence:

* the innermost ``with stream(s):`` block of the calling thread;
* a stream *provider* installed with :func:`set_stream_provider`, so a
  program that already manages streams with another GPU framework can have
  this package follow that framework's current stream (for PyTorch:
  ``set_stream_provider(lambda d: torch.cuda.current_stream(d).cuda_stream)``);
* the device's null stream.

Streams created here run at the default priority.
"""

from __future__ import annotations

import ctypes
import threading
import weakref
from contextlib import contextmanager

import numpy as np

from . import _native

_local = threading.local()
_provider = None


def set_stream_provider(provider) -> None:
    """Install (or, with None, remove) a function ``provider(device) ->
    stream handle`` that names the current stream when no ``with stream(...)``
    block is active."""
    global _provider
    if provider is not None and not callable(provider):
        raise TypeError("The stream provider must be callable or None.")
    _provider = provider


def _stacks() -> dict:
    stacks = getattr(_local, "stacks", None)
    if stacks is None:
        stacks = _local.stacks = {}
    return stacks


def current_stream(device: int) -> int:
    """Handle (a hipStream_t as an int; 0 = the null stream) of the calling
    thread's current stream on `device`."""
    stack = _stacks().get(device)
    if stack:
        return stack[-1][0]
    provider = _provider
    if provider is not None:
        return int(provider(device) or 0)
    return 0


def current_stream_owner(device: int):
    """The :class:`Stream` object behind the current stream of `device` when
    a ``with stream(Stream)`` block selected it, else None.  Holders of
    library objects bound to a stream (plans) keep it alive with this."""
    stack = _stacks().get(device)
    return stack[-1][1] if stack else None


@contextmanager
def device_scope(index: int):
    """Make device `index` the calling thread's current HIP device inside the
    block (restored after), so that null-stream work lands on it."""
    previous = ctypes.c_int32()
    _native.call("nt_get_device", ctypes.byref(previous))
    if previous.value == index:
        yield
        return
    _native.call("nt_set_device", index)
    try:
        yield
    finally:
        _native.call("nt_set_device", previous.value)


class Stream:
    """A HIP stream of one device: created here (and destroyed with this
    object), or wrapping a handle owned elsewhere (``Stream.wrap``)."""

    __slots__ = ("handle", "device", "_owned", "__weakref__")

    def __init__(self, device: int = 0):
        handle = ctypes.c_void_p()
        _native.call("nt_stream_create", device, ctypes.byref(handle))
        self.handle = handle.value or 0
        self.device = device
        self._owned = True

    @classmethod
    def wrap(cls, handle: int, device: int = 0) -> "Stream":
        wrapped = cls.__new__(cls)
        wrapped.handle = int(handle or 0)
        wrapped.device = device
        wrapped._owned = False
        return wrapped

    def synchronize(self) -> None:
        _native.call("nt_stream_synchronize", self.handle)

    def wait_event(self, event: "Event") -> None:
        _native.call("nt_stream_wait_event", self.handle, event.handle)

    def wait_stream(self, other: "Stream") -> None:
        marker = Event()
        marker.record(other.handle)
        self.wait_event(marker)

    def __eq__(self, other):
        return isinstance(other, Stream) and other.handle == self.handle

    def __hash__(self):
        return hash(self.handle)

    def __del__(self):
        try:                           # module globals may already be gone at interpreter exit
            if self._owned and self.handle and not _native.shutting_down():
                _native.load().nt_stream_destroy(self.handle)
        except Exception:
            pass


@contextmanager
def stream(selected):
    """Make `selected` (a Stream, or ``(handle, device)``) the calling thread's
    current stream of its device inside the block."""
    if isinstance(selected, Stream):
        handle, device, owner = selected.handle, selected.device, selected
    else:
        handle, device, owner = int(selected[0] or 0), int(selected[1]), None
    stack = _stacks().setdefault(device, [])
    stack.append((handle, owner))
    try:
        yield selected
    finally:
        stack.pop()


class Event:
    """A HIP event (``timing=True`` for :meth:`elapsed_time`)."""

    __slots__ = ("handle", "__weakref__")

    def __init__(self, timing: bool = False):
        handle = ctypes.c_void_p()
        _native.call("nt_event_create", int(timing), ctypes.byref(handle))
        self.handle = handle.value

    def record(self, stream_handle: int) -> "Event":
        _native.call("nt_event_record", self.handle, stream_handle)
        return self

    def synchronize(self) -> None:
        _native.call("nt_event_synchronize", self.handle)

    def query(self) -> bool:
        done = ctypes.c_int32()
        _native.call("nt_event_query", self.handle, ctypes.byref(done))
        return bool(done.value)

    def elapsed_time(self, end: "Event") -> float:
        milliseconds = ctypes.c_float()
        _native.call("nt_event_elapsed", self.handle, end.handle, ctypes.byref(milliseconds))
        return float(milliseconds.value)

    def __del__(self):
        try:                           # module globals may already be gone at interpreter exit
            if self.handle and not _native.shutting_down():
                _native.load().nt_event_destroy(self.handle)
        except Exception:
            pass


def _release_host(address: int) -> None:
    try:                               # module globals may already be gone at interpreter exit
        if not _native.shutting_down():
            _native.load().nt_host_free(address)
    except Exception:
        pass


def pinned(nbytes: int) -> np.ndarray:
    """A uint8 NumPy array over page-locked host memory (released with the
    array), for asynchronous device-to-host snapshots."""
    address = ctypes.c_void_p()
    _native.call("nt_host_alloc", max(1, nbytes), ctypes.byref(address))
    buffer = (ctypes.c_uint8 * max(1, nbytes)).from_address(address.value)
    array = np.frombuffer(buffer, dtype=np.uint8, count=nbytes)
    weakref.finalize(buffer, _release_host, address.value)
    array.flags.writeable = True
    return array


# Releasing page-locked memory waits for the whole device, which would stall
# the host behind every kernel queued so far; buffers that are used once per
# optimizer step are therefore recycled through this pool.
_PINNED_KEEP = 64                  # idle buffers kept per size
_pinned_idle: dict = {}            # size -> idle arrays


def take_pinned(nbytes: int) -> np.ndarray:
    """A page-locked buffer from the pool (or a new one).  Safe across
    threads: another thread may empty the list between the look and the pop."""
    idle = _pinned_idle.get(nbytes)
    if idle:
        try:
            return idle.pop()
        except IndexError:
            pass
    return pinned(nbytes)


def give_pinned(array: np.ndarray) -> None:
    """Return a buffer of :func:`take_pinned` to the pool.  The caller
    guarantees that no queued copy still writes or reads it; a buffer never
    given back is released when it is garbage collected."""
    idle = _pinned_idle.setdefault(array.nbytes, [])
    if len(idle) < _PINNED_KEEP:
        idle.append(array)


# ---- control-block mirrors -------------------------------------------------------------------
# Fine-grained page-locked host copies of control blocks (``nt_amp_mirror``),
# written by the finalize kernel itself so that reading an iteration's
# decisions needs no event on the launch stream.  Slabs are allocated once
# and kept (releasing page-locked memory waits for the device).  A mirror is
# reused only after its ``ready`` flag was seen set: no earlier launch still
# writes it then.
_MIRROR_SLAB = 256
_mirror_lock = threading.Lock()
_mirror_idle: list = []            # addresses free for reuse
_mirror_waiting: list = []         # given back before their writer was seen to finish
_mirror_returned: list = []        # (address, launched) given back, not yet sorted
_mirror_slabs: list = []


def take_mirror():
    """A cleared ``_native.AmpMirror`` (``ready`` == 0) for the next finalize."""
    with _mirror_lock:
        while True:
            try:
                address, launched = _mirror_returned.pop()
            except IndexError:
                break
            ready = _native.AmpMirror.from_address(address).ready
            (_mirror_idle if ready or not launched else _mirror_waiting).append(address)
        if not _mirror_idle and _mirror_waiting:
            still = []
            for address in _mirror_waiting:
                (_mirror_idle if _native.AmpMirror.from_address(address).ready else still).append(address)
            _mirror_waiting[:] = still
        if not _mirror_idle:
            slab = ctypes.c_void_p()
            _native.call("nt_mirror_alloc", _MIRROR_SLAB, ctypes.byref(slab))
            _mirror_slabs.append(slab.value)
            size = ctypes.sizeof(_native.AmpMirror)
            _mirror_idle.extend(slab.value + k * size for k in reversed(range(_MIRROR_SLAB)))
        address = _mirror_idle.pop()
    mirror = _native.AmpMirror.from_address(address)
    mirror.ready = 0
    return mirror


def give_mirror(mirror, launched: bool = True) -> None:
    """Return a mirror of :func:`take_mirror`.  `launched`: a kernel was
    queued to write it (it is reused once its flag shows that write done).
    Takes no lock (one list append), so a finalizer may give a mirror back
    while this thread is inside :func:`take_mirror`; the next take sorts it."""
    _mirror_returned.append((ctypes.addressof(mirror), launched))


def memory_stats(device: int = 0) -> dict:
    """Bytes of device memory handed out and held by the library's pool."""
    in_use = ctypes.c_uint64()
    reserved = ctypes.c_uint64()
    _native.call("nt_memory_stats", device, ctypes.byref(in_use), ctypes.byref(reserved))
    return {"in_use": in_use.value, "reserved": reserved.value}


def empty_cache(device: int = 0) -> None:
    """Return the pool's unused blocks to the device (waits for the device)."""
    _native.call("nt_empty_cache", device)


__all__ = ["Stream", "Event", "stream", "current_stream", "current_stream_owner", "set_stream_provider", "pinned",
           "take_pinned", "give_pinned", "take_mirror", "give_mirror", "memory_stats", "empty_cache", "device_scope"]
