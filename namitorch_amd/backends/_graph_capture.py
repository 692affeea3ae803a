"""Rejection of optimizer-path operations during graph capture
(namitorch/backends/_graph_capture.py:12-14).

The reference rejects these operations while one of its CUDA graphs is
being prepared or captured:
- optimizer steps;
- GradScaler calls;
- in-place Tensor updates;
- host reads of Tensors;
- moving optimizer state.

Here the capture in question is a HIP stream capture
(``hipStreamBeginCapture``, also what ``torch.cuda.graph`` does) on the
calling thread's current stream of a device this package has used
(``nt_stream_capturing``).  The same operations raise the reference's
RuntimeError, with its message, before anything is queued.
"""

from __future__ import annotations

import ctypes

from .. import _native, runtime


def capturing() -> bool:
    """True while the calling thread's current stream of a device with a
    HIP backend is being captured.  Before any backend exists no device
    work of this package can be in progress, so nothing is captured."""
    from . import _backends
    status = ctypes.c_int32()
    for device in list(_backends):
        if device.type == "cpu":
            continue
        _native.call("nt_stream_capturing", runtime.current_stream(device.index), ctypes.byref(status))
        if status.value:
            return True
    return False


def reject_during_capture(operation: str) -> None:
    if capturing():
        raise RuntimeError(f"{operation} is not supported in CUDA graph preparation or capture; "
                           "only deterministic FP32 inference is supported.")
