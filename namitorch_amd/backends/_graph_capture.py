"""Rejection of optimizer-path operations during graph capture
(namitorch/backends/_graph_capture.py:12-14).

The reference rejects these operations while one of its CUDA graphs is
being prepared or captured:
- optimizer steps;
- GradScaler calls;
- in-place Tensor updates;
- host reads of Tensors;
- moving optimizer state.

Here the capture in question is a HIP stream capture (``torch.cuda.graph``,
``hipStreamBeginCapture``) on the calling thread's current stream.  The
same operations raise the reference's RuntimeError, with its message,
before anything is queued.
"""

from __future__ import annotations

import torch


def capturing() -> bool:
    """True while the calling thread's current stream is being captured.
    Without an initialised HIP runtime no capture can be in progress."""
    return torch.cuda.is_initialized() and torch.cuda.is_current_stream_capturing()


def reject_during_capture(operation: str) -> None:
    if capturing():
        raise RuntimeError(f"{operation} is not supported in CUDA graph preparation or capture; "
                           "only deterministic FP32 inference is supported.")
