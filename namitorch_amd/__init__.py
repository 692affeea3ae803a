"""namitorch_amd — NamiTorch's optimizer-step hot path, native to the MI355X.

AdamW.step(), GradScaler unscale_/finite check/update and clip_grad_norm_
behind NamiTorch's Python API, computed by hand-written gfx950 HIP kernels
(``libnamitorch_amd.so``, C ABI in ``include/namitorch_amd.h``) reached
through ctypes.  Optimizer and scaler state read and write NamiTorch's
``.nt`` archive and checkpoint layout (``serialization``, ``checkpoint``).

The package needs NumPy and the library, not PyTorch: device memory comes
from the library's caching allocator (``array.DeviceArray``) and streams and
events from its C ABI (``runtime``).  Device arrays of other frameworks are
wrapped without a copy, and ``runtime.set_stream_provider`` makes launches
follow another framework's current stream.
"""

from . import amp, checkpoint, grads, optim, runtime, serialization
from .array import DeviceArray
from .amp import GradScaler
from .checkpoint import load_checkpoint, save_checkpoint
from .grads import accumulate_grads
from .serialization import SerializationError, load, save
from .backends import enable_fused_kernels, fused_kernels_enabled, get_backend
from .device import Device, device
from .dtype import DType, bfloat16, float16, float32, float64
from .tensor import Parameter, Tensor, enable_grad, is_grad_enabled, no_grad, tensor

__all__ = [
    "amp", "checkpoint", "grads", "accumulate_grads", "optim", "runtime", "DeviceArray", "serialization", "GradScaler", "SerializationError", "save", "load",
    "save_checkpoint", "load_checkpoint", "enable_fused_kernels", "fused_kernels_enabled", "get_backend",
    "Device", "device", "DType", "bfloat16", "float16", "float32", "float64",
    "Parameter", "Tensor", "enable_grad", "is_grad_enabled", "no_grad", "tensor",
]
