"""namitorch_amd — NamiTorch's optimizer-step hot path, native to the MI355X.

AdamW.step(), GradScaler unscale_/finite check/update and clip_grad_norm_
behind NamiTorch's Python API, computed by hand-written gfx950 HIP kernels
(``libnamitorch_amd.so``, C ABI in ``include/namitorch_amd.h``) reached
through ctypes.
"""

from . import amp, optim
from .amp import GradScaler
from .backends import enable_fused_kernels, fused_kernels_enabled, get_backend
from .device import Device, device
from .dtype import DType, bfloat16, float16, float32, float64
from .tensor import Parameter, Tensor, enable_grad, is_grad_enabled, no_grad, tensor

__all__ = [
    "amp", "optim", "GradScaler", "enable_fused_kernels", "fused_kernels_enabled", "get_backend",
    "Device", "device", "DType", "bfloat16", "float16", "float32", "float64",
    "Parameter", "Tensor", "enable_grad", "is_grad_enabled", "no_grad", "tensor",
]
