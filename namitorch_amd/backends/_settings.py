"""Global switch for fused kernels (namitorch/backends/_settings.py:1-12).

``AdamW(fused=None)`` honours it.  Turning it off selects the array path,
which on HIP devices runs the same kernels in the reference's unfused
operation order (bit-identical for float32)."""

_fused_kernels_enabled = True


def enable_fused_kernels(mode):
    global _fused_kernels_enabled
    if type(mode) is not bool:
        raise TypeError("Fused kernel mode must be a Python bool.")
    _fused_kernels_enabled = mode


def fused_kernels_enabled():
    return _fused_kernels_enabled
