"""ctypes binding of ``libnamitorch_amd.so`` (the C ABI in ``include/namitorch_amd.h``).

The library is loaded on first use from ``namitorch_amd/_lib``.  There is no
fallback: when the library is missing every device operation raises
:class:`NativeLibraryError`, which names the build command.
"""

from __future__ import annotations

import atexit
import ctypes
import importlib.util
import os
import sys
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libnamitorch_amd.so"

NT_OK = 0
NT_ERR_VALUE = -1
NT_ERR_TYPE = -2
NT_ERR_RUNTIME = -3
NT_ERR_HIP = -4

NT_DTYPE_NONE = -1
NT_F32 = 0
NT_F16 = 1
NT_BF16 = 2
NT_F64 = 3

NT_MAX_SLOTS = 16
NT_MAX_COMBINE = 8
NT_FINALIZE_SCALER_UPDATE = 1
NT_FINALIZE_CLIP_IF_FINITE = 2
ABI_VERSION = 4
NT_NORM_POW_GUARD = 1
NT_OP_MUL = 0
NT_OP_DIV = 1

c_void_p = ctypes.c_void_p
c_int32 = ctypes.c_int32
c_int64 = ctypes.c_int64
c_uint64 = ctypes.c_uint64
c_float = ctypes.c_float
c_double = ctypes.c_double


class NativeLibraryError(RuntimeError):
    """The gfx950 library is not built or cannot be loaded."""


class MtTensor(ctypes.Structure):
    _fields_ = [
        ("param", c_void_p),
        ("grad", c_void_p),
        ("exp_avg", c_void_p),
        ("exp_avg_sq", c_void_p),
        ("model_copy", c_void_p),
        ("numel", c_uint64),
        ("slot", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


class MtLayout(ctypes.Structure):
    _fields_ = [
        ("param_dtype", c_int32),
        ("grad_dtype", c_int32),
        ("state_dtype", c_int32),
        ("copy_dtype", c_int32),
    ]


class AdamWCoefs(ctypes.Structure):
    _fields_ = [(name, c_float) for name in (
        "lr", "beta1", "beta2", "complement1", "complement2",
        "eps", "weight_decay", "decay_factor", "correction1", "correction2",
    )] + [("maximize", c_int32), ("update_parameter", c_int32), ("coupled_weight_decay", c_int32), ("reserved", c_int32)]


class AdamWCoefs64(ctypes.Structure):
    _fields_ = [(name, c_double) for name in (
        "lr", "beta1", "beta2", "complement1", "complement2",
        "eps", "weight_decay", "decay_factor", "correction1", "correction2",
    )] + [("maximize", c_int32), ("update_parameter", c_int32), ("coupled_weight_decay", c_int32), ("reserved", c_int32)]


class AmpCtrl(ctypes.Structure):
    _fields_ = [
        ("sumsq", c_double),
        ("amax", c_double),
        ("norm", c_double),
        ("clip_coef", c_double),
        ("scale", c_float),
        ("scale_used", c_float),
        ("found_inf", c_int32),
        ("has_nan", c_int32),
        ("clip", c_int32),
        ("skip", c_int32),
        ("growth_tracker", c_int32),
        ("iterations", c_int32),
        ("skipped", c_int32),
        ("reserved", c_int32),
    ]


class AmpMirror(ctypes.Structure):
    """Page-locked host copy of a control block (``nt_amp_mirror``): the
    finalize stores ``ctrl``, then sets ``ready`` to 1."""
    _fields_ = [("ctrl", AmpCtrl), ("ready", c_int32), ("reserved", c_int32)]


class GradXform(ctypes.Structure):
    _fields_ = [
        ("scale", c_float),
        ("unscale", c_int32),
        ("clip_coef", c_double),
        ("clip", c_int32),
        ("honor_skip", c_int32),
        ("ctrl", c_void_p),
    ]


assert ctypes.sizeof(MtTensor) == 56
assert ctypes.sizeof(AdamWCoefs) == 56
assert ctypes.sizeof(AdamWCoefs64) == 96
assert ctypes.sizeof(AmpCtrl) == 72
assert ctypes.sizeof(AmpMirror) == 80
assert ctypes.sizeof(GradXform) == 32

# name -> (restype, argtypes); every entry point returns an int32 status.
SIGNATURES = {
    "nt_last_error": (ctypes.c_char_p, []),
    "nt_abi_version": (c_int32, []),
    "nt_hip_version": (c_int32, [ctypes.POINTER(c_int32), ctypes.POINTER(c_int32)]),
    "nt_device_count": (c_int32, [ctypes.POINTER(c_int32)]),
    "nt_device_arch": (c_int32, [c_int32, ctypes.c_char_p, c_int32]),
    "nt_set_device": (c_int32, [c_int32]),
    "nt_get_device": (c_int32, [ctypes.POINTER(c_int32)]),
    "nt_stream_synchronize": (c_int32, [c_void_p]),
    "nt_memcpy_d2h": (c_int32, [c_void_p, c_void_p, c_uint64, c_void_p]),
    "nt_memcpy_h2d": (c_int32, [c_void_p, c_void_p, c_uint64, c_void_p]),
    "nt_adamw_f32": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p] + [c_float] * 10 + [c_int32, c_int32, c_uint64, c_void_p]),
    "nt_plan_create": (c_int32, [c_int32, ctypes.POINTER(MtTensor), c_int32, ctypes.POINTER(MtLayout), c_int64, c_void_p, ctypes.POINTER(c_void_p)]),
    "nt_plan_destroy": (c_int32, [c_void_p]),
    "nt_plan_info": (c_int32, [c_void_p, ctypes.POINTER(c_uint64), ctypes.POINTER(c_int32), ctypes.POINTER(c_int64)]),
    "nt_adamw_mt": (c_int32, [c_void_p, c_void_p, c_int32, ctypes.POINTER(GradXform), c_void_p]),
    "nt_amp_prepass": (c_int32, [c_void_p, c_float, c_int32, c_void_p, c_void_p]),
    "nt_amp_finalize": (c_int32, [c_void_p, c_void_p, c_void_p, c_double, c_double, c_int32, c_double, c_double, c_int32,
                                  c_void_p, c_void_p]),
    "nt_amp_combine": (c_int32, [ctypes.POINTER(c_void_p), c_int32, c_void_p, c_double, c_double, c_int32, c_double,
                                 c_double, c_int32, ctypes.POINTER(c_void_p), c_void_p]),
    "nt_grad_norm_pow": (c_int32, [c_void_p, c_void_p, c_double, c_double, c_float, c_int32, c_int32, c_int32, c_void_p]),
    "nt_grad_apply": (c_int32, [c_void_p, ctypes.POINTER(GradXform), c_void_p]),
    "nt_grad_zero": (c_int32, [c_void_p, c_void_p]),
    "nt_plan_set_pointers": (c_int32, [c_void_p, c_int32, ctypes.POINTER(c_void_p), c_int32, c_void_p]),
    "nt_grad_accumulate": (c_int32, [c_void_p, c_int32, c_void_p]),
    "nt_ctrl_reset": (c_int32, [c_void_p, c_float, c_int32, c_void_p]),
    "nt_ctrl_carry": (c_int32, [c_void_p, c_void_p, c_void_p]),
    "nt_tensor_scalar": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_double, c_int32, c_void_p, c_uint64, c_void_p]),
    "nt_any_negative": (c_int32, [c_void_p, c_int32, c_uint64, c_void_p, c_void_p]),
    "nt_amp_flat_stats_noalloc": (c_int32, [c_int32, c_void_p, c_int32, c_uint64, c_float, c_int32, c_void_p, c_void_p,
                                            c_double, c_double, c_int32, c_double, c_double, c_int32, c_void_p]),
    "nt_stream_probe": (c_int32, [ctypes.POINTER(c_void_p), c_int32, c_int32, ctypes.POINTER(c_void_p), c_int32, c_int32,
                                  c_uint64, c_void_p]),
    "nt_malloc": (c_int32, [c_int32, c_uint64, c_void_p, ctypes.POINTER(c_void_p)]),
    "nt_free": (c_int32, [c_void_p]),
    "nt_record_stream": (c_int32, [c_void_p, c_void_p]),
    "nt_memory_stats": (c_int32, [c_int32, ctypes.POINTER(c_uint64), ctypes.POINTER(c_uint64)]),
    "nt_empty_cache": (c_int32, [c_int32]),
    "nt_host_alloc": (c_int32, [c_uint64, ctypes.POINTER(c_void_p)]),
    "nt_host_free": (c_int32, [c_void_p]),
    "nt_mirror_alloc": (c_int32, [c_int32, ctypes.POINTER(c_void_p)]),
    "nt_mirror_free": (c_int32, [c_void_p]),
    "nt_mirror_wait": (c_int32, [c_void_p, c_void_p]),
    "nt_stream_create": (c_int32, [c_int32, ctypes.POINTER(c_void_p)]),
    "nt_stream_destroy": (c_int32, [c_void_p]),
    "nt_stream_wait_event": (c_int32, [c_void_p, c_void_p]),
    "nt_event_create": (c_int32, [c_int32, ctypes.POINTER(c_void_p)]),
    "nt_event_destroy": (c_int32, [c_void_p]),
    "nt_event_record": (c_int32, [c_void_p, c_void_p]),
    "nt_event_synchronize": (c_int32, [c_void_p]),
    "nt_event_query": (c_int32, [c_void_p, ctypes.POINTER(c_int32)]),
    "nt_event_elapsed": (c_int32, [c_void_p, c_void_p, ctypes.POINTER(c_float)]),
    "nt_memcpy_async": (c_int32, [c_void_p, c_void_p, c_uint64, c_int32, c_void_p]),
    "nt_fill": (c_int32, [c_void_p, c_uint64, c_int32, c_uint64, c_void_p]),
    "nt_cast": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_uint64, c_void_p]),
    "nt_pointer_device": (c_int32, [c_void_p, ctypes.POINTER(c_int32)]),
    "nt_stream_capturing": (c_int32, [c_void_p, ctypes.POINTER(c_int32)]),
}

NT_COPY_H2D = 1
NT_COPY_D2H = 2
NT_COPY_D2D = 3

# Set at interpreter exit: objects released after that point leave their
# device memory, streams and events to the process teardown instead of
# calling into a HIP runtime that may already be gone.
_exiting = False


def _mark_exit() -> None:
    global _exiting
    _exiting = True


atexit.register(_mark_exit)


def shutting_down() -> bool:
    return _exiting

_lock = threading.Lock()
_lib = None


def _share_pytorch_runtime() -> None:
    """Keep one HIP runtime in the process.

    PyTorch's ROCm builds carry their own HIP and HSA runtime libraries
    (``torch/lib``).  When PyTorch was imported first, the dynamic linker
    binds this library's ``libamdhip64`` dependency to PyTorch's copy by
    name, and both share one runtime.  When this library loads first, it
    would bind to the system runtime, and a second runtime loaded later by
    PyTorch finds no device.  So when PyTorch is installed but not loaded
    yet, its two runtime libraries are loaded first (PyTorch itself is not
    imported), and either package may then use the GPU first.  Setting
    ``NT_SYSTEM_HIP_RUNTIME=1`` keeps the system runtime."""
    if os.environ.get("NT_SYSTEM_HIP_RUNTIME") == "1" or "torch" in sys.modules:
        return
    try:
        spec = importlib.util.find_spec("torch")
    except (ImportError, ValueError):
        return
    if spec is None or spec.origin is None:
        return
    runtime_dir = Path(spec.origin).parent / "lib"
    for name in ("libhsa-runtime64.so", "libamdhip64.so"):
        path = runtime_dir / name
        if not path.exists():
            return
        try:
            ctypes.CDLL(str(path), mode=ctypes.RTLD_GLOBAL)
        except OSError:
            return


def load() -> ctypes.CDLL:
    """Load the library (once) and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise NativeLibraryError(
                f"{LIB_PATH} is missing; build it with `python -m namitorch_amd.build` "
                "(hipcc --offload-arch=gfx950)."
            )
        _share_pytorch_runtime()
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as error:
            raise NativeLibraryError(f"cannot load {LIB_PATH}: {error}") from error
        for name, (restype, argtypes) in SIGNATURES.items():
            function = getattr(lib, name)
            function.restype = restype
            function.argtypes = argtypes
        if lib.nt_abi_version() != ABI_VERSION:
            raise NativeLibraryError(f"{LIB_PATH} has ABI {lib.nt_abi_version()}, expected {ABI_VERSION}; rebuild it.")
        _check_runtime(lib)
        _lib = lib
        return lib


HIP_VERSIONS = None     # (built, bound runtime), both HIP_VERSION-encoded, once loaded


def _check_runtime(lib) -> None:
    """The HIP runtime the library is bound to (PyTorch's bundled one or the
    system's) must have the major version of the HIP headers the library was
    built with: HIP keeps its runtime interface within a major version."""
    global HIP_VERSIONS
    built, runtime = c_int32(), c_int32()
    if lib.nt_hip_version(ctypes.byref(built), ctypes.byref(runtime)) != NT_OK:
        return                 # no runtime answer (no driver): nothing to compare, device calls fail on their own
    HIP_VERSIONS = (built.value, runtime.value)
    if built.value // 10_000_000 != runtime.value // 10_000_000:
        raise NativeLibraryError(
            f"{LIB_PATH} was built with HIP {_hip_text(built.value)} but is bound to HIP runtime "
            f"{_hip_text(runtime.value)}: rebuild it with that ROCm, or set NT_SYSTEM_HIP_RUNTIME=1 to bind it to the "
            f"system runtime.")


def _hip_text(version: int) -> str:
    return f"{version // 10_000_000}.{version // 100_000 % 100}.{version % 100_000}"


_ERRORS = {NT_ERR_VALUE: ValueError, NT_ERR_TYPE: TypeError, NT_ERR_RUNTIME: RuntimeError, NT_ERR_HIP: RuntimeError}


def check(status: int) -> None:
    """Raise the exception class a negative status code names."""
    if status == NT_OK:
        return
    message = load().nt_last_error().decode("utf-8", "replace")
    raise _ERRORS.get(status, RuntimeError)(message)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))
