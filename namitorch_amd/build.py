"""Build recipe of the gfx950 shared library ``libnamitorch_amd.so``.

One ``hipcc`` invocation compiles every ``csrc/*.hip`` file for gfx950 (and the
host-only ``csrc/*.cpp``) and
links them into ``namitorch_amd/_lib/libnamitorch_amd.so`` (in-tree, so the
built library travels with the source tree).  The flags fix the numerics the
kernels rely on:

* ``-ffp-contract=off`` — no FMA contraction: each fp32 multiply and add
  rounds separately, as NumPy's ufuncs do;
* ``-fhip-fp32-correctly-rounded-divide-sqrt`` — IEEE-correct fp32 ``/`` and
  ``sqrt``;
* ``-fno-gpu-flush-denormals-to-zero`` — fp32 subnormals are kept;
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` — no packed-fp32
  instructions are generated.

Run ``python -m namitorch_amd.build`` or call :func:`build`.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR / "csrc"
INCLUDE_DIR = PACKAGE_DIR.parent / "include"
LIB_DIR = PACKAGE_DIR / "_lib"
LIB_PATH = LIB_DIR / "libnamitorch_amd.so"
ARCH = "gfx950"

NUMERIC_FLAGS = (
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
)


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc was not found; the gfx950 library cannot be built.")
    return found


def sources() -> list[Path]:
    """The HIP sources plus the plain C++ plan-table builder."""
    return sorted(SOURCE_DIR.glob("*.hip")) + sorted(SOURCE_DIR.glob("*.cpp"))


def command(output: Path = LIB_PATH) -> list[str]:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        *NUMERIC_FLAGS,
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-function",
        f"-I{INCLUDE_DIR}",
        *(str(path) for path in sources()),
        "-o", str(output),
    ]


def build(verbose: bool = False) -> Path:
    """Compile the library for gfx950; returns the path of the built .so."""
    LIB_DIR.mkdir(exist_ok=True)
    temporary = LIB_PATH.with_name(LIB_PATH.name + f".tmp{os.getpid()}")
    cmd = command(temporary)
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        temporary.unlink(missing_ok=True)
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{result.stdout}\n{result.stderr}")
    os.replace(temporary, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
