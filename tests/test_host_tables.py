"""Host unit tests of the library's plain C++ parts — the plan-table builder,
the caching memory pools, the GradScaler / clip decisions the finalize
kernels make and the kernels' workgroup -> element arithmetic — compiled
with g++ under AddressSanitizer and UndefinedBehaviorSanitizer (no GPU
involved)."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _run_sanitized(tmp_path, test_source: str, library_source: str | None) -> None:
    binary = tmp_path / Path(test_source).stem
    library = [] if library_source is None else [str(ROOT / "namitorch_amd" / "csrc" / library_source)]
    compile_cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                   "-fno-sanitize-recover=undefined", "-ffp-contract=off", "-Wall", "-Wextra", "-Werror",
                   str(ROOT / "tests" / "host" / test_source), *library, "-o", str(binary)]
    built = subprocess.run(compile_cmd, capture_output=True, text=True)
    assert built.returncode == 0, built.stderr
    ran = subprocess.run([str(binary)], capture_output=True, text=True, timeout=60,
                         env={"ASAN_OPTIONS": "detect_leaks=1", "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert ran.returncode == 0, ran.stdout + ran.stderr
    assert "all checks passed" in ran.stdout
    assert "runtime error" not in ran.stderr and "AddressSanitizer" not in ran.stderr


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
def test_plan_tables_under_sanitizers(tmp_path):
    _run_sanitized(tmp_path, "plan_tables_test.cpp", "nt_tables.cpp")


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
def test_memory_pools_under_sanitizers(tmp_path):
    _run_sanitized(tmp_path, "pool_test.cpp", "nt_pool.cpp")


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
def test_scaler_decisions_under_sanitizers(tmp_path):
    """Header-only: nt_scaler.hpp is the code the finalize and combine kernels
    run for the norm, clip, skip and loss-scale decisions."""
    _run_sanitized(tmp_path, "scaler_test.cpp", None)


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
def test_workgroup_layout_under_sanitizers(tmp_path):
    """Header-only: nt_layout.hpp's XCD-grouped grid renumbering (a bijection
    for every grid size) and task slicing (each element exactly once)."""
    _run_sanitized(tmp_path, "layout_test.cpp", None)
