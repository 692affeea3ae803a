"""bench.py's host-side contract: more than one GPU is refused with a
message and a nonzero status before anything touches the GPU, and the
roofline's `traffic` comes from the committed rocprofv3 PMC summary, whose
bytes per launch sit just above the algorithmic 28 B/param of the C2 pass."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
C2_PARAMS = 124_439_808


def test_more_than_one_gpu_is_refused_with_a_message():
    done = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)
    assert done.returncode == 2
    line = json.loads(done.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_traffic_comes_from_the_committed_pmc_summary():
    sys.path.insert(0, str(ROOT))
    try:
        import bench
    finally:
        sys.path.remove(str(ROOT))
    traffic = bench.pmc_traffic()
    algorithmic = 28 * C2_PARAMS
    assert isinstance(traffic, int)
    assert algorithmic <= traffic <= 1.01 * algorithmic
    text = bench.PROFILE_PMC.read_text()
    assert "rocprofv3 --pmc FETCH_SIZE" in text and "rocprofv3 --pmc WRITE_SIZE" in text
