"""One HIP runtime per process, whichever package uses the GPU first.

PyTorch's ROCm builds carry their own HIP/HSA runtime libraries.  A child
process uses this package on the GPU before it imports PyTorch, then runs a
PyTorch kernel: both must work, and only one copy of each runtime library
may be mapped (two runtimes in one process leave the later one without a
device).  The reverse order is what the rest of the GPU suite does.
"""

from __future__ import annotations

import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]

SCRIPT = """
import sys
sys.path.insert(0, {root!r})
import numpy as np
import namitorch_amd as nt
assert "torch" not in sys.modules
p = nt.Parameter(np.full(4099, 0.5, np.float32), device="cuda:0")
p.grad = nt.Tensor(np.full(4099, 1e-2, np.float32), device="cuda:0")
nt.optim.AdamW([p], lr=1e-3).step()
before = p.numpy().copy()
import torch
x = torch.arange(5, device="cuda", dtype=torch.float32) * 2
assert x.cpu().tolist() == [0.0, 2.0, 4.0, 6.0, 8.0]
maps = {{line.split()[-1] for line in open("/proc/self/maps")}}
hip = sorted(m for m in maps if "libamdhip64" in m)
hsa = sorted(m for m in maps if "libhsa-runtime64" in m)
print("HIP", hip)
print("HSA", hsa)
assert len(hip) == 1 and len(hsa) == 1, (hip, hsa)
p.grad = nt.Tensor(torch.full((4099,), 1e-2, device="cuda"))
nt.optim.AdamW([p], lr=1e-3).step()
assert not np.array_equal(p.numpy(), before)
print("ok")
"""


def test_package_first_then_pytorch_share_one_runtime():
    done = subprocess.run([sys.executable, "-c", textwrap.dedent(SCRIPT.format(root=str(ROOT)))], cwd=ROOT,
                          capture_output=True, text=True, timeout=240)
    print(done.stdout[-2000:], done.stderr[-2000:], flush=True)
    assert done.returncode == 0 and done.stdout.strip().endswith("ok")
