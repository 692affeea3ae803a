"""The package without PyTorch: each check runs in a child process in which
``import torch`` fails, so any use of PyTorch by the package shows up as an
ImportError there.

On the CPU: importing the package, host Tensors, optimizer construction and
state_dict round trips, the CPU backend's errors.  On the GPU: the
reference's per-tensor ``backend.adamw`` hook (backends/cuda/adamw.py:32-73)
on device arrays of the library's own allocator, then ``AdamW.step`` on a
stream created through the C ABI, both against the reference's golden
vectors (tests/golden/adamw_f32.npz), and the allocator's accounting.
"""

from __future__ import annotations

import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

PRELUDE = """
import sys
sys.modules["torch"] = None            # `import torch` raises ImportError from here on
import json
import numpy as np
import namitorch_amd as nt
assert "torch" not in sys.modules or sys.modules["torch"] is None
"""

HOST = """
p = nt.Parameter(np.arange(6, dtype=np.float32).reshape(2, 3), dtype="bfloat16")
assert p.dtype is nt.bfloat16 and p.bits().dtype == np.uint16
assert np.array_equal(p.numpy(), np.arange(6, dtype=np.float32).reshape(2, 3))
q = nt.Tensor(p, dtype="float64")
q[...] = 0.1
assert q.numpy()[0, 0] == 0.1 and q._version == 1
optimizer = nt.optim.AdamW([p], lr=1e-3, master_weights=True)
state = optimizer.state_dict()
optimizer.load_state_dict(state)
p.grad = nt.Tensor(np.ones((2, 3), np.float32), dtype="bfloat16")
try:
    optimizer.step()
except RuntimeError as error:
    assert "HIP devices" in str(error), error
else:
    raise AssertionError("a host step must raise")
print("HOST OK")
"""

DEVICE = """
from namitorch_amd.array import DeviceArray
from oracle import adam as oadam

DEV = "cuda:0"
data = np.load("tests/golden/adamw_f32.npz")
options = json.loads(str(data["options"]))
options["betas"] = tuple(options["betas"])


def same(got, want):
    return got.shape == want.shape and np.array_equal(got.view(np.uint32), want.view(np.uint32))


# 1. The reference protocol's per-tensor hook on the library's device arrays.
backend = nt.get_backend(DEV)
p = DeviceArray.empty(data["p0"].shape, nt.float32, DEV).upload(data["p0"])
m = DeviceArray.zeros(p.shape, nt.float32, DEV)
v = DeviceArray.zeros(p.shape, nt.float32, DEV)
g = DeviceArray.empty(p.shape, nt.float32, DEV)
assert backend.array_type is DeviceArray
assert backend.adamw.supports(p, g, m, v)
assert not backend.adamw.supports(p, p, m, v)                       # overlapping
assert not backend.adamw.supports(p, g.narrow(0, p.numel() - 1), m, v)   # shapes differ
for step, grad in enumerate(data["grads"], start=1):
    g.upload(grad)
    coefficients = oadam.coefficients(np.float32, options["lr"], options["betas"], options["eps"],
                                      options["weight_decay"], step)
    assert backend.adamw.run(p, g, m, v, coefficients=coefficients, maximize=False, update_parameter=True)
for label, array in (("p", p), ("m", m), ("v", v)):
    assert same(array.download(), data[label]), label
print("HOOK OK", flush=True)

# 2. AdamW.step through the optimizer API, queued on a stream of the C ABI.
stream = nt.runtime.Stream(0)
with nt.runtime.stream(stream):
    param = nt.Parameter(data["p0"], device=DEV)
    optimizer = nt.optim.AdamW([param], **options)
    for grad in data["grads"]:
        param.grad = nt.Tensor(grad, device=DEV)
        optimizer.step()
    stream.synchronize()
    state = optimizer.state[id(param)]
    assert same(param.numpy(), data["p"]) and same(state["exp_avg"].numpy(), data["m"])
    assert same(state["exp_avg_sq"].numpy(), data["v"]) and state["step"] == int(data["step"])
print("STEP OK", flush=True)

# 3. The caching allocator: blocks return to the pool and are reused.
import gc
before = nt.runtime.memory_stats(0)
del param, optimizer, state
gc.collect()
after = nt.runtime.memory_stats(0)
assert after["in_use"] < before["in_use"], (before, after)
with nt.runtime.stream(stream):                  # blocks are reused on the stream they were allocated on
    again = DeviceArray.empty((4099,), nt.float32, DEV)
assert nt.runtime.memory_stats(0)["reserved"] == after["reserved"]       # served from the pool
del again
nt.runtime.empty_cache(0)
assert nt.runtime.memory_stats(0)["reserved"] <= after["reserved"]
print("POOL OK", flush=True)
"""


def _run(script: str) -> str:
    done = subprocess.run([sys.executable, "-c", textwrap.dedent(PRELUDE + script)], cwd=ROOT, capture_output=True,
                          text=True, timeout=240)
    assert done.returncode == 0, done.stdout + done.stderr
    return done.stdout


def test_host_api_without_torch():
    assert "HOST OK" in _run(HOST)


@pytest.mark.gpu
def test_reference_hook_and_step_without_torch():
    out = _run(DEVICE)
    for line in ("HOOK OK", "STEP OK", "POOL OK"):
        assert line in out, out
