import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"

# The tests allocate device buffers and order work with PyTorch; make the
# package queue its launches on PyTorch's current stream of each device.
try:
    import torch
except ImportError:          # the package itself does not need PyTorch
    torch = None
if torch is not None:
    from namitorch_amd import runtime

    runtime.set_stream_provider(lambda device: torch.cuda.current_stream(device).cuda_stream)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built gfx950 library")


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN
