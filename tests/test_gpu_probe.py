"""The streaming probe behind bench.py's ceilings (nt_stream_probe): every
supported read/write mix writes exactly what it is documented to write
(write stream w = read w mod R + read R-1, 1.0 with no reads), a read-only
probe leaves its spare stream alone, and bad arguments raise."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from namitorch_amd import _native

pytestmark = pytest.mark.gpu

MIXES = ((0, 1), (0, 3), (1, 0), (1, 1), (2, 2), (4, 0), (4, 3), (5, 4))
COUNT = 3 * 4096


def _pointers(tensors):
    return (ctypes.c_void_p * 8)(*[t.data_ptr() for t in tensors])


def _probe(reads, writes, count=COUNT):
    stream = torch.cuda.current_stream().cuda_stream
    _native.call("nt_stream_probe", _pointers(reads), len(reads), _pointers(writes), len(writes), count, stream)


@pytest.mark.parametrize("mix", MIXES, ids=[f"r{r}w{w}" for r, w in MIXES])
def test_probe_writes_what_it_documents(mix):
    nreads, nwrites = mix
    rng = np.random.default_rng(nreads * 16 + nwrites)
    host = [rng.standard_normal(COUNT).astype(np.float32) for _ in range(nreads)]
    reads = [torch.from_numpy(h).to("cuda:0") for h in host]
    writes = [torch.full((COUNT,), -7.0, dtype=torch.float32, device="cuda:0") for _ in range(max(nwrites, 1))]
    if nwrites:
        _probe(reads, writes)
    else:
        _probe_read_only(reads, writes[0])
    torch.cuda.synchronize()
    for w in range(nwrites):
        expected = (host[w % nreads] + host[nreads - 1]) if nreads else np.ones(COUNT, np.float32)
        assert np.array_equal(writes[w].cpu().numpy(), expected), w
    if nwrites == 0:
        assert torch.all(writes[0] == -7.0)


def _probe_read_only(reads, spare):
    stream = torch.cuda.current_stream().cuda_stream
    _native.call("nt_stream_probe", _pointers(reads), len(reads), _pointers([spare]), 0, COUNT, stream)


def test_probe_rejects_bad_arguments():
    a = torch.ones(COUNT, dtype=torch.float32, device="cuda:0")
    b = torch.ones(COUNT, dtype=torch.float32, device="cuda:0")
    with pytest.raises(ValueError, match="supported"):
        _probe([a, a, a], [b])
    with pytest.raises(ValueError, match="multiple of 4096"):
        _probe([a], [b], count=COUNT - 1)
    with pytest.raises(ValueError, match="multiple of 4096"):
        _probe([a], [b], count=0)
    with pytest.raises(ValueError, match="aligned"):
        _probe([a[1:]], [b])
    stream = torch.cuda.current_stream().cuda_stream
    for nreads, nwrites in ((-1, 17), (8, 0), (0, 8), (2, -1)):          # out of range, or aliases of a mix
        with pytest.raises(ValueError, match="supported"):
            _native.call("nt_stream_probe", _pointers([a]), nreads, _pointers([b]), nwrites, COUNT, stream)
    with pytest.raises(ValueError, match="NULL"):
        _native.call("nt_stream_probe", None, 1, _pointers([b]), 1, COUNT, stream)
    torch.cuda.synchronize()
    assert torch.all(b == 1.0)
