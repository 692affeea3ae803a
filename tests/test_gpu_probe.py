"""The streaming probe behind bench.py's ceilings (nt_stream_probe): every
supported read/write mix writes exactly what it is documented to write
(write stream w = read (w mod R) + read R-1, 1.0 with no reads; 16-bit
streams read as bfloat16 and written truncated to bfloat16), a read-only
probe leaves its spare stream alone, and bad arguments raise."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from namitorch_amd import _native
from oracle import lowp

pytestmark = pytest.mark.gpu

# (fp32 reads, 16-bit reads, fp32 writes, 16-bit writes)
MIXES = ((0, 0, 1, 0), (0, 0, 3, 0), (1, 0, 0, 0), (1, 0, 1, 0), (2, 0, 2, 0), (4, 0, 0, 0), (4, 0, 3, 0),
         (5, 0, 4, 0), (1, 3, 1, 3), (3, 1, 3, 1))
COUNT = 3 * 4096


def _pointers(tensors):
    return (ctypes.c_void_p * 8)(*[t.data_ptr() for t in tensors])


@pytest.mark.parametrize("mix", MIXES, ids=[f"r{a}+{b}h_w{c}+{d}h" for a, b, c, d in MIXES])
def test_probe_writes_what_it_documents(mix):
    r32, r16, w32, w16 = mix
    rng = np.random.default_rng(sum(m * 7 ** i for i, m in enumerate(mix)))
    host = [rng.standard_normal(COUNT).astype(np.float32) for _ in range(r32)]
    host += [lowp.round_bf16(rng.standard_normal(COUNT).astype(np.float32)) for _ in range(r16)]
    reads = [torch.from_numpy(h).to("cuda:0") for h in host[:r32]]
    reads += [torch.from_numpy(h).to("cuda:0", torch.bfloat16) for h in host[r32:]]
    if w32 + w16:
        writes = [torch.full((COUNT,), -7.0, dtype=torch.float32, device="cuda:0") for _ in range(w32)]
        writes += [torch.full((COUNT,), -7.0, dtype=torch.bfloat16, device="cuda:0") for _ in range(w16)]
    else:
        writes = [torch.full((COUNT,), -7.0, dtype=torch.float32, device="cuda:0")]      # the spare stream
    stream = torch.cuda.current_stream().cuda_stream
    _native.call("nt_stream_probe", _pointers(reads), r32 + r16, r16, _pointers(writes), w32 + w16, w16, COUNT, stream)
    torch.cuda.synchronize()
    nreads = r32 + r16
    for w in range(w32 + w16):
        expected = (host[w % nreads] + host[nreads - 1]) if nreads else np.ones(COUNT, np.float32)
        if w < w32:
            got = writes[w].cpu().numpy()
            assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), w
        else:
            got = writes[w].cpu().view(torch.int16).numpy().view(np.uint16)
            assert np.array_equal(got, (expected.view(np.uint32) >> 16).astype(np.uint16)), w
    if w32 + w16 == 0:
        assert torch.all(writes[0] == -7.0)


def test_probe_rejects_bad_arguments():
    a = torch.ones(COUNT, dtype=torch.float32, device="cuda:0")
    b = torch.ones(COUNT, dtype=torch.float32, device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream

    def call(reads, nreads, nreads16, writes, nwrites, nwrites16, count=COUNT):
        _native.call("nt_stream_probe", reads, nreads, nreads16, writes, nwrites, nwrites16, count, stream)

    for shape in ((3, 0, 1, 0), (-1, 0, 17, 0), (8, 0, 0, 0), (0, 0, 8, 0), (2, 0, -1, 0), (4, 2, 4, 2), (1, 1, 1, 0)):
        with pytest.raises(ValueError, match="supported"):
            call(_pointers([a]), shape[0], shape[1], _pointers([b]), shape[2], shape[3])
    with pytest.raises(ValueError, match="multiple of 4096"):
        call(_pointers([a]), 1, 0, _pointers([b]), 1, 0, count=COUNT - 1)
    with pytest.raises(ValueError, match="multiple of 4096"):
        call(_pointers([a]), 1, 0, _pointers([b]), 1, 0, count=0)
    with pytest.raises(ValueError, match="aligned"):
        call(_pointers([a[1:]]), 1, 0, _pointers([b]), 1, 0)
    with pytest.raises(ValueError, match="aligned"):
        call(_pointers([a]), 1, 0, _pointers([b[2:]]), 1, 0)
    with pytest.raises(ValueError, match="NULL"):
        call(None, 1, 0, _pointers([b]), 1, 0)
    torch.cuda.synchronize()
    assert torch.all(b == 1.0)
