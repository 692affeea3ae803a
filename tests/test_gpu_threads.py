"""Threads: launches go to the calling thread's current stream, plans are
cached per stream, and the step memo and control blocks belong to their
optimizer and scaler.  Two threads stepping their own optimizers on their
own streams at the same time (plain AdamW, and the AMP fused step with a
skipped step and clip decisions settled from both threads) give results,
step counts and version counters identical to the same work run one after
the other."""

from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

import namitorch_amd as nt
from oracle import lowp

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
SHAPES = [(257, 129), (129,), (4096, 3), (5000,)]


def _work(seed: int, amp: bool, steps: int = 8):
    rng = np.random.Generator(np.random.PCG64(seed))
    dtype = "bfloat16" if amp else "float32"
    host = [(rng.standard_normal(s) * 0.05).astype(np.float32) for s in SHAPES]
    params = [nt.Parameter(lowp.round_bf16(h) if amp else h, dtype=dtype, device=DEV) for h in host]
    optimizer = nt.optim.AdamW([{"params": params[:2], "weight_decay": 0.1}, {"params": params[2:], "weight_decay": 0.0}],
                               lr=1e-3, master_weights=amp)
    scaler = nt.GradScaler(init_scale=1024.0, growth_interval=3) if amp else None
    loss = nt.Tensor(np.float32(1.0), device=DEV)
    for k in range(steps):
        for p, s in zip(params, SHAPES):
            g = (rng.standard_normal(s) * 1e-3 * (1024.0 if amp else 1.0)).astype(np.float32)
            if amp and k == 4:
                g.reshape(-1)[3] = np.inf
            p.grad = nt.Tensor(g, dtype="float16" if amp else "float32", device=DEV)
        if amp:
            scaler.scale(loss)
            nt.amp.fused_step(optimizer, scaler, max_norm=0.05)
        else:
            optimizer.step()
    torch.cuda.current_stream().synchronize()
    states = [optimizer.state[id(p)] for p in params]
    out = [p.numpy() for p in params] + [s["exp_avg"].numpy() for s in states] + [s["exp_avg_sq"].numpy() for s in states]
    if amp:
        out += [s["master"].numpy() for s in states] + [np.float64(scaler.get_scale())]
    # Version reads settle every pending device-decided step, the other
    # thread's included: each step's rollback must still run once.
    versions = [t._version for t in params + [p.grad for p in params]]
    versions += [s[key]._version for s in states for key in ("exp_avg", "exp_avg_sq")]
    return out + [np.array([s["step"] for s in states]), np.array(versions)]


@pytest.mark.parametrize("amp", [False, True])
def test_two_threads_on_their_own_streams_match_sequential(amp):
    seeds = (11, 12)
    expected = [_work(seed, amp) for seed in seeds]
    results: dict = {}
    errors: list = []
    start = threading.Barrier(len(seeds))

    def worker(seed):
        try:
            stream = torch.cuda.Stream(device=DEV)
            with torch.cuda.stream(stream):
                start.wait()
                results[seed] = _work(seed, amp)
        except BaseException as error:                      # reported in the main thread
            errors.append(error)

    threads = [threading.Thread(target=worker, args=(seed,)) for seed in seeds]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join(timeout=120)
    assert not errors, errors
    for seed, want in zip(seeds, expected):
        got = results[seed]
        assert len(got) == len(want)
        for a, b in zip(got, want):
            a, b = np.asarray(a), np.asarray(b)
            assert a.shape == b.shape and a.dtype == b.dtype
            assert np.array_equal(a.view(f"u{a.itemsize}"), b.view(f"u{b.itemsize}")), seed
