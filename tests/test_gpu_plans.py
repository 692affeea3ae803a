"""Multi-tensor plans with gradients reallocated every step: one cached plan
is re-pointed on the device (nt_plan_set_pointers) instead of rebuilt, and
the results equal those of gradients kept in place."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import namitorch_amd as nt

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
SHAPES = [(301, 17), (17,), (4099,), (64, 64)]


def _setup(seed=3):
    rng = np.random.default_rng(seed)
    params = [nt.Parameter((rng.standard_normal(s) * 0.05).astype(np.float32), dtype="bfloat16", device=DEV)
              for s in SHAPES]
    optimizer = nt.optim.AdamW(params, lr=1e-3, master_weights=True)
    return params, optimizer


def _grad_values(k):
    rng = np.random.default_rng(100 + k)
    return [(rng.standard_normal(s) * 1e-3 * 1024).astype(np.float32) for s in SHAPES]


def _run(mode, steps=6):
    params, optimizer = _setup()
    scaler = nt.GradScaler(init_scale=1024.0)
    held = []
    stable = None
    for k in range(steps):
        values = _grad_values(k)
        if mode == "stable":
            if stable is None:
                stable = [nt.Tensor(v, dtype="bfloat16", device=DEV) for v in values]
                for p, g in zip(params, stable):
                    p.grad = g
            else:
                for g, v in zip(stable, values):
                    g.copy_(nt.Tensor(v, dtype="bfloat16", device=DEV))
        else:
            grads = [nt.Tensor(v, dtype="bfloat16", device=DEV) for v in values]
            for p, g in zip(params, grads):
                p.grad = g
            held.append(grads)                              # old gradients stay alive: new addresses
        scaler.scale(nt.Tensor(np.float32(1.0), device=DEV))
        nt.amp.fused_step(optimizer, scaler, max_norm=0.5)
    state = [optimizer.state[id(p)] for p in params]
    return ([p.bits().tobytes() for p in params], [s["master"].bits().tobytes() for s in state],
            [s["exp_avg"].bits().tobytes() for s in state], scaler.get_scale())


def test_reallocated_gradients_match_and_reuse_plans():
    backend = nt.get_backend(DEV)
    stable = _run("stable")
    before = len(backend._plans)
    moving = _run("moving")
    assert moving == stable
    # One AdamW plan and one gradient plan serve all steps of the moving run.
    assert len(backend._plans) <= before + 2


def test_alignment_change_builds_a_new_plan():
    params, optimizer = _setup()
    base = torch.zeros(sum(int(np.prod(s)) for s in SHAPES) + 64, dtype=torch.bfloat16, device=DEV)
    for k in range(3):
        values = _grad_values(k)
        offset = 8 if k == 0 else 1                         # 16-byte aligned, then 2-byte aligned
        for p, v in zip(params, values):
            n = v.size
            view = base[offset: offset + n].view(p.shape)
            view.copy_(torch.from_numpy(v).to(torch.bfloat16))
            p.grad = nt.Tensor._from_storage(view)
            offset += n
        optimizer.step()
    reference_params, reference_optimizer = _setup()
    for k in range(3):
        for p, v in zip(reference_params, _grad_values(k)):
            p.grad = nt.Tensor(v, dtype="bfloat16", device=DEV)
        reference_optimizer.step()
    assert [p.bits().tobytes() for p in params] == [p.bits().tobytes() for p in reference_params]


def test_reallocated_fp32_gradients_through_optimizer_step():
    """fp32 parameters without master weights: the full step re-points the
    cached plan; results equal gradients rewritten in place."""
    rng = np.random.default_rng(4)
    p0 = [(rng.standard_normal(s) * 0.05).astype(np.float32) for s in SHAPES]
    values = [[(np.random.default_rng(200 + k).standard_normal(s) * 1e-3).astype(np.float32) for s in SHAPES]
              for k in range(5)]
    results = []
    for mode in ("stable", "moving"):
        params = [nt.Parameter(v, device=DEV) for v in p0]
        optimizer = nt.optim.AdamW(params, lr=1e-3, weight_decay=0.1)
        held = []
        for k in range(5):
            if mode == "stable" and k > 0:
                for p, v in zip(params, values[k]):
                    p.grad.copy_(nt.Tensor(v, device=DEV))
            else:
                grads = [nt.Tensor(v, device=DEV) for v in values[k]]
                held.append(grads)
                for p, g in zip(params, grads):
                    p.grad = g
            optimizer.step()
        state = [optimizer.state[id(p)] for p in params]
        results.append(([p.bits().tobytes() for p in params], [s["exp_avg_sq"].bits().tobytes() for s in state]))
    assert results[0] == results[1]


def test_destroying_a_plan_does_not_wait_and_its_memory_is_reused():
    """Plan tables live in the library's pools: destroying a plan while
    kernels are queued returns at once (the queued work is still running
    afterwards), and a plan built next on the same stream reuses the memory.
    Cache evictions therefore cost no device synchronisation."""
    import ctypes
    import gc
    from namitorch_amd import _native, runtime
    big = nt.Parameter(np.zeros(1 << 27, np.float32), device=DEV)       # 128 M fp32: ~0.6 ms per pass
    big.grad = nt.Tensor(np.full(1 << 27, 1e-3, np.float32), device=DEV)
    optimizer = nt.optim.AdamW([big], lr=1e-3)
    optimizer.step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    grads = [torch.zeros(n, dtype=torch.bfloat16, device=DEV) for n in (5000, 70000)]
    rows = [_native.MtTensor(None, g.data_ptr(), None, None, None, g.numel(), 0, 0) for g in grads]
    layout = _native.MtLayout(-1, _native.NT_BF16, -1, -1)

    def make():
        plan = ctypes.c_void_p()
        _native.call("nt_plan_create", 0, (_native.MtTensor * 2)(*rows), 2, ctypes.byref(layout), 0, stream,
                     ctypes.byref(plan))
        return plan

    first = make()
    _native.call("nt_grad_zero", first, stream)
    torch.cuda.synchronize()
    reserved = runtime.memory_stats(0)["reserved"]
    # No garbage collection in between: collecting another test's page-locked
    # buffer would wait for the device on its own.
    gc.collect()
    gc.disable()
    try:
        for _ in range(30):
            optimizer.step()                             # ~18 ms of queued passes
        done = runtime.Event().record(stream)
        queued = not done.query()
        _native.call("nt_plan_destroy", first)
        still_queued = not done.query()
    finally:
        gc.enable()
    assert queued and still_queued                       # the destroy did not wait for the queue
    second = make()                                      # same sizes, same stream: the pool's blocks
    _native.call("nt_grad_zero", second, stream)
    assert runtime.memory_stats(0)["reserved"] == reserved
    _native.call("nt_plan_destroy", second)
    done.synchronize()
    torch.cuda.synchronize()
    assert all(not bool(g.any()) for g in grads)


def test_plan_cache_churn_across_streams_matches_oracle():
    """24 optimizers stepped in shuffled order on two library streams for
    three rounds: more (layout, stream, buffer) combinations than the plan
    cache holds, so plans are evicted and rebuilt while earlier steps may
    still be queued.  Every optimizer matches the oracle bit for bit."""
    from oracle import adam as oadam
    rng = np.random.default_rng(11)
    streams = [nt.runtime.Stream(0), nt.runtime.Stream(0)]
    runs = []
    for _ in range(24):
        sizes = [int(rng.choice([257, 2049, 4097, 12289])) for _ in range(int(rng.integers(1, 4)))]
        hosts = [(rng.standard_normal(n) * 0.02).astype(np.float32) for n in sizes]
        with nt.runtime.stream(streams[0]):
            params = [nt.Parameter(h, device=DEV) for h in hosts]
        optimizer = nt.optim.AdamW(params, lr=1e-3, weight_decay=0.01)
        runs.append((params, optimizer, [h.copy() for h in hosts], [np.zeros_like(h) for h in hosts],
                     [np.zeros_like(h) for h in hosts]))
    backend = nt.get_backend(DEV)
    for round_ in range(1, 4):
        for k in rng.permutation(len(runs)):
            params, optimizer, ref_p, ref_m, ref_v = runs[k]
            grads = [(rng.standard_normal(h.size) * 1e-3).astype(np.float32) for h in ref_p]
            with nt.runtime.stream(streams[(int(k) + round_) % 2]):
                for p, g in zip(params, grads):
                    p.grad = nt.Tensor(g, device=DEV)
                optimizer.step()
            for i, g in enumerate(grads):
                oadam.adam_step(ref_p[i], g, ref_m[i], ref_v[i], round_, lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
                                weight_decay=0.01)
        # A caller that moves an optimizer to another stream orders the streams itself.
        for stream in streams:
            stream.synchronize()
    assert len(backend._plans) <= 16
    for params, optimizer, ref_p, ref_m, ref_v in runs:
        for i, p in enumerate(params):
            state = optimizer.state[id(p)]
            assert p.numpy().tobytes() == ref_p[i].tobytes()
            assert state["exp_avg"].numpy().tobytes() == ref_m[i].tobytes()
            assert state["exp_avg_sq"].numpy().tobytes() == ref_v[i].tobytes()
            assert state["step"] == 3


def test_stream_destroyed_before_its_plan_and_block():
    """When a reference cycle is collected, Python finalizes its objects in
    any order, so a library stream can be destroyed before a plan built on it
    and before a pool block used on it.  Destroying the plan and freeing the
    block afterwards must not use the destroyed stream (nt_stream_destroy
    waits for the stream's work, so they need no ordering after it).  A step
    on a new stream, which may get the same handle, then matches the first."""
    import gc
    from namitorch_amd import _native
    backend = nt.get_backend(DEV)
    host = (np.random.default_rng(3).standard_normal(6000) * 0.02).astype(np.float32)
    grad = np.full(6000, 1e-3, np.float32)

    def two_steps():
        param = nt.Parameter(host, device=DEV)
        optimizer = nt.optim.AdamW([param], lr=1e-3)
        for _ in range(2):
            param.grad = nt.Tensor(grad, device=DEV)   # a new gradient: the plan's column is rewritten on the stream
            optimizer.step()
        return param, optimizer

    stream = nt.runtime.Stream(0)
    with nt.runtime.stream(stream):
        param, optimizer = two_steps()
        values = param.numpy()
    block = nt.DeviceArray.empty((4096,), nt.float32, DEV)    # allocated on the default stream
    block.record_stream(stream.handle)
    keys = [key for key in backend._plans if key[2] == stream.handle]
    assert keys
    print(f"destroying stream {stream.handle:#x} before {len(keys)} plan(s) and one block", flush=True)
    _native.call("nt_stream_destroy", stream.handle)          # what finalizing the Stream first does
    stream._owned = False
    for key in keys:
        del backend._plans[key]
    del optimizer, param                                       # the step memo held the plan
    gc.collect()
    del block
    fresh = nt.runtime.Stream(0)
    with nt.runtime.stream(fresh):
        again, _ = two_steps()
        assert again.numpy().tobytes() == values.tobytes()
    fresh.synchronize()


def test_destroyed_stream_blocks_serve_other_streams():
    """Blocks of a destroyed library stream are reused by allocations on
    other streams: the idle ones at once, one freed after the destroy as
    well, while the pool reserves no more memory.  The data written through
    a reused block is intact."""
    import ctypes
    from namitorch_amd import _native
    size = 3 << 20                                             # a 4 MiB pool block
    torch.cuda.synchronize()
    nt.runtime.empty_cache(0)                                  # no idle block of other tests competes
    stream = nt.runtime.Stream(0)
    first, second = ctypes.c_void_p(), ctypes.c_void_p()
    _native.call("nt_malloc", 0, size, stream.handle, ctypes.byref(first))
    _native.call("nt_malloc", 0, size, stream.handle, ctypes.byref(second))
    _native.call("nt_fill", first.value, size // 4, 4, 0x3F800000, stream.handle)
    _native.call("nt_free", first.value)                       # idle before the destroy
    reserved = nt.runtime.memory_stats(0)["reserved"]
    _native.call("nt_stream_destroy", stream.handle)
    stream._owned = False
    _native.call("nt_free", second.value)                      # freed after the destroy
    other = nt.runtime.Stream(0)
    got = []
    for _ in range(2):
        block = ctypes.c_void_p()
        _native.call("nt_malloc", 0, size, other.handle, ctypes.byref(block))
        got.append(block.value)
    assert sorted(got) == sorted([first.value, second.value])
    assert nt.runtime.memory_stats(0)["reserved"] == reserved
    _native.call("nt_fill", got[0], size // 4, 4, 0x40000000, other.handle)
    out = np.empty(size // 4, np.float32)
    _native.call("nt_memcpy_d2h", out.ctypes.data, got[0], size, other.handle)
    assert np.all(out == 2.0)
    for block in got:
        _native.call("nt_free", block)
    other.synchronize()
