"""Optimizer-step benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c2,c1,c3,c4,c5,c4s8,c5s8,ceilings] [--no-cpu]

Headline (the JSON line's ``value``): configuration C2 — multi-tensor fp32
AdamW over the GPT-2-124M parameter list (148 tensors, 124,439,808 params,
weight decay 0.1 on matrices and 0 on vectors, lr 3e-4, betas (0.9, 0.999),
eps 1e-8), one ``optimizer.step()`` through the public API per step, inputs
resident in HBM.  ``value`` = params/s over K timed steps bracketed by
``torch.cuda.synchronize()``.

``roofline`` is the dominant kernel (the multi-tensor AdamW pass): 28
algorithmic bytes per parameter (read p, g, m, v; write p, m, v) times the
parameters of one launch, over its average duration measured here with HIP
events on the launch stream.  ``traffic`` is read from the committed
rocprofv3 PMC summary when present.  ``cpu_baseline`` times the NumPy oracle
(the reference's NumPy path restated op for op) on a bounded sample of the
same workload on this host, one core.

The other configurations (C1 flat 4M fp32 hot and MALL-flushed, C3 AMP
GPT-2, C4 GPT-1.3B bf16 + clip, C5 Llama-7B AMP + clip) are reported under
``extra`` with their own B/param accounting; C3, C4 and C5 each through
``fused_step`` (``fused``) and the reference call sequence (``api``:
unscale_, clip when finite, step, update), C3 also through ``step`` alone (``step``: scale,
step, update, the reference API without unscale_), together with one GPU's share
of an 8-way sharded C4 and C5 step (``c4s8``, ``c5s8``: every tensor split
into 8 contiguous slices, the local work between the collectives).
``chunks`` (optional) times the pass with 4096- and 2048-element tasks,
alternately on the same buffers, for the C2-C5 layouts.
``ceilings`` adds the bandwidth of each read/write stream mix under the
pass's access pattern (``nt_stream_probe``), the C4/C5 pass mixes included;
``roofline.frac_of_mix_ceiling`` is the pass against the probe with its own
mix, in place (16 B read, 12 B written back where they were read).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "AdamW step params/sec + achieved HBM GB/s (% of peak), GPT-2 124M & 1.3B"
HBM_PEAK_GBPS = 8000.0
PROFILE_PMC = ROOT / "profiles" / "adamw_mt_f32_gpt2-124m.md"


def log(message: str) -> None:
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def parse_args():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--configs", default="c2,c1,c3,c4,c5,c4s8,c5s8,ceilings")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--kernel-only", action="store_true", help="only the C2 kernel loop (for profilers)")
    parser.add_argument("--calibrate", action="store_true",
                        help="with --kernel-only or --profile: also run 3 plain 1 GiB device copies (known bytes, "
                             "for PMC scaling)")
    parser.add_argument("--profile", default=None, choices=sorted(MIXED),
                        help="only this config's step (for profilers): --warmup untimed, --steps timed")
    parser.add_argument("--profile-modes", default="fused",
                        help="with --profile: the step paths to run in turn, 'fused', 'api' (the reference "
                             "call sequence) and/or 'step' (scale, step, update; c3 only), comma-separated")
    return parser.parse_args()


# ---- workload construction ---------------------------------------------------------------------
def make_params(nt, torch, shapes, dtype, seed=1337, sigma=0.02):
    generator = torch.Generator(device="cuda").manual_seed(seed)
    params = []
    for shape in shapes:
        data = torch.randn(shape, generator=generator, device="cuda", dtype=torch.float32).mul_(sigma)
        storage = data.to(dtype.torch_dtype) if dtype is not nt.float32 else data
        param = nt.Parameter.__new__(nt.Parameter)
        nt.Tensor._initialize(param, storage.contiguous(), True)
        params.append(param)
    return params


def attach_grads(nt, torch, params, dtype, sigma=1e-3, scale=1.0, seed=2337):
    generator = torch.Generator(device="cuda").manual_seed(seed)
    for param in params:
        data = torch.randn(param.shape, generator=generator, device="cuda", dtype=torch.float32).mul_(sigma * scale)
        param.grad = nt.Tensor._from_storage(data.to(dtype.torch_dtype).contiguous())


def decay_groups(params, mask=None):
    """Weight decay 0.1 on matrices, 0 on vectors (runner.py:83-90); `mask`
    overrides the ndim rule (shards are flat slices of the original tensors)."""
    mask = [p.ndim >= 2 for p in params] if mask is None else mask
    return [{"params": [p for p, m in zip(params, mask) if m], "weight_decay": 0.1},
            {"params": [p for p, m in zip(params, mask) if not m], "weight_decay": 0.0}]


def release(nt, torch):
    """Return cached device memory of both allocators (PyTorch's, which holds
    the synthetic inputs, and the library's, which holds optimizer state)."""
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    nt.runtime.empty_cache(0)


def calibration_copies(torch) -> dict:
    """Three plain 1 GiB device-to-device copies (known traffic: 1 GiB read
    and 1 GiB written each), which scale the PMC byte counters."""
    source = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    target = torch.empty_like(source)
    for _ in range(3):
        target.copy_(source)
    torch.cuda.synchronize()
    record = {"read": source.numel() * 4, "write": target.numel() * 4, "launches": 3}
    del source, target
    torch.cuda.empty_cache()
    return record


def event_pair(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def median_interval(marks) -> float:
    """Median of the intervals between consecutive recorded events (ms): the
    per-step times on the device timeline, launch gaps included."""
    intervals = sorted(a.elapsed_time(b) for a, b in zip(marks, marks[1:]))
    middle = len(intervals) // 2
    return intervals[middle] if len(intervals) % 2 else 0.5 * (intervals[middle - 1] + intervals[middle])


def timed_steps(torch, one_step, steps: int) -> tuple:
    """(mean ms per step, median ms per step) of `one_step`.

    The mean times exactly `steps` steps between two device synchronisations
    with nothing else queued between the steps.  The median comes from a
    second run of `steps` steps with a timing event recorded between
    consecutive steps; each such event is a marker on the launch stream that
    costs the device about 6 us, so that run's intervals carry it and it is
    kept out of the mean."""
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        one_step()
    torch.cuda.synchronize()
    mean_ms = (time.perf_counter() - start) * 1e3 / steps
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    for k in range(steps):
        marks[k].record()
        one_step()
    marks[steps].record()
    torch.cuda.synchronize()
    return mean_ms, median_interval(marks)


# ---- C2: the headline ----------------------------------------------------------------------------
def bench_c2(nt, torch, steps, warmup):
    from namitorch_amd.param_lists import gpt2_shapes, total_params
    shapes = gpt2_shapes()
    n = total_params(shapes)
    params = make_params(nt, torch, shapes, nt.float32)
    attach_grads(nt, torch, params, nt.float32)
    optimizer = nt.optim.AdamW(decay_groups(params), lr=3e-4, betas=(0.9, 0.999), eps=1e-8)
    for _ in range(warmup):
        optimizer.step()
    ms_per_step, median_ms = timed_steps(torch, optimizer.step, steps)
    # Dominant kernel: re-launch the cached plan back to back between HIP events
    # on the launch stream (torch's current stream, where the library launches).
    kernel_ms = kernel_time_c2(nt, torch, optimizer, params, steps)
    result = dict(params=n, tensors=len(shapes), ms_per_step=ms_per_step, params_per_s=n / (ms_per_step / 1e3),
                  median_ms_per_step=median_ms, kernel_ms=kernel_ms, bytes_per_param=28)
    del optimizer, params
    release(nt, torch)
    return result


def kernel_time_c2(nt, torch, optimizer, params, launches):
    """Average duration (ms) of the optimizer's float32 AdamW pass relaunched
    back to back through its cached plan, between two events on the launch
    stream."""
    from namitorch_amd import _native
    backend = nt.get_backend("cuda:0")
    numel = sum(p.numel() for p in params)
    plan = next(p for p in backend._plans.values() if p.numel == numel and p.layout[0] == _native.NT_F32)
    group = optimizer.param_groups
    records = []
    for g in group:
        options = optimizer._prepare_options({k: v for k, v in g.items() if k != "params"}, "g")
        step = optimizer.state[id(g["params"][0])]["step"] + 1
        records.append(optimizer._coefficients(nt.float32, options, step, True))
    slots = (_native.AdamWCoefs * len(records))(*records)
    start, stop = event_pair(torch)
    backend.adamw_multi(plan, slots, None)
    torch.cuda.synchronize()
    start.record()
    for _ in range(launches):
        backend.adamw_multi(plan, slots, None)
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / launches


# ---- C1: flat 4,194,304 fp32 ------------------------------------------------------------------------
def bench_c1(nt, torch, steps, warmup):
    n = 4_194_304
    (param,) = make_params(nt, torch, [(n,)], nt.float32)
    attach_grads(nt, torch, [param], nt.float32)
    optimizer = nt.optim.AdamW([param], lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
    for _ in range(warmup):
        optimizer.step()
    torch.cuda.synchronize()
    start, stop = event_pair(torch)
    start.record()
    for _ in range(steps):
        optimizer.step()
    stop.record()
    stop.synchronize()
    hot_ms = start.elapsed_time(stop) / steps
    # The pass alone, relaunched back to back (the step loop above can wait
    # for the host at this size).
    hot_kernel_ms = kernel_time_c2(nt, torch, optimizer, [param], steps)
    # MALL flush: stream 1 GiB through HBM before every step.  The step's cost
    # is the difference between `steps` x (fill + step) and `steps` x fill,
    # each timed between two events only: a timing event between every fill
    # and step would add its own device time (about 6 us) to each step.
    scratch = torch.empty(1 << 28, dtype=torch.float32, device="cuda")

    def loop(with_step: bool) -> float:
        a, b = event_pair(torch)
        torch.cuda.synchronize()
        a.record()
        for _ in range(steps):
            scratch.fill_(1.0)
            if with_step:
                optimizer.step()
        b.record()
        b.synchronize()
        return a.elapsed_time(b) / steps

    loop(True)
    differences = []
    for _ in range(5):
        differences.append(loop(True) - loop(False))
    flushed_ms = statistics.median(differences)
    del scratch, optimizer, param
    release(nt, torch)
    return dict(params=n, bytes_per_param=28, hot_ms=hot_ms, hot_kernel_ms=hot_kernel_ms, flushed_ms=flushed_ms,
                flushed_rounds_ms=differences, hot_GBps=28 * n / hot_ms / 1e6,
                hot_kernel_GBps=28 * n / hot_kernel_ms / 1e6, flushed_GBps=28 * n / flushed_ms / 1e6,
                flushed_method="median over 5 rounds of [steps x (1 GiB fill + step) - steps x 1 GiB fill], "
                               "two events per loop")


# ---- C3 / C4 / C5: mixed precision through the public API -------------------------------------------
def fresh_gradients(grads):
    """What a new backward writing into the existing gradient buffers leaves:
    no pending unscale/clip and a bumped version (Tensor.copy_ semantics).
    The stored (scaled) values stay the same every step."""
    for gradient in grads:
        gradient._pending = None
        gradient._incoming = None
        gradient._version_counter.value += 1


def evicted_step_ms(torch, one_step, steps: int, rounds: int = 5) -> dict:
    """ms per step when the MALL holds nothing of the step's data as it
    starts: the median over `rounds` of [steps x (1 GiB read + step) -
    steps x 1 GiB read].  The read (an ordinary-load reduction) leaves the
    MALL full of clean, unrelated lines, so the step keeps only what it makes
    resident itself (the pre-pass's gradient window), and nothing from the
    step before."""
    flush = torch.ones(1 << 28, device="cuda")
    sink = torch.empty((), device="cuda")

    def loop(with_step: bool) -> float:
        torch.cuda.synchronize()
        start = time.perf_counter()
        for _ in range(steps):
            torch.sum(flush, dim=0, out=sink)
            if with_step:
                one_step()
        torch.cuda.synchronize()
        return (time.perf_counter() - start) * 1e3 / steps

    differences = [loop(True) - loop(False) for _ in range(rounds)]
    del flush, sink
    return dict(ms_per_step=statistics.median(differences), rounds_ms=differences,
                method="median over rounds of [steps x (1 GiB ordinary read + step) - steps x 1 GiB read]")


def bench_mixed(nt, torch, name, shapes, *, param_dtype, grad_dtype, state_dtype, amp, max_norm, bytes_per_param,
                steps, warmup, modes=("fused", "api"), mask=None, evict=False):
    from namitorch_amd.param_lists import total_params
    n = total_params(shapes)
    params = make_params(nt, torch, shapes, param_dtype)
    attach_grads(nt, torch, params, grad_dtype, scale=65536.0 if amp else 1.0)
    grads = [p.grad for p in params]
    loss = nt.Tensor._from_storage(torch.ones((), device="cuda"))
    result = dict(params=n, tensors=len(shapes), bytes_per_param=bytes_per_param, steps=steps, warmup=warmup)
    for mode in modes:
        optimizer = nt.optim.AdamW(decay_groups(params, mask), lr=3e-4, betas=(0.9, 0.999), eps=1e-8,
                                   master_weights=True, state_dtype=state_dtype)
        scaler = nt.GradScaler(init_scale=65536.0) if amp else None

        def one_step():
            fresh_gradients(grads)
            if mode == "fused":
                if amp:
                    scaler.scale(loss)
                nt.amp.fused_step(optimizer, scaler, max_norm=max_norm)
            elif mode == "step":
                # the reference API without unscale_ (no clip): step unscales itself
                scaler.scale(loss)
                scaler.step(optimizer)
                scaler.update()
            elif amp:
                scaler.scale(loss)
                finite = scaler.unscale_(optimizer)
                if finite and max_norm is not None:
                    nt.optim.clip_grad_norm_(params, max_norm)
                scaler.step(optimizer)
                scaler.update()
            else:
                if max_norm is not None:
                    nt.optim.clip_grad_norm_(params, max_norm)
                optimizer.step()

        for _ in range(warmup):
            one_step()
        wall_ms, median_ms = timed_steps(torch, one_step, steps)
        result[mode] = dict(ms_per_step=wall_ms, median_ms_per_step=median_ms, params_per_s=n / (wall_ms / 1e3),
                            GBps=bytes_per_param * n / wall_ms / 1e6,
                            pct_hbm_peak=100 * bytes_per_param * n / wall_ms / 1e6 / HBM_PEAK_GBPS,
                            median_pct_hbm_peak=100 * bytes_per_param * n / median_ms / 1e6 / HBM_PEAK_GBPS,
                            scale=None if scaler is None else scaler.get_scale())
        log(f"{name} {mode}: {wall_ms:.3f} ms/step (median {median_ms:.3f})")
        if evict and mode == "fused":
            evicted = evicted_step_ms(torch, one_step, max(10, steps // 4))
            evicted["pct_hbm_peak"] = 100 * bytes_per_param * n / evicted["ms_per_step"] / 1e6 / HBM_PEAK_GBPS
            result[mode]["mall_evicted"] = evicted
            log(f"{name} {mode} after a MALL eviction: {evicted['ms_per_step']:.3f} ms/step")
        for p in params:
            p._grad = None
        del optimizer, scaler
        for p, g in zip(params, grads):
            p.grad = g
        release(nt, torch)
    del params, grads
    release(nt, torch)
    return result


# ---- gradient producer edges ------------------------------------------------------------------------------
def bench_edges(nt, torch, shapes, steps, warmup):
    """accumulate_grads (incoming bf16 into stored bf16: 6 B/param) and
    zero_grad(set_to_none=False) (2 B/param) over a parameter list, each one
    launch per step; HIP-event timed on the launch stream."""
    from namitorch_amd.param_lists import total_params
    n = total_params(shapes)
    params = make_params(nt, torch, shapes, nt.bfloat16)
    attach_grads(nt, torch, params, nt.bfloat16)
    incoming = [nt.Tensor._from_storage(torch.full(p.shape, 2.0 ** -12, dtype=torch.bfloat16, device="cuda"))
                for p in params]
    optimizer = nt.optim.AdamW(params, master_weights=True)
    result = dict(params=n, tensors=len(shapes))
    for name, bytes_per_param, action in (
            ("accumulate", 6, lambda: nt.accumulate_grads(params, incoming)),
            ("zero_grad", 2, lambda: optimizer.zero_grad(set_to_none=False))):
        for _ in range(warmup):
            action()
        start, stop = event_pair(torch)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            action()
        stop.record()
        stop.synchronize()
        ms = start.elapsed_time(stop) / steps
        result[name] = dict(ms=ms, bytes_per_param=bytes_per_param, GBps=bytes_per_param * n / ms / 1e6,
                            pct_hbm_peak=100 * bytes_per_param * n / ms / 1e6 / HBM_PEAK_GBPS)
        log(f"edges {name}: {ms:.3f} ms")
    del params, incoming, optimizer
    release(nt, torch)
    return result


def bench_accumulate(nt, torch, steps, warmup, rounds=3):
    """The C5 step (Llama-7B list, bf16 model + fp32 master, bf16 grads,
    AMP + clip at 1.0) after a second micro-batch's gradients, three ways,
    interleaved over `rounds` on the same buffers:
    - none: the step alone (30 B/param: pre-pass 2, pass 28);
    - separate: accumulate_grads launch (6 B/param), then the step (36 B/param);
    - deferred: accumulate_grads(defer=True), the pre-pass and the pass add
      the incoming gradient as they read (pre-pass 4 + pass 30 = 34 B/param).
    Each step starts from fresh gradient objects over the same buffers, as
    a new backward leaves them.  Per mode: the median step of each round."""
    from namitorch_amd.param_lists import llama7b_shapes, total_params
    shapes = llama7b_shapes()
    n = total_params(shapes)
    params = make_params(nt, torch, shapes, nt.bfloat16)
    attach_grads(nt, torch, params, nt.bfloat16, scale=65536.0)
    grads = [p.grad for p in params]
    generator = torch.Generator(device="cuda").manual_seed(4337)
    incoming = []
    for p in params:
        data = torch.randn(p.shape, generator=generator, device="cuda", dtype=torch.float32).mul_(1e-3 * 8192.0)
        incoming.append(nt.Tensor._from_storage(data.to(torch.bfloat16).contiguous()))
        del data
    loss = nt.Tensor._from_storage(torch.ones((), device="cuda"))
    optimizer = nt.optim.AdamW(decay_groups(params), lr=3e-4, betas=(0.9, 0.999), eps=1e-8, master_weights=True)
    scaler = nt.GradScaler(init_scale=65536.0)
    modes = {"none": 30, "separate": 36, "deferred": 34}

    def one_step(mode):
        fresh_gradients(grads)
        if mode != "none":
            nt.accumulate_grads(params, incoming, defer=mode == "deferred")
        scaler.scale(loss)
        nt.amp.fused_step(optimizer, scaler, max_norm=1.0)

    medians = {mode: [] for mode in modes}
    for _ in range(rounds):
        for mode in modes:
            for _ in range(warmup):
                one_step(mode)
            marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
            torch.cuda.synchronize()
            for k in range(steps):
                marks[k].record()
                one_step(mode)
            marks[steps].record()
            torch.cuda.synchronize()
            medians[mode].append(median_interval(marks))
    result = dict(params=n, tensors=len(shapes), rounds=rounds, steps_per_round=steps, scale=scaler.get_scale())
    for mode, bytes_per_param in modes.items():
        ms = statistics.median(medians[mode])
        result[mode] = dict(median_ms_per_step=ms, round_medians_ms=medians[mode], bytes_per_param=bytes_per_param,
                            GBps=bytes_per_param * n / ms / 1e6,
                            pct_hbm_peak=100 * bytes_per_param * n / ms / 1e6 / HBM_PEAK_GBPS)
        log(f"c5 accumulate {mode}: median {ms:.3f} ms/step ({medians[mode]})")
    result["deferred_vs_separate_speedup"] = result["separate"]["median_ms_per_step"] / result["deferred"]["median_ms_per_step"]
    for p in params:
        p._grad = None
    del params, grads, incoming, optimizer, scaler
    release(nt, torch)
    return result


# ---- streaming ceilings ---------------------------------------------------------------------------------
# (name, fp32 reads, 16-bit reads, fp32 writes, 16-bit writes, elements per stream, in-place map).  The
# in-place map names, per write stream, the read stream it rewrites (None: a separate buffer), as the
# passes rewrite parameter/master, exp_avg and exp_avg_sq where they read them.
C2_STREAM = 30376 * 4096          # the C2 parameter count rounded down to 4096
LARGE_STREAM = 1 << 28            # 1 GiB per fp32 stream: far beyond the 256 MB MALL, like the C4/C5 streams
PROBE_MIXES = (("r1w0", 1, 0, 0, 0, C2_STREAM, None), ("r4w0", 4, 0, 0, 0, C2_STREAM, None),
               ("r0w1", 0, 0, 1, 0, C2_STREAM, None), ("r0w3", 0, 0, 3, 0, C2_STREAM, None),
               ("r1w1", 1, 0, 1, 0, C2_STREAM, None), ("r2w2", 2, 0, 2, 0, C2_STREAM, None),
               ("r4w3", 4, 0, 3, 0, C2_STREAM, None), ("r5w4", 5, 0, 4, 0, C2_STREAM, None),
               ("r4w3_inplace", 4, 0, 3, 0, C2_STREAM, (0, 2, 3)),
               ("r4w3_inplace_large", 4, 0, 3, 0, LARGE_STREAM, (0, 2, 3)),
               ("c4_pass_mix_large", 1, 3, 1, 3, LARGE_STREAM, None),
               ("c4_pass_mix_inplace_large", 1, 3, 1, 3, LARGE_STREAM, (0, 2, 3, None)),
               ("c5_pass_mix_large", 3, 1, 3, 1, LARGE_STREAM, None),
               ("c5_pass_mix_inplace_large", 3, 1, 3, 1, LARGE_STREAM, (0, 1, 2, None)))


def bench_ceilings(nt, torch, steps, warmup):
    """The bandwidth each read/write stream mix reaches with the pass's
    access pattern (nt_stream_probe).  r4w3 is the fp32 AdamW pass's mix
    (16 B read, 12 B written per parameter), run at the C2 size for the
    headline's comparison; the *_large mixes run 1 GiB fp32 streams like the
    multi-GB streams of C4/C5: c4_pass_mix is the C4 pass's (fp32 master +
    bf16 grad/m/v read, fp32 master + bf16 m/v/copy written: 10 B each way)
    and c5_pass_mix the C3/C5 pass's (fp32 master/m/v + a 16-bit grad read,
    fp32 master/m/v + a bf16 copy written: 14 B each way); *_inplace
    variants rewrite the streams they read, as the passes do; r4w0 is a
    multi-stream read like the pre-pass.  HIP-event timed on the launch
    stream; every stream is a fresh allocation of this process, filled with
    random values (N(0, 0.02) fp32, N(0, 1e-3) bf16)."""
    import ctypes
    from namitorch_amd import _native
    handle = torch.cuda.current_stream().cuda_stream
    result = {"elements_per_stream": {"C2": C2_STREAM, "large": LARGE_STREAM}}
    for count in (C2_STREAM, LARGE_STREAM):
        mixes = [m for m in PROBE_MIXES if m[5] == count]
        # Random values of the passes' magnitudes, not constant bytes: the
        # bandwidth of these write-heavy mixes depends on the values moved.
        generator = torch.Generator(device="cuda").manual_seed(4242)
        wide = [torch.randn(count, generator=generator, device="cuda").mul_(0.02)
                for _ in range(max(m[1] + m[3] for m in mixes))]
        narrow = [torch.randn(count, generator=generator, device="cuda").mul_(1e-3).to(torch.bfloat16)
                  for _ in range(max(m[2] + m[4] for m in mixes))]
        for name, r32, r16, w32, w16, _, inplace in mixes:
            reads = wide[:r32] + narrow[:r16]
            writes = wide[r32:r32 + w32] + narrow[r16:r16 + w16] if w32 + w16 else wide[-1:]
            if inplace is not None:
                writes = [reads[source] if source is not None else fresh for source, fresh in zip(inplace, writes)]
            read_ptrs = (ctypes.c_void_p * 8)(*[t.data_ptr() for t in reads])
            write_ptrs = (ctypes.c_void_p * 8)(*[t.data_ptr() for t in writes])
            args = (read_ptrs, r32 + r16, r16, write_ptrs, w32 + w16, w16, count, handle)
            for _ in range(warmup):
                _native.call("nt_stream_probe", *args)
            start, stop = event_pair(torch)
            torch.cuda.synchronize()
            start.record()
            for _ in range(steps):
                _native.call("nt_stream_probe", *args)
            stop.record()
            stop.synchronize()
            ms = start.elapsed_time(stop) / steps
            gbps = (4 * (r32 + w32) + 2 * (r16 + w16)) * count / ms / 1e6
            result[name] = dict(ms=ms, GBps=gbps, pct_hbm_peak=100 * gbps / HBM_PEAK_GBPS,
                                bytes_per_element=dict(read=4 * r32 + 2 * r16, write=4 * w32 + 2 * w16))
            log(f"probe {name}: {gbps:.0f} GB/s")
        del wide, narrow
        release(nt, torch)
    return result


# ---- pass task size ---------------------------------------------------------------------------------------
def bench_chunks(nt, torch, launches=20, reps=4):
    """The AdamW pass with 4096- and 2048-element tasks, timed alternately in
    one process on the same buffers (so both see the same physical
    placement), for each configuration's layout; the optimizer picks the chunk per
    layout (optim/adam.py _pass_chunk).  Both run the same one-wave
    256-element workgroups; the task size sets the task map and the tails.  Random N(0, 0.02) params, N(0, 1e-3)
    grads, zero moments; C4/C5 launches carry their clip (and unscale)
    transforms, as in their steps."""
    import ctypes
    from namitorch_amd import _native
    from namitorch_amd.param_lists import gpt2_shapes, gpt_1p3b_shapes, llama7b_shapes
    f32, f16, bf16, none = _native.NT_F32, _native.NT_F16, _native.NT_BF16, _native.NT_DTYPE_NONE
    torch_dtype = {f32: torch.float32, f16: torch.float16, bf16: torch.bfloat16}
    size = {f32: 4, f16: 2, bf16: 2, none: 0}
    configs = (("c2", gpt2_shapes, (f32, f32, f32, none), None),
               ("c3", gpt2_shapes, (f32, f16, f32, bf16), dict(scale=65536.0, unscale=1, clip_coef=1.0, clip=0)),
               ("c4", gpt_1p3b_shapes, (f32, bf16, bf16, bf16), dict(scale=1.0, unscale=0, clip_coef=0.5, clip=1)),
               ("c5", llama7b_shapes, (f32, bf16, f32, bf16), dict(scale=65536.0, unscale=1, clip_coef=0.5, clip=1)))
    stream = torch.cuda.current_stream().cuda_stream
    coefs = (_native.AdamWCoefs * 1)(_native.AdamWCoefs(3e-4, 0.9, 0.999, 0.1, 0.001, 1e-8, 0.1, 1 - 3e-5, 0.1, 0.001,
                                                         0, 1, 0, 0))
    generator = torch.Generator(device="cuda").manual_seed(7)
    result = {}
    for name, shapes_fn, layout, xform in configs:
        pdt, gdt, sdt, cdt = layout
        rows, keep = [], []
        for shape in shapes_fn():
            n = math.prod(shape)
            p = (torch.randn(n, generator=generator, device="cuda") * 0.02).to(torch_dtype[pdt])
            g = (torch.randn(n, generator=generator, device="cuda") * 1e-3).to(torch_dtype[gdt])
            m = torch.zeros(n, dtype=torch_dtype[sdt], device="cuda")
            v = torch.zeros(n, dtype=torch_dtype[sdt], device="cuda")
            c = torch.empty(n, dtype=torch_dtype[cdt], device="cuda") if cdt != none else None
            keep += [p, g, m, v, c]
            rows.append(_native.MtTensor(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(),
                                         None if c is None else c.data_ptr(), n, 0, 0))
        table = (_native.MtTensor * len(rows))(*rows)
        params = sum(row.numel for row in rows)
        moved = params * (2 * size[pdt] + size[gdt] + 4 * size[sdt] + size[cdt])
        transform = None if xform is None else ctypes.byref(_native.GradXform(**xform))
        plans = {}
        for chunk in (4096, 2048):
            handle = ctypes.c_void_p()
            _native.call("nt_plan_create", 0, table, len(rows), ctypes.byref(_native.MtLayout(*layout)), chunk, stream,
                         ctypes.byref(handle))
            plans[chunk] = handle
        times = {chunk: [] for chunk in plans}
        for _ in range(reps):
            for chunk, handle in plans.items():
                for _ in range(2):
                    _native.call("nt_adamw_mt", handle, coefs, 1, transform, stream)
                start, stop = event_pair(torch)
                start.record()
                for _ in range(launches):
                    _native.call("nt_adamw_mt", handle, coefs, 1, transform, stream)
                stop.record()
                stop.synchronize()
                times[chunk].append(start.elapsed_time(stop) / launches)
        entry = {}
        for chunk, values in times.items():
            best = min(values)
            entry[str(chunk)] = dict(best_ms=best, median_ms=sorted(values)[len(values) // 2], GBps=moved / best / 1e6)
        entry["faster"] = min(plans, key=lambda chunk: min(times[chunk]))
        result[name] = entry
        log(f"chunks {name}: 4096 {min(times[4096]):.4f} ms, 2048 {min(times[2048]):.4f} ms")
        torch.cuda.synchronize()
        for handle in plans.values():
            _native.call("nt_plan_destroy", handle)
        del keep, rows, table
        release(nt, torch)
    return result


# ---- CPU baseline ---------------------------------------------------------------------------------------
def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), else what platform reports."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _timed_steps(step, min_seconds, max_steps):
    """One untimed step, then timed steps until `min_seconds` have passed
    (at least two, at most `max_steps`); (steps, seconds)."""
    step(1)
    steps = 0
    start = time.perf_counter()
    while True:
        step(steps + 2)
        steps += 1
        elapsed = time.perf_counter() - start
        if steps >= max_steps or (steps >= 2 and elapsed >= min_seconds):
            return steps, elapsed


def _host_tensors(shapes, seed, sigma, dtype="float32"):
    import numpy as np
    rng = np.random.Generator(np.random.PCG64(seed))
    return [(rng.standard_normal(int(np.prod(s)), dtype=np.float32) * np.float32(sigma)).astype(dtype) for s in shapes]


def _baseline_record(total, steps, elapsed, bytes_per_param, sample, *, extrapolated_to=None):
    value = total * steps / elapsed
    record = dict(value=value, unit="params/s", cores=1, kind="port", GBps=bytes_per_param * value / 1e9,
                  sample=f"{sample}; {steps} timed steps after 1 untimed step, {elapsed:.2f} s; host CPU {cpu_model()}, "
                         f"os.cpu_count()={os.cpu_count()}, 1 thread (NumPy ufuncs are single-threaded)")
    if extrapolated_to is not None:
        record["extrapolated"] = True
        record["sample"] += (f"; extrapolated linearly by parameter count to the full list ({extrapolated_to} params): "
                             f"{extrapolated_to / value:.1f} s per step")
    return record


def cpu_baseline(min_seconds=10.0, max_steps=40):
    """C2 (the headline): NumPy oracle AdamW — the reference's NumPy path
    (optim/adam.py:27-42) restated op for op, with its per-step
    ``exp_avg_sq`` check and ``Tensor.copy_`` staging
    (``oracle.adam.reference_step``) — over the whole GPT-2-124M list."""
    import numpy as np
    from namitorch_amd.param_lists import gpt2_shapes
    from oracle import adam as oadam
    shapes = gpt2_shapes()
    total = sum(int(np.prod(s)) for s in shapes)
    params = _host_tensors(shapes, 1337, 0.02)
    grads = _host_tensors(shapes, 2337, 1e-3)
    ms = [np.zeros_like(p) for p in params]
    vs = [np.zeros_like(p) for p in params]
    wds = [0.1 if len(s) >= 2 else 0.0 for s in shapes]

    def step(k):
        for p, g, m, v, wd in zip(params, grads, ms, vs, wds):
            oadam.reference_step(p, g, m, v, k, lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd)

    steps, elapsed = _timed_steps(step, min_seconds, max_steps)
    return _baseline_record(total, steps, elapsed, 28,
                            f"NumPy oracle AdamW over the full GPT-2-124M list ({len(shapes)} tensors, {total} params), "
                            f"with the reference's per-step exp_avg_sq check and Tensor.copy_ staging of every write "
                            f"(oracle.adam.reference_step)")


def cpu_baselines_other(min_seconds=3.0):
    """The other configs through the oracle on this host, one thread each:
    C1 whole; C3 (unscale_ -> finite -> master step -> bf16 copy -> scaler
    update, amp.py:169-234 over the fp32-master extension), C4 and C5 on a
    prefix of about 15 M parameters of their lists (the step is per-element
    work, so params/s carries over to the full list, stated as
    extrapolated)."""
    import numpy as np
    from namitorch_amd.param_lists import gpt2_shapes, gpt_1p3b_shapes, llama7b_shapes, total_params
    from oracle import adam as oadam
    from oracle import clip as oclip
    from oracle import lowp
    from oracle import scaler as oscaler
    options = dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8)
    out = {}

    # C1: one flat 4,194,304-element fp32 tensor.
    p, = _host_tensors([(4_194_304,)], 1337, 0.02)
    g, = _host_tensors([(4_194_304,)], 2337, 1e-3)
    m, v = np.zeros_like(p), np.zeros_like(p)
    steps, elapsed = _timed_steps(lambda k: oadam.reference_step(p, g, m, v, k, weight_decay=0.1, **options),
                                  min_seconds, 200)
    out["c1"] = _baseline_record(p.size, steps, elapsed, 28, "NumPy oracle AdamW, one flat fp32 tensor of 4,194,304, "
                                 "with the reference's exp_avg_sq check and copy_ staging (oracle.adam.reference_step)")
    del p, g, m, v

    # C3 prefix: the first two GPT-2-124M layers, AMP: fp16 grads x 65536, fp32 master, bf16 model copy.
    full = gpt2_shapes()
    shapes = full[2:26]
    masters = [lowp.round_bf16(x) for x in _host_tensors(shapes, 1337, 0.02)]
    grads16 = [(x * np.float32(65536.0)).astype(np.float16) for x in _host_tensors(shapes, 2337, 1e-3)]
    ms = [np.zeros_like(x) for x in masters]
    vs = [np.zeros_like(x) for x in masters]
    wds = [0.1 if len(s) >= 2 else 0.0 for s in shapes]
    scaler = oscaler.Scaler()

    def c3_step(k):
        unscaled = [oscaler.unscale(x, scaler.scale, "float16") for x in grads16]
        finite = oscaler.finite(unscaled) and oscaler.finite(unscaled)     # unscale_ and step both check
        if finite:
            for master, u, m_, v_, wd in zip(masters, unscaled, ms, vs, wds):
                oadam.master_step(master, u, m_, v_, k, weight_decay=wd, **options)
                lowp.round_bf16(master)                                      # the bf16 model copy
        scaler.update(not finite)

    steps, elapsed = _timed_steps(c3_step, min_seconds, 40)
    out["c3"] = _baseline_record(total_params(shapes), steps, elapsed, 30,
                                 f"NumPy oracle AMP step over layers 0-1 of the GPT-2-124M list "
                                 f"({len(shapes)} tensors, {total_params(shapes)} params){OMITTED}",
                                 extrapolated_to=total_params(full))
    del masters, grads16, ms, vs

    # C4 prefix: the attention tensors of GPT-1.3B layer 0, bf16 grads/m/v, clip 1.0.
    full = gpt_1p3b_shapes()
    shapes = full[2:8]
    masters = [lowp.round_bf16(x) for x in _host_tensors(shapes, 1337, 0.02)]
    grads = [lowp.round_bf16(x) for x in _host_tensors(shapes, 2337, 1e-3)]
    ms = [np.zeros_like(x) for x in masters]
    vs = [np.zeros_like(x) for x in masters]
    wds = [0.1 if len(s) >= 2 else 0.0 for s in shapes]

    def c4_step(k):
        norm = oclip.total_norm(grads)
        coefficient = oclip.clip_coefficient(1.0, norm)
        clipped = [oclip.clip_apply(x, coefficient, "bfloat16") for x in grads] if coefficient < 1 else grads
        for master, x, m_, v_, wd in zip(masters, clipped, ms, vs, wds):
            oadam.master_step(master, x, m_, v_, k, weight_decay=wd, state_bf16=True, **options)
            lowp.round_bf16(master)

    steps, elapsed = _timed_steps(c4_step, min_seconds, 40)
    out["c4"] = _baseline_record(total_params(shapes), steps, elapsed, 22,
                                 f"NumPy oracle bf16 clip + master step over the attention tensors of GPT-1.3B "
                                 f"layer 0 ({len(shapes)} tensors, {total_params(shapes)} params){OMITTED}",
                                 extrapolated_to=total_params(full))
    del masters, grads, ms, vs

    # C5 prefix: the q projection of Llama-7B layer 0, AMP + clip.
    full = llama7b_shapes()
    shapes = full[2:3]
    masters = [x for x in _host_tensors(shapes, 1337, 0.02)]
    grads = [lowp.round_bf16(x * np.float32(65536.0)) for x in _host_tensors(shapes, 2337, 1e-3)]
    ms = [np.zeros_like(x) for x in masters]
    vs = [np.zeros_like(x) for x in masters]
    scaler = oscaler.Scaler()

    def c5_step(k):
        unscaled = [oscaler.unscale(x, scaler.scale, "bfloat16") for x in grads]
        finite = oscaler.finite(unscaled) and oscaler.finite(unscaled)
        if finite:
            norm = oclip.total_norm(unscaled)
            coefficient = oclip.clip_coefficient(1.0, norm)
            clipped = [oclip.clip_apply(x, coefficient, "bfloat16") for x in unscaled] if coefficient < 1 else unscaled
            for master, x, m_, v_ in zip(masters, clipped, ms, vs):
                oadam.master_step(master, x, m_, v_, k, weight_decay=0.1, **options)
                lowp.round_bf16(master)
        scaler.update(not finite)

    steps, elapsed = _timed_steps(c5_step, min_seconds, 40)
    out["c5"] = _baseline_record(total_params(shapes), steps, elapsed, 30,
                                 f"NumPy oracle AMP + clip + master step over the q projection of Llama-7B "
                                 f"layer 0 ({len(shapes)} tensor, {total_params(shapes)} params){OMITTED}",
                                 extrapolated_to=total_params(full))
    return out


# What the C3-C5 baselines (the fp32-master extension of the oracle) leave out
# of the reference's path.
OMITTED = ("; the oracle writes in place, without the reference's Tensor.copy_ staging (three copies per written "
           "array) or its per-step exp_avg_sq check, so this overstates the reference's CPU rate")


def pmc_traffic():
    """HBM bytes per launch of the C2 AdamW kernel from the committed rocprofv3
    PMC summary (FETCH_SIZE/WRITE_SIZE scaled by a 1 GiB copy), or None."""
    try:
        for line in PROFILE_PMC.read_text().splitlines():
            if line.startswith("hbm_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except (OSError, ValueError):
        return None
    return None


def _mixed_configs(nt):
    """(result key, bench_mixed keyword arguments) of the mixed-precision configs."""
    from namitorch_amd.param_lists import decay_mask, gpt2_shapes, gpt_1p3b_shapes, llama7b_shapes, shard_shapes
    return {
        "c3": ("c3_gpt2_amp", dict(shapes=gpt2_shapes(), param_dtype=nt.bfloat16, grad_dtype=nt.float16,
                                   state_dtype=None, amp=True, max_norm=None, bytes_per_param=30, evict=True,
                                   modes=("fused", "api", "step"))),
        "c4": ("c4_gpt1p3b_bf16_clip", dict(shapes=gpt_1p3b_shapes(), param_dtype=nt.bfloat16, grad_dtype=nt.bfloat16,
                                            state_dtype=nt.bfloat16, amp=False, max_norm=1.0, bytes_per_param=22)),
        "c5": ("c5_llama7b_amp_clip", dict(shapes=llama7b_shapes(), param_dtype=nt.bfloat16, grad_dtype=nt.bfloat16,
                                           state_dtype=None, amp=True, max_norm=1.0, bytes_per_param=30)),
        "c4s8": ("c4_shard8", dict(shapes=shard_shapes(gpt_1p3b_shapes(), 8), param_dtype=nt.bfloat16,
                                   grad_dtype=nt.bfloat16, state_dtype=nt.bfloat16, amp=False, max_norm=1.0,
                                   bytes_per_param=22, modes=("fused",), mask=decay_mask(gpt_1p3b_shapes()),
                                   evict=True)),
        "c5s8": ("c5_shard8", dict(shapes=shard_shapes(llama7b_shapes(), 8), param_dtype=nt.bfloat16,
                                   grad_dtype=nt.bfloat16, state_dtype=None, amp=True, max_norm=1.0,
                                   bytes_per_param=30, modes=("fused",), mask=decay_mask(llama7b_shapes()),
                                   evict=True)),
    }


MIXED = ("c3", "c4", "c5", "c4s8", "c5s8")


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "namitorch_amd benchmarks one GPU; the optimizer step has no multi-GPU path in this build "
                                   "(one GPU's share of a sharded step is what it measures).", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    import namitorch_amd as nt
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a HIP device")
    # The synthetic inputs and the timing events live on PyTorch's current
    # stream: make the library launch there too.
    nt.runtime.set_stream_provider(lambda device: torch.cuda.current_stream(device).cuda_stream)
    log(f"device {torch.cuda.get_device_name(0)}")
    wanted = [c.strip() for c in args.configs.split(",") if c.strip()]
    extra = {}
    if args.profile:
        key, spec = _mixed_configs(nt)[args.profile]
        modes = tuple(args.profile_modes.split(","))
        if not modes or any(mode not in ("fused", "api", "step") for mode in modes):
            raise SystemExit("--profile-modes takes 'fused', 'api' and/or 'step', comma-separated")
        if "step" in modes and (not spec["amp"] or spec["max_norm"] is not None):
            raise SystemExit("'step' mode (scale, step, update) is for the AMP config without a clip (c3)")
        spec = dict(spec, modes=modes, evict=False)
        shapes = spec.pop("shapes")
        log(f"{args.profile} {' then '.join(modes)} steps only ({args.warmup} untimed, {args.steps} timed each)")
        if args.calibrate:
            log(f"calibration copies: {calibration_copies(torch)}")
        print(json.dumps({key: bench_mixed(nt, torch, args.profile, shapes, steps=args.steps, warmup=args.warmup,
                                           **spec)}), flush=True)
        return
    log("C2 gpt2-124m fp32 multi-tensor AdamW")
    c2 = bench_c2(nt, torch, args.steps, args.warmup)
    log(f"C2: {c2['ms_per_step']:.3f} ms/step, kernel {c2['kernel_ms']:.3f} ms")
    if args.kernel_only:
        if args.calibrate:
            c2["calibration_copy_bytes"] = calibration_copies(torch)
        print(json.dumps(c2))
        return
    from namitorch_amd.param_lists import gpt_1p3b_shapes
    if "c1" in wanted:
        log("C1 flat 4M fp32")
        extra["c1_flat4m_fp32"] = c1 = bench_c1(nt, torch, args.steps, args.warmup)
        log(f"C1: flushed {c1['flushed_ms'] * 1e3:.1f} us/step, hot {c1['hot_ms'] * 1e3:.1f} us/step, "
            f"hot pass {c1['hot_kernel_ms'] * 1e3:.1f} us")
    # C3 GPT-2 AMP (bf16 model, fp32 master, fp16 grads x65536); C4 GPT-1.3B
    # bf16 params/m/v/grads, fp32 master, clip 1.0; C5 Llama-7B fp32
    # master/m/v, bf16 grads/params, AMP + clip; and one GPU's share of an
    # 8-way sharded C4 and C5 step (every tensor split into 8 contiguous
    # slices, ZeRO-1 style: the local pre-pass + AdamW pass each rank runs
    # between the collectives).
    # The sub-millisecond configs are timed over 4x the steps: the first step
    # after the synchronisation that opens a timed run waits for the host
    # (about 0.4 ms), which 50 steps would spread as ~8 us over each.  Their
    # warm-up runs at least 30 steps, past the first steps' one-time host work.
    counts = {"c3": 4 * args.steps, "c4": args.steps, "c5": max(10, args.steps // 2), "c4s8": 4 * args.steps,
              "c5s8": args.steps}
    warmups = {"c3": max(args.warmup, 30), "c4": max(args.warmup, 10), "c5": min(args.warmup, 3),
               "c4s8": max(args.warmup, 30), "c5s8": max(args.warmup, 10)}
    for name, (key, spec) in _mixed_configs(nt).items():
        if name not in wanted:
            continue
        spec = dict(spec)
        shapes = spec.pop("shapes")
        log(f"{name}: {key}")
        extra[key] = bench_mixed(nt, torch, name, shapes, steps=counts[name], warmup=warmups[name], **spec)
    if "chunks" in wanted:
        log("AdamW pass task size: 4096 against 2048 elements, same buffers")
        extra["pass_chunks"] = bench_chunks(nt, torch)
    if "accum" in wanted:
        log("c5 after a second micro-batch: separate accumulate launch against the deferred addend")
        extra["c5_accumulate"] = bench_accumulate(nt, torch, max(5, args.steps // 4), min(args.warmup, 2))
    if "edges" in wanted:
        log("gradient edges: accumulate and zero over the gpt-1.3b list (bf16)")
        extra["grad_edges_gpt1p3b"] = bench_edges(nt, torch, gpt_1p3b_shapes(), max(5, args.steps // 2), args.warmup)
    ceilings = None
    if "ceilings" in wanted:
        log("streaming ceilings of the read/write mixes (nt_stream_probe)")
        ceilings = bench_ceilings(nt, torch, max(10, args.steps // 2), args.warmup)
        extra["stream_ceilings"] = ceilings
    baseline = None
    if not args.no_cpu:
        log("CPU baseline (NumPy oracle)")
        baseline = cpu_baseline()
        log(f"CPU C2: {baseline['value']:.3g} params/s")
        extra["cpu_baselines"] = cpu_baselines_other()
        for name, record in extra["cpu_baselines"].items():
            log(f"CPU {name}: {record['value']:.3g} params/s")
    achieved = 28 * c2["params"] / (c2["kernel_ms"] / 1e3) / 1e9
    line = {
        "metric": METRIC,
        "value": c2["params_per_s"],
        "unit": "params/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": c2["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) params, N(0,1e-3) grads, resident in HBM)",
        "config": {"workload": "C2: GPT-2-124M parameter list, multi-tensor fp32 AdamW (148 tensors, 124,439,808 params, "
                               "2 weight-decay groups), one optimizer.step() per step",
                   "params": c2["params"], "tensors": c2["tensors"], "bytes_per_param": 28,
                   "step_GBps": 28 * c2["params_per_s"] / 1e9,
                   "step_pct_hbm_peak": 100 * 28 * c2["params_per_s"] / 1e9 / HBM_PEAK_GBPS},
        "median_ms_per_step": c2["median_ms_per_step"],
        "median_method": "median interval of a second run of the same steps with a timing event between "
                         "consecutive steps (each event adds about 6 us of device time); ms_per_step has none",
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": pmc_traffic(),
                     "traffic_source": f"FETCH_SIZE/WRITE_SIZE of the same kernel from the committed rocprofv3 PMC "
                                       f"summary {PROFILE_PMC.relative_to(ROOT)} (calibrated by a 1 GiB copy), "
                                       f"not counted in this run",
                     "kernel": "nt::adamw_mt_kernel<TF32,TF32,TF32,TNone,RoundF32,false,64,1>",
                     "kernel_ms": c2["kernel_ms"],
                     "mix_ceiling_GBps": ceilings["r4w3_inplace"]["GBps"] if ceilings else None,
                     "frac_of_mix_ceiling": achieved / ceilings["r4w3_inplace"]["GBps"] if ceilings else None},
        "cpu_baseline": baseline,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
