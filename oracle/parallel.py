"""Chunked, multi-threaded evaluation of the oracle (test infrastructure).

The oracle's element-wise functions (``adam.adam_step``, ``adam.master_step``,
``scaler.unscale``, ``clip.clip_apply``, ``lowp.round_bf16``) compute every
element from that element alone, so they give the same bits on any split of
their inputs.  Large parameter lists (the GPT-2 and GPT-1.3B layouts) are
therefore processed as 1 Mi-element slices on a thread pool; NumPy releases
the GIL inside its ufuncs.  Reductions keep the oracle's own order:
``total_norm`` evaluates each gradient's sum whole (one tensor per task) and
combines the sums in list order, exactly as ``clip.total_norm`` does.

``total_norm_streamed`` takes gradients one at a time from a callback and
splits each one's sum over the pool too: ``np.sum`` of a contiguous float64
vector adds, in order, the pairwise sums of its consecutive blocks of
``SUM_BLOCK`` (8192) elements (NumPy's reduction buffer), so ``exact_sum``
sums those blocks on the pool and adds the block sums in order, which gives
``np.sum``'s bits.

Pinned by tests/test_oracle.py: every function here equals the plain oracle
call bit for bit on random inputs whose sizes straddle the slice boundaries;
``exact_sum`` equals ``np.sum`` and ``total_norm_streamed`` equals
``clip.total_norm`` on sizes around the block and slice boundaries.
"""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import adam, clip, lowp, scaler

SLICE = 1 << 20


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


class Pool:
    """A thread pool that runs oracle functions over slices of flat arrays."""

    def __init__(self, threads: int | None = None):
        self.executor = ThreadPoolExecutor(threads or default_threads())

    def close(self) -> None:
        self.executor.shutdown(wait=True)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _slices(self, size: int):
        return [slice(start, min(start + SLICE, size)) for start in range(0, size, SLICE)] or [slice(0, 0)]

    def run(self, tasks) -> list:
        """Run callables, return their results in order (re-raising the first error)."""
        futures = [self.executor.submit(task) for task in tasks]
        return [future.result() for future in futures]

    def each_slice(self, function, *arrays) -> None:
        """``function(*views)`` on aligned slices of same-sized flat arrays."""
        size = arrays[0].size
        views = [array.reshape(-1) for array in arrays]
        self.run([lambda part=part: function(*(view[part] for view in views)) for part in self._slices(size)])

    def mapped(self, function, array: np.ndarray, dtype) -> np.ndarray:
        """``function(array)`` assembled from slices into a new array of `dtype`."""
        flat = array.reshape(-1)
        out = np.empty(flat.size, dtype=dtype)

        def one(part):
            out[part] = function(flat[part])

        self.run([lambda part=part: one(part) for part in self._slices(flat.size)])
        return out.reshape(array.shape)


def adam_step(pool: Pool, param, grad, exp_avg, exp_avg_sq, step: int, **options) -> None:
    pool.each_slice(lambda p, g, m, v: adam.adam_step(p, g, m, v, step, **options), param, grad, exp_avg, exp_avg_sq)


def master_step(pool: Pool, master, grad32, exp_avg, exp_avg_sq, step: int, **options) -> None:
    pool.each_slice(lambda p, g, m, v: adam.master_step(p, g, m, v, step, **options), master, grad32, exp_avg,
                    exp_avg_sq)


def unscale(pool: Pool, gradient: np.ndarray, scale: float, dtype: str) -> np.ndarray:
    result_dtype = np.float16 if dtype == "float16" else (np.float64 if dtype == "float64" else np.float32)
    return pool.mapped(lambda g: scaler.unscale(g, scale, dtype), gradient, result_dtype)


def clip_apply(pool: Pool, gradient: np.ndarray, coefficient: float, dtype: str) -> np.ndarray:
    result_dtype = np.float16 if dtype == "float16" else (np.float64 if dtype == "float64" else np.float32)
    return pool.mapped(lambda g: clip.clip_apply(g, coefficient, dtype), gradient, result_dtype)


def round_bf16(pool: Pool, values: np.ndarray) -> np.ndarray:
    return pool.mapped(lowp.round_bf16, values, np.float32)


def finite(pool: Pool, gradients) -> bool:
    return all(pool.run([lambda g=g: bool(np.all(np.isfinite(g))) for g in gradients]))


def total_norm(pool: Pool, gradients, norm_type: float = 2.0) -> float:
    """``clip.total_norm`` with each gradient's terms evaluated on the pool."""
    maxima = pool.run([lambda g=g: np.max(np.abs(g), initial=0) for g in gradients])
    scale = np.asarray(0.0, dtype=np.float64)
    for value in maxima:
        scale = np.maximum(scale, value)
    if not bool(np.isfinite(scale)) or bool(scale == 0) or np.isinf(norm_type):
        return float(scale)

    def terms(gradient):
        with np.errstate(over="ignore", divide="ignore", invalid="ignore", under="ignore"):
            scaled = np.abs(np.asarray(gradient, dtype=np.float64)) / scale
            return np.sum(np.power(scaled, norm_type), dtype=np.float64)

    sums = pool.run([lambda g=g: terms(g) for g in gradients])
    total = np.asarray(0.0, dtype=np.float64)
    with np.errstate(over="ignore", divide="ignore", invalid="ignore", under="ignore"):
        for value in sums:
            total = total + value
        result = scale * np.power(total, 1 / norm_type)
        if not bool(np.isfinite(result)):
            result = np.exp(np.log(scale) + np.log(total) / norm_type)
    return float(result)


SUM_BLOCK = 8192
_SUM_SLICE = SUM_BLOCK * 128          # elements per pool task of exact_sum (a whole number of blocks)


def exact_sum(pool: Pool, values: np.ndarray) -> np.float64:
    """``np.sum(values, dtype=np.float64)`` of a contiguous float64 vector,
    with its blocks summed on the pool."""
    flat = np.ascontiguousarray(values, dtype=np.float64).reshape(-1)
    size = flat.size
    whole = size // SUM_BLOCK * SUM_BLOCK

    def blocks(start: int, stop: int) -> np.ndarray:
        return flat[start:stop].reshape(-1, SUM_BLOCK).sum(axis=1, dtype=np.float64)

    parts = pool.run([lambda a=a: blocks(a, min(a + _SUM_SLICE, whole)) for a in range(0, whole, _SUM_SLICE)])
    if whole < size:
        parts.append(np.asarray([np.sum(flat[whole:], dtype=np.float64)]))
    total = np.float64(0.0)
    for part in parts:
        for value in part:
            total = total + value
    return total


def total_norm_streamed(pool: Pool, count: int, fetch, norm_type: float = 2.0) -> float:
    """``clip.total_norm`` over `count` gradients that ``fetch(i)`` returns
    one at a time (called twice per gradient: once for the maxima, once for
    the sums), so the whole set is never held.  Each gradient's maximum and
    sum run on the pool; the combination is ``total_norm``'s."""
    scale = np.asarray(0.0, dtype=np.float64)
    for index in range(count):
        gradient = np.ascontiguousarray(fetch(index)).reshape(-1)
        parts = pool.run([lambda part=part: np.max(np.abs(gradient[part]), initial=0)
                          for part in pool._slices(gradient.size)])
        value = np.max(np.abs(gradient[:0]), initial=0)
        for part_max in parts:
            value = np.maximum(value, part_max)
        scale = np.maximum(scale, value)
    if not bool(np.isfinite(scale)) or bool(scale == 0) or np.isinf(norm_type):
        return float(scale)
    total = np.asarray(0.0, dtype=np.float64)
    with np.errstate(over="ignore", divide="ignore", invalid="ignore", under="ignore"):
        for index in range(count):
            gradient = fetch(index)
            terms = pool.mapped(lambda g: np.power(np.abs(np.asarray(g, dtype=np.float64)) / scale, norm_type),
                                np.ascontiguousarray(gradient).reshape(-1), np.float64)
            total = total + exact_sum(pool, terms)
        result = scale * np.power(total, 1 / norm_type)
        if not bool(np.isfinite(result)):
            result = np.exp(np.log(scale) + np.log(total) / norm_type)
    return float(result)
