"""Timing protocol and analytic accounting for the attention core.

Follows the reference harness:

* interleaved timing -- every implementation is called once per repetition,
  in turn, each call bracketed by device events with a synchronisation after
  it, the minimum over samples as the primary statistic and the block of
  repetitions repeated so inter-run spread is visible
  (``scripts/bench_attention_core.py:255-327``, ``scripts/bench_fixed_set.py:105-132``);
* graph replay -- each call captured in its own graph and timed as a replay,
  which removes host launch latency (``scripts/bench_fixed_set.py:135-152``);
* ratios against the best dense implementation under ratio-of-minima and
  paired median (``scripts/bench_fixed_set.py:155-200``), and the
  selection-time share ``1 - t_fixed_set / t_topk``
  (``scripts/summarise_portability.py:83-88``);
* analytic work: FLOPs as ``scripts/bench_attention_core.py:196-201`` counts
  them (selection compares are 0 FLOPs), and compulsory bytes only -- q, k, v
  read and out written once, plus the index/position tensors a path reads or
  writes.
"""

from __future__ import annotations

import statistics
from typing import Any, Callable

import torch

#: MI355X datasheet peaks used for roofline fractions.
PEAK_HBM_BYTES_PER_S = 8.0e12
PEAK_FP32_FLOPS = 157.3e12
PEAK_BF16_FLOPS = 2.5e15


def analytic_flops(path: str, B: int, N: int, d: int, k: int = 0) -> int:
    """Multiply-accumulates x 2. dense: scores + aggregation over N; top-k:
    scores over N, aggregation over k; fixed set / Z-order: k scores and k rows."""
    if path == "dense":
        return 4 * B * N * N * d
    if path == "topk":
        return 2 * B * N * N * d + 2 * B * N * k * d
    if path in ("fixedset", "zorder"):
        return 4 * B * N * k * d
    raise ValueError(path)


def analytic_bytes(path: str, B: int, N: int, d: int, k: int = 0, itemsize: int = 4,
                   with_idx: bool = False) -> int:
    """Compulsory HBM bytes: q, k, v read once and out written once; top-k adds
    the int32 indices when they are written; the fixed set reads int32
    indices; Z-order reads fp32 positions (and writes indices if asked)."""
    base = 4 * B * N * d * itemsize
    if path == "dense":
        return base
    if path == "topk":
        return base + (4 * B * N * k if with_idx else 0)
    if path == "fixedset":
        return base + 4 * B * N * k
    if path == "zorder":
        return base + 8 * B * N + (4 * B * N * k if with_idx else 0)
    raise ValueError(path)


def event_time(fn: Callable[[], Any], stream: torch.cuda.Stream | None = None) -> float:
    """Milliseconds of one call, bracketed by events on the launch stream."""
    stream = stream or torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end)


def time_interleaved(fns: dict[str, Callable[[], Any]], reps: int, warmup: int,
                     runs: int) -> dict[str, list[list[float]]]:
    """Interleave every function repetition by repetition; raw samples (ms)
    per run."""
    names = list(fns)
    with torch.no_grad():
        for _ in range(warmup):
            for n in names:
                fns[n]()
        torch.cuda.synchronize()
        out: dict[str, list[list[float]]] = {n: [] for n in names}
        for _ in range(runs):
            block: dict[str, list[float]] = {n: [] for n in names}
            for _ in range(reps):
                for n in names:
                    block[n].append(event_time(fns[n]))
            for n in names:
                out[n].append(block[n])
    return out


def as_graphs(fns: dict[str, Callable[[], Any]]) -> dict[str, Callable[[], Any]]:
    """Capture each call in its own graph; return the replays."""
    out: dict[str, Callable[[], Any]] = {}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side), torch.no_grad():
        for f in fns.values():
            for _ in range(3):
                f()
    torch.cuda.current_stream().wait_stream(side)
    for n, f in fns.items():
        g = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(g):
            f()
        out[n] = g.replay
    torch.cuda.synchronize()
    return out


def stats(samples: list[list[float]]) -> dict[str, Any]:
    flat = sorted(x for run in samples for x in run)
    meds = [statistics.median(r) for r in samples]
    return {
        "min_us": 1e3 * flat[0],
        "median_us": 1e3 * statistics.median(flat),
        "run_medians_us": [1e3 * m for m in meds],
        "inter_run_spread_pct": 100.0 * (max(meds) - min(meds)) / min(meds),
        "n": len(flat),
    }


def paired_ratio(num: list[list[float]], den: list[list[float]]) -> float:
    """Median of per-repetition ratios (repetitions ran in the same round)."""
    a = [x for r in num for x in r]
    b = [x for r in den for x in r]
    return statistics.median(x / y for x, y in zip(a, b))
