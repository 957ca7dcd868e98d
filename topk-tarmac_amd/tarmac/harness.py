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

from typing import Any, Callable

import numpy as np
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


def _elapsed_ms(fn: Callable[[], Any], start: torch.cuda.Event, end: torch.cuda.Event) -> float:
    """Device time of one call: the event pair sits on the stream current
    during the call, and the host waits for the second event before the next
    call starts (calls never overlap)."""
    stream = torch.cuda.current_stream()
    start.record(stream)
    fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end)


def time_interleaved(fns: dict[str, Callable[[], Any]], reps: int, warmup: int,
                     runs: int) -> dict[str, np.ndarray]:
    """Round-robin timing: in every repetition each callable runs once, in
    turn. Returns per callable an array [runs, reps] of milliseconds."""
    names = list(fns)
    samples = np.zeros((len(names), runs, reps))
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.no_grad():
        for _ in range(warmup):
            for name in names:
                fns[name]()
        torch.cuda.synchronize()
        for run in range(runs):
            for rep in range(reps):
                for i, name in enumerate(names):
                    samples[i, run, rep] = _elapsed_ms(fns[name], start, end)
    return {name: samples[i] for i, name in enumerate(names)}


def as_graphs(fns: dict[str, Callable[[], Any]]) -> dict[str, Callable[[], Any]]:
    """Capture each callable into a graph of its own and return the replays.
    A few eager calls first keep any one-time setup out of the capture; the
    wrappers read the current stream, which during capture is the capture
    stream."""
    graphs: dict[str, torch.cuda.CUDAGraph] = {}
    with torch.no_grad():
        for name, fn in fns.items():
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                fn()
            graphs[name] = graph
    torch.cuda.synchronize()
    return {name: graph.replay for name, graph in graphs.items()}


def stats(samples) -> dict[str, Any]:
    """Summary of an array [runs, reps] of milliseconds: the minimum (the
    primary statistic), the overall median, each run's median and the spread
    between run medians."""
    arr = np.asarray(samples, dtype=float)
    per_run = np.median(arr, axis=1)
    return {
        "min_us": 1e3 * float(arr.min()),
        "median_us": 1e3 * float(np.median(arr)),
        "run_medians_us": [1e3 * float(m) for m in per_run],
        "inter_run_spread_pct": 100.0 * float((per_run.max() - per_run.min()) / per_run.min()),
        "n": int(arr.size),
    }


def paired_ratio(num, den) -> float:
    """Median of the per-repetition ratios num / den (the two ran in the same
    rounds, so each pair saw the same machine state)."""
    return float(np.median(np.asarray(num, dtype=float) / np.asarray(den, dtype=float)))
