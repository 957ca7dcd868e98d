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


# hipGraphNodeType values (hip_runtime_api.h)
_NODE_TYPES = {0: "kernel", 1: "memcpy", 2: "memset", 3: "host", 4: "graph", 5: "empty",
               6: "wait_event", 7: "event_record"}


def _hip_runtime():
    """The HIP runtime this process already runs on (loaded by torch; the
    soname resolves to that same instance)."""
    import ctypes
    lib = ctypes.CDLL("libamdhip64.so.7")
    lib.hipGraphGetNodes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t)]
    lib.hipGraphNodeGetType.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]
    return lib


def graph_node_counts(fn: Callable[[], Any]) -> dict[str, int]:
    """Capture one call of ``fn`` and count the captured graph's nodes by
    type: the number of kernel launches (and copies, fills) the call makes."""
    import ctypes
    with torch.no_grad():
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(graph):
            fn()
    handle = ctypes.c_void_p(graph.raw_cuda_graph())
    hip = _hip_runtime()
    count = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(handle, None, ctypes.byref(count)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    nodes = (ctypes.c_void_p * max(1, count.value))()
    if hip.hipGraphGetNodes(handle, nodes, ctypes.byref(count)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    out: dict[str, int] = {}
    for i in range(count.value):
        kind = ctypes.c_int(-1)
        if hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(kind)) != 0:
            raise RuntimeError("hipGraphNodeGetType failed")
        name = _NODE_TYPES.get(kind.value, f"type{kind.value}")
        out[name] = out.get(name, 0) + 1
    del graph
    return out


def _pair_us(fn: Callable[[], Any], reps: int) -> float:
    """Minimum over ``reps`` of one event pair around one call of ``fn``."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    return 1e3 * min(_elapsed_ms(fn, start, end) for _ in range(reps))


def launch_overheads(noop: Callable[[], Any], kernel: Callable[[], Any],
                     noop_capturable: Callable[[], Any], kernel_capturable: Callable[[], Any],
                     reps: int = 50, batch: int = 100) -> dict[str, float]:
    """Where the fixed cost of one timed call goes, in microseconds (minima).

    * ``event_pair_empty``: two events recorded back to back, nothing between;
    * ``noop_single``: one 1-wave kernel between the events;
    * ``noop_back_to_back``: per-launch time of ``batch`` noops under one pair
      (the launch-to-launch gap of a stream kept busy);
    * ``noop_graph_single``: one replay of a graph holding one noop;
      ``noop_graph_back_to_back``: per replay, ``batch`` replays under one
      pair; ``noop_graph_batched``: per node, one replay of a graph holding
      ``batch`` noops;
    * ``kernel_*``: the same for ``kernel``.

    ``noop`` and ``kernel`` may be pre-bound to a stream; the ``_capturable``
    forms must launch on the current stream (they are captured)."""
    def back_to_back(fn):
        def many():
            for _ in range(batch):
                fn()
        return _pair_us(many, max(5, reps // 10)) / batch

    def graph_of(fn, count):
        with torch.no_grad():
            for _ in range(2):
                fn()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(count):
                    fn()
        torch.cuda.synchronize()
        return g

    res = {}
    with torch.no_grad():
        for _ in range(10):
            noop()
            kernel()
        torch.cuda.synchronize()
        res["event_pair_empty"] = _pair_us(lambda: None, reps)
        for name, eager, capturable in (("noop", noop, noop_capturable),
                                        ("kernel", kernel, kernel_capturable)):
            res[f"{name}_single"] = _pair_us(eager, reps)
            res[f"{name}_back_to_back"] = back_to_back(eager)
            g1 = graph_of(capturable, 1)
            res[f"{name}_graph_single"] = _pair_us(g1.replay, reps)
            res[f"{name}_graph_back_to_back"] = back_to_back(g1.replay)
            gb = graph_of(capturable, batch)
            res[f"{name}_graph_batched"] = _pair_us(gb.replay, max(5, reps // 10)) / batch
            del g1, gb
    torch.cuda.synchronize()
    return {k: round(v, 3) for k, v in res.items()}


def device_probes(device, reps: int = 20) -> dict[str, float]:
    """What this device sustains on plain library work, beside the datasheet
    peaks: a 1 GiB device-to-device copy (read + write bytes per second) and
    square 8192^3 GEMMs (torch.mm on hipBLASLt) in fp32 and bf16."""
    res = {}
    src = torch.ones(256 << 20, device=device)          # 1 GiB of fp32
    dst = torch.empty_like(src)
    t = _pair_us(lambda: dst.copy_(src), reps) * 1e-6
    res["copy_1GiB_GBps"] = round(2 * src.numel() * 4 / t / 1e9, 1)
    del src, dst
    n = 8192
    for name, dt in (("gemm_fp32_TFLOPs", torch.float32), ("gemm_bf16_TFLOPs", torch.bfloat16)):
        a = torch.randn(n, n, device=device).to(dt)
        b = torch.randn(n, n, device=device).to(dt)
        c = torch.empty(n, n, device=device, dtype=dt)
        for _ in range(3):
            torch.mm(a, b, out=c)
        t = _pair_us(lambda: torch.mm(a, b, out=c), max(5, reps // 2)) * 1e-6
        res[name] = round(2 * n ** 3 / t / 1e12, 1)
        del a, b, c
    torch.cuda.synchronize()
    return res
