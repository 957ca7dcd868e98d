"""The reference's CPU path, restated in torch (CPU) -- TEST INFRASTRUCTURE ONLY.

``bench.py``'s ``cpu_baseline`` leg times the reference's compositions of
the attention core with it on the host's own cores, beside the GPU numbers, as
the reference's CPU microbenchmark does (``scripts/microbenchmark_comm.py:117-125``
``_time_cpu``, ``:236-264`` ``host_report``; ``scripts/run_microbenchmarks.sh:49-52``
warm-up 10, reps 30, runs 5); ``tests/test_oracle.py`` checks it against the
pinned numpy oracle. Nothing in the product package imports it.

Each function computes what the reference's torch composition computes, in
this module's own code:

* ``topk_gather`` -- ``scripts/bench_attention_core.py:94-101`` /
  ``src/agents/mappo.py:192-231``: all N x N scores, self pair masked,
  unsorted ``topk``, softmax over the kept scores, kept value rows gathered
  and contracted;
* ``dense_unfused`` -- ``scripts/bench_attention_core.py:74-75``: softmax over
  all peers, then the product with V;
* ``zorder`` -- ``src/kernels/prescore_selection.py:51-84,184-195``: Morton
  codes of the per-row normalised positions (``bits`` per axis, x on even
  bits), ``argsort``, each agent's curve-window peers, attention over them.
"""

from __future__ import annotations

import math
import os
import platform
import statistics
import time

import torch


def topk_gather(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, topk: int) -> torch.Tensor:
    n_batch, n_agents, dim = q.shape
    keep = max(1, min(int(topk), n_agents - 1))
    logits = torch.bmm(q, k.transpose(1, 2)) / math.sqrt(dim)
    logits.diagonal(dim1=1, dim2=2).fill_(float("-inf"))
    kept, which = torch.topk(logits, keep, dim=2, sorted=False)
    weights = torch.softmax(kept, dim=2)
    base = torch.arange(n_batch).view(n_batch, 1, 1) * n_agents
    rows = v.reshape(n_batch * n_agents, dim)[which + base]
    return (weights.unsqueeze(3) * rows).sum(dim=2)


def dense_unfused(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    dim = q.shape[-1]
    logits = torch.bmm(q, k.transpose(1, 2)) / math.sqrt(dim)
    logits.diagonal(dim1=1, dim2=2).fill_(float("-inf"))
    return torch.bmm(torch.softmax(logits, dim=2), v)


def _spread(x: torch.Tensor) -> torch.Tensor:
    """Bits 0..15 of x moved to the even bit positions 0..30."""
    x = (x | (x << 8)) & 0x00FF00FF
    x = (x | (x << 4)) & 0x0F0F0F0F
    x = (x | (x << 2)) & 0x33333333
    return (x | (x << 1)) & 0x55555555


def morton_codes(pos: torch.Tensor, bits: int) -> torch.Tensor:
    lo = pos.amin(dim=1, keepdim=True)
    span = (pos.amax(dim=1, keepdim=True) - lo).clamp_min(1e-6)
    top = float((1 << bits) - 1)
    cells = ((pos - lo) / span * top).to(torch.int64).clamp(0, int(top))
    return _spread(cells[..., 0]) | (_spread(cells[..., 1]) << 1)


def zorder(q, k, v, pos, topk: int, bits: int) -> torch.Tensor:
    n_batch, n_agents, dim = q.shape
    order = torch.argsort(morton_codes(pos, bits), dim=1)
    rank = torch.empty_like(order)
    rank.scatter_(1, order, torch.arange(n_agents).expand(n_batch, n_agents).contiguous())
    steps = [s for s in range(1, (topk + 1) // 2 + 1)] + [-s for s in range(1, topk // 2 + 1)]
    offs = torch.tensor(steps[:topk])
    peers = torch.gather(order, 1, ((rank.unsqueeze(2) + offs) % n_agents).reshape(n_batch, -1))
    peers = peers.view(n_batch, n_agents, topk)
    base = torch.arange(n_batch).view(n_batch, 1, 1) * n_agents
    k_rows = k.reshape(-1, dim)[peers + base]
    v_rows = v.reshape(-1, dim)[peers + base]
    logits = (q.unsqueeze(2) * k_rows).sum(-1) / math.sqrt(dim)
    return (torch.softmax(logits, dim=2).unsqueeze(3) * v_rows).sum(dim=2)


def host_report() -> dict:
    """Host facts the measurement depends on (``microbenchmark_comm.py:236-264``)."""
    model = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "cpu_model": model,
        "logical_cpus_affinity": len(os.sched_getaffinity(0)),
        "os_cpu_count": os.cpu_count(),
        "torch_threads": torch.get_num_threads(),
        "torch_interop_threads": torch.get_num_interop_threads(),
        "env": {name: os.environ.get(name) for name in
                ("OMP_NUM_THREADS", "MKL_NUM_THREADS", "OPENBLAS_NUM_THREADS",
                 "KMP_AFFINITY", "OMP_PROC_BIND")},
        "torch": torch.__version__,
        "python": platform.python_version(),
    }


def time_protocol(fn, warmup: int = 10, reps: int = 30, runs: int = 5) -> dict:
    """perf_counter around one call; warm-up, then ``runs`` runs of ``reps``
    calls. Reports the minimum, each run's median and the spread between run
    medians, in microseconds."""
    with torch.inference_mode():
        for _ in range(warmup):
            fn()
        run_medians = []
        best = float("inf")
        for _ in range(runs):
            samples = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn()
                samples.append(time.perf_counter() - t0)
            best = min(best, min(samples))
            run_medians.append(statistics.median(samples))
    return {
        "min_us": best * 1e6,
        "run_medians_us": [m * 1e6 for m in run_medians],
        "inter_run_spread_pct": 100.0 * (max(run_medians) - min(run_medians)) / min(run_medians),
        "calls": warmup + reps * runs,
    }
