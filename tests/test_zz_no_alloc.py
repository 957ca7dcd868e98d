"""tarmac_dense_bwd_noalloc: the dense backward with its [B, 2, N] statistics
in the library's own device array instead of a caller workspace.

Called through the C ABI and compared with tarmac_dense_bwd (stats computed
in the call, caller workspace) on the same inputs: both run the same two
kernels, which have no atomics, so dq, dk and dv must agree bit for bit. Two
calls in a row, the second on a smaller input, so the second runs over what
the first left in the shared array; a call beyond the array's size is refused
before anything is launched; and a process's first call (the one that looks
up the array's address) made under graph capture, replayed three times.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(B, N, d, seed):
    g = np.random.default_rng(seed)
    return [torch.from_numpy(g.standard_normal((B, N, d)).astype(np.float32)).cuda()
            for _ in range(4)]


def _with_workspace(q, k, v, out, dout):
    from tarmac import _launch, _lib
    B, N, d = q.shape
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    stats = torch.empty(B, 2, N, device=q.device, dtype=torch.float32)
    P = _launch.ptr
    rc = _lib.LIB.tarmac_dense_bwd(P(q), P(k), P(v), P(out), P(dout), P(dq), P(dk), P(dv),
                                   P(stats), 0, B, N, d, _launch.stream(q))
    _lib.check(rc)
    return dq, dk, dv


def _no_alloc(q, k, v, out, dout):
    from tarmac import _launch, _lib
    B, N, d = q.shape
    dq, dk, dv = (torch.full_like(q, float("nan")) for _ in range(3))
    P = _launch.ptr
    rc = _lib.LIB.tarmac_dense_bwd_noalloc(P(q), P(k), P(v), P(out), P(dout), P(dq), P(dk),
                                           P(dv), B, N, d, _launch.stream(q))
    _lib.check(rc)
    return dq, dk, dv


@pytest.mark.parametrize("shapes", [((64, 256, 16), (8, 96, 16)), ((16, 200, 32), (3, 37, 8))])
def test_no_alloc_matches_workspace_entry(shapes):
    from tarmac.kernels import fused_dense_attention
    for i, (B, N, d) in enumerate(shapes):
        print(f"tarmac_dense_bwd_noalloc call {i}: B={B} N={N} d={d}", flush=True)
        q, k, v, dout = _inputs(B, N, d, seed=100 + i)
        out = fused_dense_attention(q, k, v)
        want = _with_workspace(q, k, v, out, dout)
        got = _no_alloc(q, k, v, out, dout)
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv"), got, want):
            assert torch.isfinite(a).all(), name
            assert torch.equal(a, b), f"{name} differs on call {i} (B={B}, N={N}, d={d})"


def test_no_alloc_at_the_scratch_limit_and_beyond():
    from tarmac import _launch, _lib
    from tarmac.kernels import fused_dense_attention
    # B * N = 2^20 statistics pairs is exactly the 8 MiB array
    B, N, d = 4096, 256, 8
    q, k, v, dout = _inputs(B, N, d, seed=7)
    out = fused_dense_attention(q, k, v)
    want = _with_workspace(q, k, v, out, dout)
    got = _no_alloc(q, k, v, out, dout)
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv"), got, want):
        assert torch.equal(a, b), name
    # one row more is refused on the host, before any launch
    P = _launch.ptr
    rc = _lib.LIB.tarmac_dense_bwd_noalloc(P(q), P(k), P(v), P(out), P(dout), P(q), P(k), P(v),
                                           B, N + 1, d, _launch.stream(q))
    assert rc == _lib.TARMAC_ERR_UNSUPPORTED
    assert "scratch" in _lib.last_error()


_CAPTURE_SCRIPT = r"""
import numpy as np
import torch
from tarmac import _launch, _lib
from tarmac.kernels import fused_dense_attention

B, N, d = 32, 256, 16
g = np.random.default_rng(11)
q, k, v, dout = (torch.from_numpy(g.standard_normal((B, N, d)).astype(np.float32)).cuda()
                 for _ in range(4))
out = fused_dense_attention(q, k, v)
P = _launch.ptr
want = [torch.empty_like(q) for _ in range(3)]
stats = torch.empty(B, 2, N, device="cuda")
_lib.check(_lib.LIB.tarmac_dense_bwd(P(q), P(k), P(v), P(out), P(dout), *map(P, want), P(stats),
                                     0, B, N, d, _launch.stream(q)))
got = [torch.full_like(q, float("nan")) for _ in range(3)]
torch.cuda.synchronize()
print("capturing the first tarmac_dense_bwd_noalloc call of this process", flush=True)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    rc = _lib.LIB.tarmac_dense_bwd_noalloc(P(q), P(k), P(v), P(out), P(dout), *map(P, got),
                                           B, N, d, _launch.stream(q))
_lib.check(rc)
for rep in range(3):
    for t in got:
        t.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv"), got, want):
        assert torch.equal(a, b), f"{name} differs on replay {rep}"
    print(f"replay {rep}: dq, dk, dv equal to tarmac_dense_bwd", flush=True)
print("CAPTURE_OK", flush=True)
"""


def test_no_alloc_first_call_under_graph_capture():
    """The entry point's first call in a process (where it looks up the
    array's device address) made inside torch.cuda.graph capture (global
    capture mode, which refuses allocations); three replays, each compared
    bit for bit with tarmac_dense_bwd. Runs in a child process so that the
    call is the process's first."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    env = dict(os.environ, PYTHONPATH=os.pathsep.join(
        [str(root / "topk-tarmac_amd"), os.environ.get("PYTHONPATH", "")]))
    res = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT], env=env, capture_output=True,
                         text=True, timeout=110)
    print(res.stdout[-2000:], res.stderr[-2000:])
    assert res.returncode == 0 and "CAPTURE_OK" in res.stdout
