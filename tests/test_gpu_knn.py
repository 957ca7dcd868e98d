"""kNN pre-score selectors on the GPU against the oracle.

Bar: bit-exact. The radius selector emits the k nearest by (squared fp32
distance, agent index) in ascending agent index; the grid selector emits the
k smallest (distance, slot) in ascending slot. Both are compared entry for
entry with the oracle (tests/test_oracle.py pins the oracle to scipy's
cKDTree, torch's fp32 evaluation of the distance and the reference's own
grid outputs), and the grid selector also directly with the reference's
golden outputs on the rows they pin.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import tarmac_oracle as O
from test_oracle import _grid_row_flags, _lattice

pytestmark = pytest.mark.gpu


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def positions(kind, B, N, seed):
    rng = np.random.default_rng(seed)
    if kind == "uniform":
        return rng.random((B, N, 2)).astype(np.float32)
    if kind == "signed":
        return (rng.random((B, N, 2)) * 2 - 1).astype(np.float32)
    if kind == "cluster":          # a crowded cell block: runs cut at capacity
        p = rng.random((B, N, 2))
        m = N // 3
        p[:, :m] = 0.45 + 0.08 * p[:, :m]
        return p.astype(np.float32)
    if kind == "sparse":           # an empty corner: short candidate lists
        return (rng.random((B, N, 2)) ** 3).astype(np.float32)
    if kind == "dup":              # repeated points: distance-0 ties
        p = rng.random((B, (N + 3) // 4, 2)).astype(np.float32)
        return np.repeat(p, 4, axis=1)[:, :N].copy()
    if kind == "lattice":          # integer lattice: many equal distances
        side = int(np.ceil(np.sqrt(N)))
        return _lattice(B, side, rng)[:, :N].copy()
    raise ValueError(kind)


RADIUS_CASES = [(N, kk) for N in (2, 3, 6, 17, 48, 96, 192, 512, 1000)
                for kk in (1, 2, 3, 4, 7, 8, 16, 17, 40) if kk < N] + [(2048, 4), (2048, 16),
                                                                       (4099, 2), (8192, 8)]


@pytest.mark.parametrize("N,kk", RADIUS_CASES)
def test_radius_knn_exact(N, kk):
    from tarmac.kernels import select_radius_knn
    B = max(1, min(8, 2_000_000 // (N * N)))
    pos = positions("signed", B, N, N * 31 + kk)
    got = host(select_radius_knn(dev(pos), kk))
    assert got.dtype == np.int64 and got.shape == (B, N, kk)
    assert np.array_equal(got, np.sort(O.select_radius_knn(pos, kk), -1))


@pytest.mark.parametrize("kind", ["dup", "lattice", "cluster"])
@pytest.mark.parametrize("N,kk", [(64, 1), (64, 4), (100, 8), (100, 16), (225, 20), (512, 5)])
def test_radius_knn_ties(kind, N, kk):
    """Exact ties (repeated points, lattices) go through the verified-or-exact
    path; the tie rule is the lower agent index."""
    from tarmac.kernels import select_radius_knn
    pos = positions(kind, 3, N, N + kk)
    got = host(select_radius_knn(dev(pos), kk))
    assert np.array_equal(got, np.sort(O.select_radius_knn(pos, kk), -1))


def test_radius_knn_int32_and_stream():
    from tarmac import _launch, _lib
    pos = positions("uniform", 4, 300, 7)
    p = dev(pos)
    idx = torch.empty(4, 300, 6, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        _lib.check(_lib.LIB.tarmac_knn_radius(_launch.ptr(p), _launch.ptr(idx), _lib.IDX_I32,
                                              4, 300, 6, _launch.stream(p)))
    s.synchronize()
    assert np.array_equal(idx.cpu().numpy(), np.sort(O.select_radius_knn(pos, 6), -1))


GRID_CASES = [(N, kk) for N in (48, 96, 192, 512, 1000) for kk in (1, 2, 3, 4, 8, 16, 24, 40)
              if kk < N] + [(4096, 2), (4096, 8), (3000, 16)]


@pytest.mark.parametrize("N,kk", GRID_CASES)
@pytest.mark.parametrize("kind", ["uniform", "cluster", "sparse"])
def test_grid_knn_exact(kind, N, kk):
    from tarmac.kernels import select_grid_knn
    B = 2 if N <= 1000 else 1
    pos = positions(kind, B, N, N * 7 + kk)
    got = host(select_grid_knn(dev(pos), kk))
    assert got.shape == (B, N, kk)
    assert np.array_equal(got, O.select_grid_knn(pos, kk, slot_order=True))


@pytest.mark.parametrize("kind", ["dup", "lattice"])
@pytest.mark.parametrize("N,kk", [(200, 2), (400, 4), (900, 8), (900, 16), (1024, 30)])
def test_grid_knn_ties(kind, N, kk):
    from tarmac.kernels import select_grid_knn
    pos = positions(kind, 2, N, N + 3 * kk)
    got = host(select_grid_knn(dev(pos), kk))
    assert np.array_equal(got, O.select_grid_knn(pos, kk, slot_order=True))


def test_grid_knn_reference_golden(golden):
    """The reference's own select_grid_knn outputs, on the rows they pin
    (no run cut at capacity, at least k candidates)."""
    from tarmac.kernels import select_grid_knn
    checked = 0
    for name in ("g96", "g192", "g512", "gclus", "gsparse"):
        pos = golden[f"{name}_pos"]
        for key in [f for f in golden.files if f.startswith(name + "_grid")]:
            kk = int(key[len(name) + 5:])
            cut, short = _grid_row_flags(pos, kk)
            use = ~cut & ~short
            got = np.sort(host(select_grid_knn(dev(pos), kk)), -1)
            assert np.array_equal(got[use], golden[key].astype(np.int64)[use]), key
            checked += int(use.sum())
    assert checked > 3000


def test_grid_recall_and_selectors_table():
    from tarmac.kernels import SELECTORS, grid_knn_recall
    assert set(SELECTORS) == {"radius_knn", "grid_knn", "morton_window"}
    pos = dev(positions("uniform", 8, 512, 3))
    r = grid_knn_recall(pos, 4)
    assert 0.99 <= r <= 1.0


@pytest.mark.parametrize("selector", ["radius_knn", "grid_knn", "morton_window"])
def test_prescore_full(selector):
    """prescore_full (prescore_selection.py:198-200): selector then attention
    over the selected set, against the oracle composition."""
    from conftest import qkv
    from tarmac.kernels import prescore_full
    q, k, v = qkv(91, 4, 192, 16)
    pos = positions("uniform", 4, 192, 91)
    out = host(prescore_full(*(torch.from_numpy(x).cuda() for x in (q, k, v)), dev(pos), 4,
                             selector))
    sel = {"radius_knn": O.select_radius_knn, "grid_knn": O.select_grid_knn,
           "morton_window": O.select_morton_window}[selector]
    ref = O.prescore_attention(q.astype(np.float64), k.astype(np.float64),
                               v.astype(np.float64), sel(pos, 4))
    assert np.abs(out - ref).max() / np.abs(ref).max() <= 1e-5
