"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against something that is not a retyping of
its own formula: a library routine (torch in float64), a closed form, brute
force on tiny inputs, or golden vectors written by the reference's own code
(tests/golden/make_golden.py). The mutation tests at the end plant plausible
mistakes in copies of the oracle and check that these pins catch them.
"""

from __future__ import annotations

import itertools
from fractions import Fraction

import numpy as np
import pytest
import torch

import tarmac_oracle as O
from conftest import qkv

F64 = np.float64


def _sdpa_ref(q, k, v):
    """torch's SDPA in float64 with the -inf diagonal mask (a library routine)."""
    N = q.shape[1]
    mask = torch.zeros(N, N, dtype=torch.float64)
    mask.masked_fill_(torch.eye(N, dtype=torch.bool), float("-inf"))
    t = [torch.from_numpy(np.asarray(x, F64)).unsqueeze(1) for x in (q, k, v)]
    return torch.nn.functional.scaled_dot_product_attention(*t, attn_mask=mask).squeeze(1).numpy()


# ---------------------------------------------------------------------------
# pins as reusable predicates (so the mutation tests can run them on mutants)
# ---------------------------------------------------------------------------

def pin_scores(scores_fn) -> bool:
    q, k, _ = qkv(1, 3, 9, 16, F64)
    s = scores_fn(q, k)
    ref = torch.matmul(torch.from_numpy(q), torch.from_numpy(k).transpose(-1, -2)).numpy() / 4.0
    off = ~np.eye(9, dtype=bool)[None].repeat(3, 0)
    ok = np.allclose(s[off], ref[off], rtol=1e-12, atol=1e-12)
    ok &= bool(np.all(np.isneginf(s[:, np.arange(9), np.arange(9)])))
    # unit-vector closed form: q = e_c gives column c of K / sqrt(d)
    e = np.zeros((1, 4, 16)); e[0, :, :4] = np.eye(4)
    kk = np.random.default_rng(3).standard_normal((1, 4, 16))
    s2 = scores_fn(e, kk)
    for i in range(4):
        for j in range(4):
            if i != j:
                ok &= abs(s2[0, i, j] - kk[0, j, i] / 4.0) < 1e-15
    return bool(ok)


def pin_dense(dense_fn) -> bool:
    q, k, v = qkv(2, 4, 11, 16, F64)
    out = dense_fn(q, k, v)
    ok = np.allclose(out, _sdpa_ref(q, k, v), rtol=1e-12, atol=1e-12)
    # constant V rows -> the output is that constant
    vc = np.broadcast_to(np.arange(16, dtype=F64), v.shape).copy()
    ok &= np.allclose(dense_fn(q, k, vc), vc, atol=1e-12)
    # equal keys -> uniform weights over the N-1 peers
    ke = np.broadcast_to(k[:, :1, :], k.shape).copy()
    want = (v.sum(1, keepdims=True) - v) / (v.shape[1] - 1)
    ok &= np.allclose(dense_fn(q, ke, v), want, atol=1e-12)
    return bool(ok)


def pin_topk_indices(topk_fn) -> bool:
    rng = np.random.default_rng(4)
    ok = True
    s = rng.standard_normal((5, 7, 13))
    for kk in (1, 2, 5, 12):
        got = topk_fn(s, kk)
        ref = torch.from_numpy(s).topk(kk, dim=-1).indices.numpy()  # library, tie-free rows
        ok &= np.array_equal(np.sort(got, -1), np.sort(ref, -1))
    # brute force: the retained set is the k-subset whose worst beats the best outside
    row = rng.standard_normal(7)
    for kk in range(1, 7):
        best = [c for c in itertools.combinations(range(7), kk)
                if min(row[list(c)]) > max(np.delete(row, list(c)), default=-np.inf)]
        ok &= sorted(topk_fn(row[None, None], kk)[0, 0].tolist()) == list(best[0])
    # ties keep the lower index; order is score desc then index asc
    tied = np.array([[[0.5, 1.0, 0.25, 1.0, 1.0, -2.0]]])
    ok &= topk_fn(tied, 2)[0, 0].tolist() == [1, 3]
    ok &= topk_fn(tied, 4)[0, 0].tolist() == [1, 3, 4, 0]
    ok &= topk_fn(np.array([[[0.0, -0.0, 0.0]]]), 1)[0, 0].tolist() == [0]
    return bool(ok)


def pin_topk_gather(gather_fn, masked_fn, dense_fn) -> bool:
    ok = True
    for N in (6, 12, 24):
        for kk in (1, 2, 3, N - 1):
            q, k, v = qkv(N * 100 + kk, 8, N, 8, F64)
            a = masked_fn(q, k, v, kk)
            b, idx = gather_fn(q, k, v, kk)
            ok &= float(np.abs(a - b).max()) < 1e-10       # test_comm_module.py:322-344
            ok &= idx.shape == (8, N, kk)
            ok &= not np.any(idx == np.arange(N)[None, :, None])  # never self
        q, k, v = qkv(N, 3, N, 8, F64)
        ok &= float(np.abs(gather_fn(q, k, v, N - 1)[0] - dense_fn(q, k, v)).max()) < 1e-12
    return bool(ok)


def _morton_bitloop(g0, g1, bits):
    c = 0
    for b in range(bits):
        c |= ((g0 >> b) & 1) << (2 * b)
        c |= ((g1 >> b) & 1) << (2 * b + 1)
    return c


def pin_morton(code_fn, golden) -> bool:
    ok = True
    for name in ("m6", "m64", "m512", "mgrid", "mflat", "mline"):
        pos = golden[f"{name}_pos"]
        for bits in (10, 16):
            ok &= np.array_equal(code_fn(pos, bits), golden[f"{name}_code{bits}"].astype(np.int64))
    # the interleave itself, against a bit-by-bit loop on every 8-bit pair
    g = np.arange(256)
    x, y = np.meshgrid(g, g, indexing="ij")
    spread = O.spread_bits(x.ravel()) | (O.spread_bits(y.ravel()) << 1)
    ok &= all(int(spread[i]) == _morton_bitloop(int(a), int(b), 8)
              for i, (a, b) in enumerate(zip(x.ravel(), y.ravel())) if i % 37 == 0)
    return bool(ok)


def _tie_rows(seed, B, N):
    """fp32 score rows with exact ties: values on a coarse grid, -inf self pair."""
    rng = np.random.default_rng(seed)
    s = rng.integers(-3, 4, size=(B, N, N)).astype(np.float32) * np.float32(0.5)
    s[:, np.arange(N), np.arange(N)] = -np.inf
    return s


def pin_ordered_key(key_fn) -> bool:
    specials = np.array([-np.inf, -3e38, -1.0, -1e-40, -0.0, 0.0, 1e-40, 1.0, 3e38, np.inf],
                        np.float32)
    rng = np.random.default_rng(11)
    rand = (rng.standard_normal(2000) * np.exp(rng.uniform(-20, 20, 2000))).astype(np.float32)
    vals = np.concatenate([specials, rand])
    keys = key_fn(vals).astype(np.int64)
    a, b = vals[:, None], vals[None, :]
    ka, kb = keys[:, None], keys[None, :]
    # strict order agrees wherever the floats are ordered (-0 == +0 is a tie
    # for floats, ordered by sign for keys)
    ok = np.all((a < b) <= (ka < kb)) and np.all((a > b) <= (ka > kb))
    return bool(ok and key_fn(np.float32([-0.0]))[0] < key_fn(np.float32([0.0]))[0])


def pin_masked_keep(keep_fn) -> bool:
    ok = True
    for seed, (B, N) in enumerate([(3, 7), (2, 12), (2, 33)]):
        for s in (_tie_rows(seed, B, N), O.scores(*qkv(seed, B, N, 16, np.float32)[:2]).astype(np.float32)):
            for kk in (1, 2, N // 2, N - 1):
                # closed form at full precision: every peer at or above the k-th score
                kth = -np.sort(-s, -1)[..., kk - 1:kk]
                ok &= np.array_equal(keep_fn(s, kk, 34), s >= kth)
                ok &= np.array_equal(keep_fn(s, kk, 32), s >= kth)
                # no halving keeps every valid peer; fewer halvings keep a superset
                ok &= np.array_equal(keep_fn(s, kk, 0), ~np.eye(N, dtype=bool)[None].repeat(B, 0))
                for b in (3, 10, 20):
                    ok &= bool(np.all(keep_fn(s, kk, b) >= (s >= kth)))
                    ok &= bool(np.all(keep_fn(s, kk, b) >= keep_fn(s, kk, b + 1)))
    return bool(ok)


def pin_sort_select(sel_fn) -> bool:
    ok = True
    for seed, (B, N) in enumerate([(2, 6), (3, 9)]):
        s = _tie_rows(seed, B, N)
        for kk in (1, 2, 3, N - 1):
            got = sel_fn(s, kk)
            for b in range(B):
                for i in range(N):
                    # brute force: sort (score, index) pairs, both descending
                    pairs = sorted(((float(s[b, i, j]), j) for j in range(N)), reverse=True)
                    ok &= sorted(int(x) for x in got[b, i]) == sorted(j for _, j in pairs[:kk])
    return bool(ok)


# ---------------------------------------------------------------------------
# the pins, applied to the oracle
# ---------------------------------------------------------------------------

def test_ordered_key_pinned():
    assert pin_ordered_key(O.ordered_key)


def test_masked_threshold_pinned():
    assert pin_masked_keep(O.masked_threshold_keep)


def test_sort_select_pinned():
    assert pin_sort_select(O.sort_select)


def test_weights_attention_is_topk_gather_on_the_topk_set():
    q, k, v = qkv(8, 3, 10, 16, F64)
    s = O.scores(q, k)
    for kk in (1, 3, 9):
        idx = O.topk_indices(s, kk)
        keep = np.zeros_like(s, dtype=bool)
        np.put_along_axis(keep, idx, True, -1)
        assert np.allclose(O.weights_attention(s, keep, v), O.topk_gather(q, k, v, kk)[0],
                           rtol=1e-12, atol=1e-12)


def test_scores_pinned():
    assert pin_scores(O.scores)


def test_dense_pinned():
    assert pin_dense(O.dense_unfused)


def test_dense_rows_are_distributions_excluding_self():
    q, k, _ = qkv(5, 4, 6, 16, F64)
    w = O.softmax(O.scores(q, k))
    assert np.allclose(w.sum(-1), 1.0, atol=1e-12)
    assert np.abs(w[:, np.arange(6), np.arange(6)]).max() == 0.0


def test_topk_indices_pinned():
    assert pin_topk_indices(O.topk_indices)


def test_topk_gather_pinned():
    assert pin_topk_gather(O.topk_gather, O.topk_masked, O.dense_unfused)


def test_topk_exactly_k_nonzero_weights():
    for N in (6, 12):
        for kk in (1, 2, N - 1):
            q, k, v = qkv(N + kk, 3, N, 16, F64)
            s = O.scores(q, k)
            idx = O.topk_indices(s, kk)
            w = np.zeros_like(s)
            np.put_along_axis(w, idx, O.softmax(np.take_along_axis(s, idx, -1)), -1)
            assert np.all((w > 0).sum(-1) == kk)
            assert np.allclose(w.sum(-1), 1.0, atol=1e-12)


def test_k_eff_clamp():
    assert [O.k_eff(k, 6) for k in (-3, 0, 1, 5, 6, 99)] == [1, 1, 1, 5, 5, 5]


def test_morton_pinned(golden):
    assert pin_morton(O.morton_code, golden)


def test_morton_window_golden(golden):
    """select_morton_window against the reference's own outputs (bits = 10),
    on batch rows whose codes are distinct (the reference's argsort is not
    stable, so rows with equal codes have no pinned order)."""
    checked = 0
    for name in ("m6", "m64", "m512", "mgrid"):
        pos = golden[f"{name}_pos"]
        distinct = golden[f"{name}_distinct10"]
        for kk in (1, 2, 3, 4):
            key = f"{name}_win{kk}"
            if key not in golden:
                continue
            got = O.select_morton_window(pos, kk, 10)
            ref = golden[key].astype(np.int64)
            for b in np.flatnonzero(distinct):
                assert np.array_equal(got[b], ref[b]), (name, kk, b)
                checked += 1
    assert checked >= 10


@pytest.mark.parametrize("N,kk", [(6, 1), (6, 2), (6, 4), (12, 3), (64, 5)])
def test_morton_window_properties(N, kk):
    rng = np.random.default_rng(N * 10 + kk)
    pos = (rng.random((16, N, 2)) * 2 - 1).astype(np.float32)
    idx = O.select_morton_window(pos, kk, 16)
    assert idx.shape == (16, N, kk)
    assert not np.any(idx == np.arange(N)[None, :, None])
    srt = np.sort(idx, -1)
    assert np.all(srt[..., 1:] != srt[..., :-1])
    # curve neighbours, from an independent ordering by the bit-loop code
    half = (kk + 1) // 2
    offs = list(range(1, half + 1)) + [-o for o in range(1, kk - half + 1)]
    for b in range(4):
        lo, hi = pos[b].min(0), pos[b].max(0)
        span = np.maximum(hi - lo, np.float32(1e-6))
        g = ((pos[b] - lo) / span * np.float32(65535)).astype(np.int64).clip(0, 65535)
        codes = [_morton_bitloop(int(x), int(y), 16) for x, y in g]
        order = sorted(range(N), key=lambda i: (codes[i], i))
        rank = {a: r for r, a in enumerate(order)}
        for i in range(N):
            assert set(idx[b, i].tolist()) == {order[(rank[i] + o) % N] for o in offs}


def test_prescore_equals_dense_restricted_to_selected():
    """src tests/test_zorder_comm.py:74-89, on the oracle."""
    q, k, v = qkv(9, 5, 10, 16, F64)
    rng = np.random.default_rng(9)
    pos = rng.random((5, 10, 2)).astype(np.float32)
    idx = O.select_morton_window(pos, 3, 10)
    got = O.prescore_attention(q, k, v, idx)
    s = O.scores(q, k)
    keep = np.zeros_like(s, dtype=bool)
    np.put_along_axis(keep, idx, True, -1)
    w = O.softmax(np.where(keep, np.matmul(q, np.swapaxes(k, -1, -2)) / 4.0, -np.inf))
    assert np.abs(got - w @ v).max() < 1e-12


# ---------------------------------------------------------------------------
# the canonical-order C oracle
# ---------------------------------------------------------------------------

def _rf32(fr: Fraction) -> np.float32:
    """Correctly rounded Fraction -> float32 (round to nearest even)."""
    if fr == 0:
        return np.float32(0.0)
    x = np.float32(float(fr))
    best = None
    for c in (np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))):
        e = abs(Fraction(float(c)) - fr)
        if best is None or e < best[0] or (e == best[0] and int(c.view(np.uint32)) & 1 == 0):
            best = (e, c)
    return best[1]


def test_canon_scores_match_exact_fmaf_chain():
    """Brute force: the C oracle's score equals an exactly-rounded fmaf chain in
    slot order (c = kk*(d/4)+t), times fp32(1/sqrt(d))."""
    for d in (8, 16, 32):
        q, k, _ = qkv(d, 1, 5, d)
        s = O.canon_scores(q, k)
        sc = np.float32(1.0 / np.sqrt(d))
        for i in range(5):
            for j in range(5):
                if i == j:
                    continue
                acc = np.float32(0.0)
                for t in range(d // 4):
                    for kk in range(4):
                        c = kk * (d // 4) + t
                        acc = _rf32(Fraction(float(q[0, i, c])) * Fraction(float(k[0, j, c]))
                                    + Fraction(float(acc)))
                want = _rf32(Fraction(float(acc)) * Fraction(float(sc)))
                assert s[0, i, j] == want, (d, i, j)


@pytest.mark.parametrize("N,d,kk", [(6, 16, 2), (32, 16, 1), (64, 8, 4), (100, 32, 3), (128, 64, 8)])
def test_canon_topk_matches_float64_oracle(N, d, kk):
    q, k, v = qkv(N * 131 + d * 17 + kk, 6, N, d)
    out_c, idx_c = O.canon_topk(q, k, v, kk)
    out_r, idx_r = O.topk_gather(q.astype(F64), k.astype(F64), v.astype(F64), kk)
    s64 = O.scores(q.astype(F64), k.astype(F64))
    ambiguous = O.near_tie_rows(s64, kk, O.score_error_bound(q, k).max(-1))
    same = np.all(np.sort(idx_c, -1) == np.sort(idx_r, -1), -1)
    assert np.all(same | ambiguous)
    assert ambiguous.mean() < 0.01
    scale = np.abs(out_r).max()
    assert np.abs(out_c - out_r)[same].max() <= 1e-6 * scale


def test_canon_morton_matches_numpy_oracle(golden):
    for name in ("m6", "m64", "m512", "mgrid", "mflat", "mline"):
        pos = golden[f"{name}_pos"]
        for bits in (10, 16):
            assert np.array_equal(O.canon_morton_codes(pos, bits), O.morton_code(pos, bits))
            n = pos.shape[1]
            for kk in (1, 2, min(5, n - 1)):
                assert np.array_equal(O.canon_morton_window(pos, kk, bits),
                                      O.select_morton_window(pos, kk, bits))


def test_canon_dense_and_fixedset():
    q, k, v = qkv(21, 3, 17, 16)
    ref = O.dense_unfused(q.astype(F64), k.astype(F64), v.astype(F64))
    assert np.abs(O.canon_dense(q, k, v) - ref).max() < 1e-12
    pos = np.random.default_rng(2).random((3, 17, 2)).astype(np.float32)
    idx = O.select_morton_window(pos, 4, 16)
    ref = O.prescore_attention(q.astype(F64), k.astype(F64), v.astype(F64), idx)
    assert np.abs(O.canon_fixedset(q, k, v, idx) - ref).max() < 1e-12


def test_bf16_round_matches_torch():
    x = np.random.default_rng(0).standard_normal(4096).astype(np.float32) * 100
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.bf16_round(x), want)


# ---------------------------------------------------------------------------
# planted mistakes: the pins must reject these mutants
# ---------------------------------------------------------------------------

# ---------------------------------------------------------------------------
# kNN selectors
# ---------------------------------------------------------------------------

def _lattice(B, side, rng):
    """Agents on an integer lattice (shuffled): many exactly equal distances."""
    g = np.stack(np.meshgrid(np.arange(side), np.arange(side), indexing="ij"), -1).reshape(-1, 2)
    return np.stack([g[rng.permutation(len(g))] for _ in range(B)]).astype(np.float32)


def pin_pair_d2(fn) -> bool:
    rng = np.random.default_rng(5)
    p = rng.random((64, 2)).astype(np.float32)
    c = (rng.random((64, 2)) * 3 - 1).astype(np.float32)
    got = fn(p, c).astype(F64)
    ref = ((c.astype(F64) - p.astype(F64)) ** 2).sum(-1)
    ok = np.allclose(got, ref, rtol=4 * 2.0 ** -24, atol=0)
    li = _lattice(1, 5, rng)[0]
    ok &= np.array_equal(fn(li[:1], li), ((li - li[:1]) ** 2).sum(-1))
    # bit for bit: torch's fp32 evaluation of the reference expression
    # (pc - pos).square().sum(-1), prescore_selection.py:155-156
    pt = (torch.from_numpy(c) - torch.from_numpy(p)).square().sum(-1).numpy()
    ok &= np.array_equal(fn(p, c), pt)
    return bool(ok)


def pin_radius_knn(fn) -> bool:
    """Against scipy's cKDTree (float64) on rows with no near-tie at the k-th
    neighbour, and against brute force (index tie rule) on lattices."""
    from scipy.spatial import cKDTree
    rng = np.random.default_rng(11)
    ok = True
    for N, kk in ((7, 1), (7, 6), (48, 4), (96, 16), (300, 9)):
        pos = (rng.random((3, N, 2)) * 2 - 1).astype(np.float32)
        got = np.sort(fn(pos, kk), -1)
        for b in range(3):
            dist, ii = cKDTree(pos[b].astype(F64)).query(pos[b].astype(F64), kk + 2)
            # drop the self pair, keep rows where the k-th and (k+1)-th differ clearly
            for i in range(N):
                row = [(d, j) for d, j in zip(dist[i], ii[i]) if j != i][: kk + 1]
                if len(row) == kk + 1 and row[kk][0] - row[kk - 1][0] <= 1e-5 * (1 + row[kk][0]):
                    continue
                ok &= np.array_equal(got[b, i], np.sort([j for _, j in row[:kk]]))
    lat = _lattice(2, 6, rng)
    got = fn(lat, 5)
    for b in range(2):
        for i in range(36):
            d = ((lat[b] - lat[b, i]) ** 2).sum(-1).astype(F64)
            d[i] = np.inf
            want = sorted(range(36), key=lambda j: (d[j], j))[:5]
            ok &= sorted(got[b, i].tolist()) == sorted(want)
    return bool(ok)


def pin_grid_knn(fn, golden) -> bool:
    """The reference's own outputs on rows whose runs were not cut and hold at
    least k candidates; on other rows the unstable argsort / topk decide."""
    checked = 0
    ok = True
    for name in ("g96", "g192", "g512", "gclus", "gsparse"):
        pos = golden[f"{name}_pos"]
        for key in [f for f in golden.files if f.startswith(name + "_grid")]:
            kk = int(key[len(name) + 5:])
            cut, short = _grid_row_flags(pos, kk)
            got = np.sort(fn(pos, kk), -1)
            ref = golden[key].astype(np.int64)
            use = ~cut & ~short
            ok &= np.array_equal(got[use], ref[use])
            checked += int(use.sum())
    return bool(ok) and checked > 3000


def _grid_row_flags(pos, kk):
    """(a run was cut at capacity, fewer than k candidates) per query."""
    B, N, _ = pos.shape
    G, M = O.grid_knn_shape(N, kk)
    L = 3 * M
    cxy = O.grid_cells(pos, G)
    cell = cxy[..., 0] * G + cxy[..., 1]
    start = np.zeros((B, G * G + 1), np.int64)
    for b in range(B):
        start[b, 1:] = np.cumsum(np.bincount(cell[b], minlength=G * G))
    x = cxy[..., 0][..., None] + np.arange(-1, 2)
    y = cxy[..., 1][..., None]
    okc = (x >= 0) & (x < G)
    xc = np.clip(x, 0, G - 1)
    s_lo = np.take_along_axis(start, (xc * G + np.maximum(y - 1, 0)).reshape(B, -1), 1).reshape(B, N, 3)
    s_hi = np.take_along_axis(start, (xc * G + np.minimum(y + 1, G - 1) + 1).reshape(B, -1), 1).reshape(B, N, 3)
    cut = ((s_hi - s_lo > L) & okc).any(-1)
    short = (np.minimum(s_hi - s_lo, L) * okc).sum(-1) - 1 < kk
    return cut, short


def test_pair_d2_pinned():
    assert pin_pair_d2(O.pair_d2)


def test_radius_knn_pinned():
    assert pin_radius_knn(O.select_radius_knn)


def test_grid_knn_shape_golden(golden):
    for N, kk, G, M in golden["grid_shape"]:
        assert O.grid_knn_shape(int(N), int(kk)) == (G, M)


def test_grid_knn_pinned(golden):
    assert pin_grid_knn(O.select_grid_knn, golden)


@pytest.mark.parametrize("N,kk", [(96, 2), (512, 4), (512, 16)])
def test_grid_knn_equals_radius_where_exact(N, kk):
    """The reference's exactness condition: the k-th neighbour no farther
    than the nearest edge of the 3x3 block, and no run cut."""
    rng = np.random.default_rng(N + kk)
    pos = rng.random((3, N, 2)).astype(np.float32)
    grid = np.sort(O.select_grid_knn(pos, kk), -1)
    rad = O.select_radius_knn(pos, kk)
    G, M = O.grid_knn_shape(N, kk)
    lo = pos.min(1, keepdims=True)
    span = np.maximum(pos.max(1, keepdims=True) - lo, np.float32(1e-6))
    u = ((pos - lo) / span * G).astype(F64)             # position in cell units
    c = np.clip(np.floor(u), 0, G - 1)
    # distance (cell units) to the nearest block edge that is not the grid border
    edge = np.minimum(np.where(c > 0, u - (c - 1), np.inf), np.where(c < G - 1, c + 2 - u, np.inf)).min(-1)
    kth = np.sqrt(O.pair_d2(pos, np.take_along_axis(pos, rad[..., -1:].repeat(2, -1), 1)))
    kth_cells = kth * G / span.min(-1)
    cut, short = _grid_row_flags(pos, kk)
    safe = (kth_cells < edge * 0.999) & ~cut & ~short
    assert safe.mean() > 0.5
    assert np.array_equal(grid[safe], np.sort(rad, -1)[safe])


def test_grid_knn_all_pairs_route():
    """9M >= N: the reference calls select_radius_knn (:127-128)."""
    rng = np.random.default_rng(2)
    pos = rng.random((2, 48, 2)).astype(np.float32)
    G, M = O.grid_knn_shape(48, 4)
    assert 9 * M >= 48
    assert np.array_equal(O.select_grid_knn(pos, 4), O.select_radius_knn(pos, 4))


def test_pins_reject_planted_mistakes(golden):
    def scores_mul_sqrt(q, k):         # multiplies by sqrt(d) instead of dividing
        s = O.scores(q, k)
        return s * q.shape[-1]

    def scores_no_mask(q, k):          # forgets the self-diagonal
        return np.matmul(q, np.swapaxes(k, -1, -2)) / np.sqrt(q.shape[-1])

    def scores_transposed(q, k):       # Q^T K-style index mix-up (S_ji)
        return np.swapaxes(O.scores(q, k), -1, -2) if q is not k else O.scores(q, k)

    assert not pin_scores(scores_mul_sqrt)
    assert not pin_scores(scores_no_mask)

    def dense_uses_k_for_v(q, k, v):
        return np.matmul(O.softmax(O.scores(q, k)), k)

    def dense_transposed_weights(q, k, v):
        return np.matmul(np.swapaxes(O.softmax(O.scores(q, k)), -1, -2), v)

    assert not pin_dense(dense_uses_k_for_v)
    assert not pin_dense(dense_transposed_weights)
    assert not pin_dense(lambda q, k, v: np.matmul(O.softmax(scores_transposed(q, k)), v))

    assert not pin_topk_indices(lambda s, kk: np.argsort(s, -1, kind="stable")[..., :kk])
    assert not pin_topk_indices(lambda s, kk: np.argsort(-s, -1, kind="stable")[..., -kk:])
    # ties resolved to the higher index
    assert not pin_topk_indices(
        lambda s, kk: (s.shape[-1] - 1 - np.argsort(-s[..., ::-1], -1, kind="stable"))[..., :kk])

    def gather_softmax_all(q, k, v, topk):   # softmax over all N, not the kept k
        out, idx = O.topk_gather(q, k, v, topk)
        w = O.softmax(O.scores(q, k))
        return np.einsum("bnk,bnkd->bnd", np.take_along_axis(w, idx, -1), O.gather_rows(v, idx)), idx

    assert not pin_topk_gather(gather_softmax_all, O.topk_masked, O.dense_unfused)

    def morton_swapped_axes(pos, bits):
        return O.morton_code(pos[..., ::-1].copy(), bits)

    def morton_rounding(pos, bits):     # rounds instead of truncating
        pos = np.asarray(pos, np.float32)
        lo, hi = pos.min(1, keepdims=True), pos.max(1, keepdims=True)
        span = np.maximum(hi - lo, np.float32(1e-6))
        g = np.rint((pos - lo) / span * np.float32((1 << bits) - 1)).astype(np.int64)
        return O.spread_bits(g[..., 0]) | (O.spread_bits(g[..., 1]) << 1)

    assert not pin_morton(morton_swapped_axes, golden)
    assert not pin_morton(morton_rounding, golden)

    # ordered key without the sign fix-up, or with the wrong mask
    assert not pin_ordered_key(lambda x: np.ascontiguousarray(x, np.float32).view(np.int32))
    assert not pin_ordered_key(
        lambda x: (lambda i: i ^ ((i >> 31) & np.int32(0x7FFFFF)))(
            np.ascontiguousarray(x, np.float32).view(np.int32)))

    def masked_strict(s, topk, bisect=34):         # keys > lo drops the k-th itself
        keys = O.ordered_key(s).astype(np.int64)
        return keys > np.where(O.masked_threshold_keep(s, topk, bisect),
                               keys, np.iinfo(np.int64).max).min(-1, keepdims=True)

    def masked_counts_above(s, topk, bisect=34):  # off by one: needs more than topk
        keys = O.ordered_key(s).astype(np.int64)
        n = s.shape[-1]
        lo = np.where(~np.eye(n, dtype=bool), keys, np.iinfo(np.int64).max).min(-1)
        hi = keys.max(-1)
        for _ in range(bisect):
            mid = lo + (hi - lo + 1) // 2
            take = (keys >= mid[..., None]).sum(-1) > topk
            lo, hi = np.where(take, mid, lo), np.where(take, hi, mid - 1)
        return keys >= lo[..., None]

    assert not pin_masked_keep(masked_strict)
    assert not pin_masked_keep(masked_counts_above)

    def sort_low_index(s, topk):                   # ties keep the lower index
        return O.topk_indices(s, topk)

    assert not pin_sort_select(sort_low_index)

    # kNN: fused multiply-add in the distance; largest instead of smallest;
    # self pair not excluded; cell rounding instead of truncation
    def d2_fma(p, c):                   # x*x + (y*y) with one rounding (contracted)
        diff = (np.asarray(c, np.float32) - np.asarray(p, np.float32)).astype(F64)
        yy = (diff[..., 1] * diff[..., 1]).astype(np.float32).astype(F64)
        return (diff[..., 0] * diff[..., 0] + yy).astype(np.float32)

    assert not pin_pair_d2(d2_fma)

    def radius_farthest(pos, kk):
        d2 = O.pair_d2(pos[:, :, None, :], pos[:, None, :, :])
        d2[:, np.arange(pos.shape[1]), np.arange(pos.shape[1])] = -np.inf
        return np.argsort(-d2, -1, kind="stable")[..., :kk]

    def radius_with_self(pos, kk):
        d2 = O.pair_d2(pos[:, :, None, :], pos[:, None, :, :])
        return np.argsort(d2, -1, kind="stable")[..., :kk]

    def radius_high_index_ties(pos, kk):
        n = pos.shape[1]
        return n - 1 - O.select_radius_knn(pos[:, ::-1].copy(), kk)

    assert not pin_radius_knn(radius_farthest)
    assert not pin_radius_knn(radius_with_self)
    assert not pin_radius_knn(radius_high_index_ties)

    real_cells = O.grid_cells
    try:
        O.grid_cells = lambda pos, G: np.clip(np.rint(
            (pos - pos.min(1, keepdims=True)) / np.maximum(
                pos.max(1, keepdims=True) - pos.min(1, keepdims=True), np.float32(1e-6))
            * np.float32(G)).astype(np.int64), 0, G - 1)
        assert not pin_grid_knn(O.select_grid_knn, golden)
    finally:
        O.grid_cells = real_cells


# ---------------------------------------------------------------------------
# score_error_bound and near_tie_rows
# ---------------------------------------------------------------------------

def _chain_order(d):
    """Elements of a row in the canonical chain's order: c = kk*(d/4) + t at
    step t, slot kk."""
    return [kk * (d // 4) + t for t in range(d // 4) for kk in range(4)]


def _worst_case_pair(d):
    """A query/key pair whose canonical score loses close to half an ulp at
    every one of its d roundings, in the same direction: the first product
    (1 + 2^-23)(1 - 2^-24) = 1 + 2^-24 - 2^-47 rounds down to 1, and every later
    term 2^-24 - 2^-34 is just under half an ulp of the running 1.0, so it is
    lost too. Returns q, k as [1, 2, d] (query 0 against key 1)."""
    q = np.zeros((1, 2, d), np.float32)
    k = np.zeros((1, 2, d), np.float32)
    order = _chain_order(d)
    q[0, 0, order[0]] = np.float32(1 + 2.0 ** -23)
    k[0, 1, order[0]] = np.float32(1 - 2.0 ** -24)
    for c in order[1:]:
        q[0, 0, c] = np.float32(2.0 ** -24 - 2.0 ** -34)
        k[0, 1, c] = np.float32(1.0)
    return q, k


def _score_errors(q, k):
    """|canonical fp32 score - exact q.k/sqrt(d)| for every off-diagonal pair,
    evaluated in 60-digit decimal from the exact rational dot."""
    import decimal
    ctx = decimal.Context(prec=60)
    d = q.shape[-1]
    inv_sqrt = ctx.divide(decimal.Decimal(1), ctx.sqrt(decimal.Decimal(d)))
    s = O.canon_scores(q, k)
    B, N, _ = q.shape
    err = np.zeros((B, N, N))
    for b in range(B):
        for i in range(N):
            for j in range(N):
                if i == j:
                    continue
                dot = sum(Fraction(float(q[b, i, c])) * Fraction(float(k[b, j, c])) for c in range(d))
                exact = ctx.multiply(ctx.divide(decimal.Decimal(dot.numerator),
                                                decimal.Decimal(dot.denominator)), inv_sqrt)
                err[b, i, j] = float(abs(ctx.subtract(decimal.Decimal(float(s[b, i, j])), exact)))
    return err


def _cancelling_rows(d, seed):
    """Rows whose products nearly cancel: large alternating terms and a small
    remainder, so |q.k| is far below sum |q_c k_c|."""
    rng = np.random.default_rng(seed)
    q = np.empty((1, 4, d), np.float32)
    k = np.empty((1, 4, d), np.float32)
    big = rng.uniform(50, 100, (4, d // 2)).astype(np.float32)
    q[0, :, 0::2] = big
    q[0, :, 1::2] = -big * np.float32(1 + 2.0 ** -20)
    k[0] = rng.uniform(0.999, 1.001, (4, d)).astype(np.float32)
    return q, k


def pin_score_error_bound(bound_fn) -> bool:
    """The bound must dominate the exact error of every canonical score
    (random, cancellation-heavy and worst-case chains), and the worst-case
    chain must reach at least 0.85 of it (the bound is tight, not just safe:
    0.89 at d = 16, 0.95 at d = 32)."""
    for d in (16, 32):
        cases = [qkv(d + 1, 2, 5, d)[:2], _cancelling_rows(d, d), _worst_case_pair(d)]
        for q, k in cases:
            single = bound_fn(q, k) / 2
            err = _score_errors(q, k)
            off = np.broadcast_to(~np.eye(q.shape[1], dtype=bool), err.shape)
            if not np.all(err[off] <= single[off]):
                return False
        q, k = _worst_case_pair(d)
        if _score_errors(q, k)[0, 0, 1] < 0.85 * bound_fn(q, k)[0, 0, 1] / 2:
            return False
    return True


def pin_near_tie_rows(fn) -> bool:
    """Brute force over Python-sorted rows, and exact gaps at the boundary."""
    rng = np.random.default_rng(3)
    s = rng.standard_normal((40, 9))
    s[:, 0] = -np.inf  # a masked self pair
    for kk in (1, 2, 4, 7):
        eps = rng.uniform(0, 0.5, 40)
        want = []
        for row, e in zip(s, eps):
            srt = sorted(row.tolist(), reverse=True)
            want.append(srt[kk - 1] - srt[kk] <= e)
        if not np.array_equal(fn(s, kk, eps), np.array(want)):
            return False
    row = np.array([[-np.inf, 5.0, 4.0, 3.0, 2.75, 1.0]])
    if not (fn(row, 3, 0.25)[0] and not fn(row, 3, 0.2)[0] and not fn(row, 2, 0.25)[0]):
        return False
    return not fn(row, 6, 10.0)[0]  # no (k+1)-th score: never a near-tie


def test_score_error_bound_pinned():
    assert pin_score_error_bound(O.score_error_bound)


def test_near_tie_rows_pinned():
    assert pin_near_tie_rows(O.near_tie_rows)


def test_error_bound_pins_reject_planted_mistakes():
    u = 2.0 ** -24

    def halved(q, k):
        return O.score_error_bound(q, k) / 2

    def gamma_d(q, k):                 # counts d roundings: misses the scale's two
        d = q.shape[-1]
        a = np.matmul(np.abs(q.astype(np.float64)), np.abs(np.swapaxes(k, -1, -2)).astype(np.float64))
        return 2 * (d * u / (1 - d * u)) * a / np.sqrt(d)

    def no_abs(q, k):                  # |q.k| instead of sum |q_c k_c|
        d = q.shape[-1]
        g = (d + 2) * u / (1 - (d + 2) * u)
        return 2 * g * np.abs(np.matmul(q.astype(np.float64),
                                        np.swapaxes(k, -1, -2).astype(np.float64))) / np.sqrt(d)

    def no_scale(q, k):                # forgets the 1/sqrt(d): safe but sqrt(d) too loose
        return O.score_error_bound(q, k) * np.sqrt(q.shape[-1])

    for mutant in (halved, gamma_d, no_abs, no_scale):
        assert not pin_score_error_bound(mutant), mutant.__name__

    def strict(s, kk, eps):
        srt = -np.sort(-s, axis=-1)
        if kk >= s.shape[-1]:
            return np.zeros(s.shape[:-1], dtype=bool)
        return srt[..., kk - 1] - srt[..., kk] < eps

    def off_by_one(s, kk, eps):
        srt = -np.sort(-s, axis=-1)
        if kk >= s.shape[-1]:
            return np.zeros(s.shape[:-1], dtype=bool)
        return srt[..., max(kk - 2, 0)] - srt[..., kk - 1] <= eps

    def ascending(s, kk, eps):
        srt = np.sort(s, axis=-1)
        if kk >= s.shape[-1]:
            return np.zeros(s.shape[:-1], dtype=bool)
        return np.abs(srt[..., kk - 1] - srt[..., kk]) <= eps

    for mutant in (strict, off_by_one, ascending):
        assert not pin_near_tie_rows(mutant), mutant.__name__


# ---------------------------------------------------------------------------
# entmax (the reference's training-study arm, src/agents/mappo.py:294-330)
# ---------------------------------------------------------------------------

def _sparsemax(s):
    """Closed-form sparsemax (alpha = 2 entmax) per row."""
    out = np.zeros_like(s)
    for idx in np.ndindex(s.shape[:-1]):
        row = s[idx]
        fin = np.isfinite(row)
        zs = np.sort(row[fin])[::-1]
        cs = np.cumsum(zs)
        ks = np.arange(1, len(zs) + 1)
        k = ks[1 + ks * zs > cs].max()
        tau = (cs[k - 1] - 1) / k
        out[idx] = np.where(fin, np.maximum(row - tau, 0.0), 0.0)
    return out


def _entmax15_brute(row):
    """Every support of a small row: the one whose weights are consistent."""
    fin = [j for j in range(len(row)) if np.isfinite(row[j])]
    z = row / 2.0
    for r in range(1, len(fin) + 1):
        for sup in itertools.combinations(fin, r):
            zs = z[list(sup)]
            m = zs.mean()
            disc = m * m - ((zs ** 2).sum() - 1.0) / r
            if disc < 0:
                continue
            tau = m - np.sqrt(disc)
            p = np.where(np.isfinite(z), np.maximum(z - tau, 0.0) ** 2, 0.0)
            if set(np.flatnonzero(p > 0)) == set(sup) and abs(p.sum() - 1) < 1e-9:
                return p
    raise AssertionError("no consistent support")


def pin_entmax(fn) -> bool:
    rng = np.random.default_rng(11)
    s = rng.standard_normal((3, 6, 6)) * 2.0
    for i in range(6):
        s[:, i, i] = -np.inf
    p = fn(s, 1.5)
    if not np.allclose(p.sum(-1), 1.0, atol=1e-9) or np.any(p[:, range(6), range(6)] != 0):
        return False
    if np.abs(p - O.entmax15_exact(s)).max() > 1e-6:
        return False
    return np.abs(fn(s, 2.0) - _sparsemax(s)).max() <= 1e-6


def test_entmax15_exact_matches_brute_force():
    rng = np.random.default_rng(5)
    s = rng.standard_normal((4, 5)) * 3.0
    s[0, 2] = -np.inf
    want = np.stack([_entmax15_brute(r) for r in s])
    assert np.abs(O.entmax15_exact(s) - want).max() <= 1e-12


def test_entmax_bisect_pinned():
    assert pin_entmax(O.entmax_bisect)


def test_entmax_pin_rejects_planted_mistakes():
    def wrong_power(s, alpha):          # squares the weights for every alpha
        z = np.where(np.isneginf(s), -np.inf, s * (alpha - 1.0))
        hi = z.max(-1, keepdims=True)
        lo = hi - 1.0
        for _ in range(24):
            mid = 0.5 * (lo + hi)
            above = (np.maximum(z - mid, 0.0) ** 2).sum(-1, keepdims=True) > 1.0
            lo, hi = np.where(above, mid, lo), np.where(above, hi, mid)
        p = np.maximum(z - 0.5 * (lo + hi), 0.0) ** 2
        return p / p.sum(-1, keepdims=True)

    def few_steps(s, alpha):            # 6 halvings instead of 24
        return O.entmax_bisect(s, alpha, iters=6)

    def softmax_instead(s, alpha):
        return O.softmax(s)

    for mutant in (wrong_power, few_steps, softmax_instead):
        assert not pin_entmax(mutant), mutant.__name__


def test_cpu_baseline_restatement_matches_oracle(golden):
    """The torch-CPU compositions bench.py times as the CPU baseline compute
    what the pinned numpy oracle computes (float64 inputs: 1e-12; Morton codes
    and window peers bit-exact on the golden positions)."""
    import cpu_reference as C
    q, k, v = qkv(31, 3, 40, 16, F64)
    t = [torch.from_numpy(x) for x in (q, k, v)]
    for kk in (1, 2, 7):
        got = C.topk_gather(*t, kk).numpy()
        assert np.abs(got - O.topk_gather(q, k, v, kk)[0]).max() < 1e-12
    assert np.abs(C.dense_unfused(*t).numpy() - O.dense_unfused(q, k, v)).max() < 1e-12
    for name in ("m64", "m512", "mgrid"):
        pos = golden[f"{name}_pos"]
        for bits in (10, 16):
            codes = C.morton_codes(torch.from_numpy(pos), bits).numpy()
            assert np.array_equal(codes, O.morton_code(pos, bits))
    pos = golden["m64_pos"]
    B, N = pos.shape[:2]
    q, k, v = qkv(32, B, N, 16, F64)
    for kk in (1, 2, 5):
        got = C.zorder(*(torch.from_numpy(x) for x in (q, k, v, pos)), kk, 16).numpy()
        want, _ = O.zorder_attention(q, k, v, pos, kk, 16)
        assert np.abs(got - want).max() < 1e-12
