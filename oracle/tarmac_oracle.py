"""CPU oracle for the TarMAC attention core -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The product path (``topk-tarmac_amd/tarmac``) never imports it and
fails loudly when its HIP library is missing.

Two layers:

* ``numpy`` restatements (float64 by default) of the reference's PyTorch
  compositions, one function per reference symbol, each citing the reference
  file:line it follows.  Paths are relative to the reference checkout.
* ``canon_*`` wrappers around ``tarmac_oracle.c`` (built into
  ``oracle/_build/libtarmac_oracle.so``): the fp32 score computed in the exact
  rounding order the HIP kernels use, so that retained index sets can be
  compared bit for bit.

Pinning (what checks each function against something other than itself):

==========================  ===================================================
function                    pinned by
==========================  ===================================================
scores                      torch.matmul (float64) and unit-vector closed form
dense_unfused               torch SDPA (float64, -inf diagonal mask); rows sum
                            to 1; constant-V and equal-key closed forms
topk_indices                torch.topk on tie-free rows; brute force over all
                            k-subsets on tiny rows; constructed ties
topk_gather                 masked formulation to 1e-10 (float64); k = N-1
                            equals dense; exactly k nonzero weights
topk_masked                 equals topk_gather on tie-free inputs (two
                            independent formulations)
morton_code                 bit-by-bit interleave loop; golden vectors written
                            by the reference's own ``_morton_code``
select_morton_window        golden vectors from the reference; k distinct
                            peers, never self; curve-neighbour sets
prescore_attention          dense softmax restricted to the selected set
pair_d2                     float64 distances: within one fp32 rounding chain
                            (3 ulp) of (c-p).(c-p); exact on integer grids
select_radius_knn           scipy cKDTree (float64 kNN, an independent
                            implementation) on rows without near-ties;
                            brute-force ties on integer lattices
grid_knn_shape              the reference's own values (golden vectors)
grid_cells                  through select_grid_knn's golden vectors
select_grid_knn             golden vectors from the reference on rows whose
                            runs were not cut and hold >= k candidates; equals
                            select_radius_knn where the k-th neighbour lies
                            inside the 3x3 block and no run was cut; the
                            all-pairs route when 9M >= N. Parity unpinned on
                            cut / short rows (the reference's unstable argsort
                            and topk tie order decide them)
ordered_key                 exhaustive order check on special values and
                            random fp32 pairs (a < b iff key(a) < key(b))
masked_threshold_keep       bisect >= 32: exactly {j : s_j >= k-th largest}
                            (closed form, ties included); bisect = 0 keeps
                            every valid peer; monotone in bisect
sort_select                 brute force: k largest by (score, index) desc
weights_attention           equals topk_gather when the kept set is the
                            top-k set
canon_topk (C)              numpy oracle: same sets off near-ties, outputs to
                            1e-6; brute force of the fmaf chain in Python
score_error_bound           exact-rational error of canonical scores (random,
                            cancellation-heavy and constructed worst-case
                            chains) stays within it; the constructed chain
                            reaches over 0.85 of it (tight, so a halved bound,
                            gamma_d or a dropped |.| or scale fails)
near_tie_rows               brute force on Python-sorted rows; exact gaps at
                            the eps boundary; k >= N-1 rows
entmax_bisect               entmax15_exact (closed form) to 1e-6 at alpha=1.5;
                            alpha -> 2 equals sparsemax's closed form; rows sum
                            to 1, the self pair gets 0
entmax15_exact              its own definition: weights sum to 1 and
                            (z_j - tau)_+^2 with one tau; brute force over all
                            supports on small rows
canon_morton_window (C)     numpy oracle bit-exact (codes and indices)
==========================  ===================================================
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent

# ---------------------------------------------------------------------------
# numpy restatements of the reference compositions
# ---------------------------------------------------------------------------


def scores(q: np.ndarray, k: np.ndarray) -> np.ndarray:
    """``S = Q K^T / sqrt(d)`` with the self-diagonal at -inf.

    Follows ``scripts/bench_attention_core.py:69-71`` and
    ``src/agents/mappo.py:210-211`` (division by sqrt(d), masked_fill of the
    identity). Computed in the dtype of ``q``.
    """
    d = q.shape[-1]
    s = np.matmul(q, np.swapaxes(k, -1, -2)) / q.dtype.type(np.sqrt(d))
    n = q.shape[1]
    s[:, np.arange(n), np.arange(n)] = -np.inf
    return s


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """Numerically stable softmax (``torch.softmax`` semantics on finite rows)."""
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=axis, keepdims=True)


def k_eff(topk: int, n: int) -> int:
    """``min(max(topk, 1), N - 1)`` -- ``src/agents/mappo.py:171-172``."""
    return min(max(int(topk), 1), n - 1)


def dense_unfused(q, k, v):
    """``softmax(S) V`` -- ``scripts/bench_attention_core.py:74-75``;
    ``src/agents/mappo.py:361-372,418``."""
    return np.matmul(softmax(scores(q, k)), v)


def topk_indices(s: np.ndarray, topk: int) -> np.ndarray:
    """Indices of the ``topk`` largest entries of each row, ordered by
    (score descending, index ascending).

    The reference calls ``Tensor.topk(sorted=False)`` (``mappo.py:217``),
    which documents no tie rule; this build fixes the rule of the reference's
    fused kernels, "ties keep the lower index"
    (``src/kernels/streaming_topk_attention.py:37-44``). A stable sort of the
    negated row gives exactly that order.
    """
    order = np.argsort(-s, axis=-1, kind="stable")
    return order[..., :topk]


def gather_rows(x: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """``x[b, idx[b, i, j], :]`` -> ``[B, N, k, d]`` (``Tensor.gather`` on dim 1)."""
    b = np.arange(x.shape[0])[:, None, None]
    return x[b, idx]


def topk_gather(q, k, v, topk):
    """Score-then-select top-k attention, gathered aggregation.

    ``src/agents/mappo.py:192-231``; ``scripts/bench_attention_core.py:94-101``;
    ``src/kernels/fused_topk_attention.py:390-402``.
    Returns ``(out[B,N,d], idx[B,N,k])``.
    """
    n = q.shape[1]
    kk = k_eff(topk, n)
    s = scores(q, k)
    idx = topk_indices(s, kk)
    w = softmax(np.take_along_axis(s, idx, axis=-1))
    out = np.einsum("bnk,bnkd->bnd", w, gather_rows(v, idx))
    return out, idx


def topk_masked(q, k, v, topk):
    """Dense softmax, a {0,1} top-k mask on the weights, renormalise, dense PV.

    ``scripts/bench_attention_core.py:85-91``; ``src/agents/mappo.py:374-382``.
    """
    n = q.shape[1]
    kk = k_eff(topk, n)
    w = softmax(scores(q, k))
    idx = topk_indices(w, kk)
    keep = np.zeros_like(w)
    np.put_along_axis(keep, idx, 1.0, axis=-1)
    w = w * keep
    w = w / np.maximum(w.sum(-1, keepdims=True), 1e-8)
    return np.matmul(w, v)


#: The standard shift-and-mask bit spread ("part 1 by 1"), the same table as
#: ``src/kernels/prescore_selection.py:51-52``.
_SPREAD = ((16, 0x0000FFFF), (8, 0x00FF00FF), (4, 0x0F0F0F0F),
           (2, 0x33333333), (1, 0x55555555))


def ordered_key(s: np.ndarray) -> np.ndarray:
    """Monotone fp32 -> int32 key ``i ^ ((i >> 31) & 0x7FFFFFFF)`` --
    ``src/kernels/fused_topk_attention.py:113-124``."""
    i = np.ascontiguousarray(s, np.float32).view(np.int32)
    return i ^ ((i >> 31) & np.int32(0x7FFFFFFF))


def masked_threshold_keep(s: np.ndarray, topk: int, bisect: int = 34) -> np.ndarray:
    """Kept-peer mask of the threshold-bisection kernel, step for step --
    ``src/kernels/fused_topk_attention.py:172-186``: int64 keys of the fp32
    scores ``s`` ([..., N, N], -inf on the self pair); ``lo`` starts at the
    smallest valid key, ``hi`` at the row maximum; ``bisect`` halvings keep
    "at least topk keys >= lo"; the kept peers are the keys >= lo."""
    keys = ordered_key(s).astype(np.int64)
    n = s.shape[-1]
    valid = ~np.eye(n, dtype=bool)
    big = np.int64(np.iinfo(np.int64).max)
    lo = np.where(valid, keys, big).min(-1)
    hi = keys.max(-1)
    for _ in range(bisect):
        mid = lo + (hi - lo + 1) // 2
        cnt = (keys >= mid[..., None]).sum(-1)
        take = cnt >= topk
        lo = np.where(take, mid, lo)
        hi = np.where(take, hi, mid - 1)
    return keys >= lo[..., None]


def sort_select(s: np.ndarray, topk: int) -> np.ndarray:
    """Indices kept by the sort kernel -- ``fused_topk_attention.py:470-480``:
    a descending sort of ``key << 32 | index``, the first ``topk`` entries
    (ties at equal score keep the higher index)."""
    n = s.shape[-1]
    packed = (ordered_key(s).astype(np.int64) << 32) | np.arange(n, dtype=np.int64)
    top = np.flip(np.sort(packed, -1), -1)[..., :topk]
    return top & np.int64(0xFFFFFFFF)


def weights_attention(s: np.ndarray, keep: np.ndarray, v: np.ndarray) -> np.ndarray:
    """Softmax of ``s`` over the kept peers, then ``sum_j w_j v_j`` --
    ``fused_topk_attention.py:188-208`` (masked) and ``:482-504`` (sort)."""
    s64 = np.where(keep, s.astype(np.float64), -np.inf)
    m = s64.max(-1, keepdims=True)
    w = np.where(keep, np.exp(s64 - m), 0.0)
    return np.matmul(w, v.astype(np.float64)) / w.sum(-1, keepdims=True)


def spread_bits(x: np.ndarray) -> np.ndarray:
    """Insert a zero bit between consecutive bits -- ``prescore_selection.py:55-59``."""
    x = x.astype(np.int64)
    for shift, mask in _SPREAD:
        x = (x | (x << shift)) & mask
    return x


def morton_code(pos: np.ndarray, bits: int = 10) -> np.ndarray:
    """Per-batch normalised, quantised, interleaved 2-D Morton code.

    ``src/kernels/prescore_selection.py:62-68``: fp32 ``amin/amax`` over the
    agents, ``span.clamp_min(1e-6)``, ``((pos - lo) / span * (2**bits - 1))``
    truncated to int64 and clamped, then x in the even bits and y in the odd.
    ``pos`` must be float32 (the arithmetic is the fp32 arithmetic torch does).
    """
    pos = np.asarray(pos, dtype=np.float32)
    lo = pos.min(axis=1, keepdims=True)
    hi = pos.max(axis=1, keepdims=True)
    span = np.maximum(hi - lo, np.float32(1e-6))
    top = (1 << bits) - 1
    g = ((pos - lo) / span * np.float32(top)).astype(np.int64)
    g = np.clip(g, 0, top)
    return spread_bits(g[..., 0]) | (spread_bits(g[..., 1]) << 1)


def morton_order(code: np.ndarray) -> np.ndarray:
    """Agents in curve order, equal codes by agent index (stable sort).

    The reference's ``argsort`` (``prescore_selection.py:75``) is not stable;
    this build pins equal codes to ascending agent index.
    """
    return np.argsort(code, axis=-1, kind="stable")


def window_offsets(k: int) -> np.ndarray:
    """``+1..+ceil(k/2)`` then ``-1..-floor(k/2)`` -- ``prescore_selection.py:80-82``."""
    half = (k + 1) // 2
    return np.array(list(range(1, half + 1)) + [-o for o in range(1, k - half + 1)],
                    dtype=np.int64)


def select_morton_window(pos: np.ndarray, k: int, bits: int = 10) -> np.ndarray:
    """k peers adjacent along the Z-order curve, wrapping at the ends.

    ``src/kernels/prescore_selection.py:71-84`` (``bits`` is fixed to 10 there;
    it is a parameter here so the 16-bit configuration can be checked).
    Returns int64 ``[B, N, k]`` in offset order.
    """
    B, N, _ = pos.shape
    order = morton_order(morton_code(pos, bits))
    rank = np.empty_like(order)
    np.put_along_axis(rank, order, np.broadcast_to(np.arange(N), (B, N)), axis=-1)
    nr = (rank[..., None] + window_offsets(k)[None, None, :]) % N
    return np.take_along_axis(order, nr.reshape(B, N * k), axis=1).reshape(B, N, k)


def pair_d2(pos: np.ndarray, cand_pos: np.ndarray) -> np.ndarray:
    """Squared distance in fp32, ``(c - p)^2`` summed x then y.

    The arithmetic of ``(pc - pos.unsqueeze(2)).square().sum(-1)`` in
    ``src/kernels/prescore_selection.py:155-156``: each difference, each square
    and the one addition rounded to fp32 (no fused multiply-add).
    ``pos`` [..., 2] broadcasts against ``cand_pos`` [..., 2].
    """
    diff = (np.asarray(cand_pos, np.float32) - np.asarray(pos, np.float32)).astype(np.float32)
    sq = (diff * diff).astype(np.float32)
    return (sq[..., 0] + sq[..., 1]).astype(np.float32)


def select_radius_knn(pos: np.ndarray, k: int) -> np.ndarray:
    """k nearest peers per agent -- ``src/kernels/prescore_selection.py:35-42``.

    All-pairs squared distances (:func:`pair_d2`), the self pair at +inf (the
    reference's ``masked_fill`` of the identity), then the k smallest by
    (distance, agent index). The reference ranks ``torch.cdist`` distances,
    which for N > 25 come from ``|x|^2 + |y|^2 - 2 x.y``; that rounding is not
    restated (it only moves near-ties), and ``topk(sorted=False)`` leaves the
    order of the k open: here the k are returned nearest first.
    Returns int64 ``[B, N, k]``.
    """
    pos = np.asarray(pos, np.float32)
    B, N, _ = pos.shape
    d2 = pair_d2(pos[:, :, None, :], pos[:, None, :, :])
    d2[:, np.arange(N), np.arange(N)] = np.inf
    return np.argsort(d2, axis=-1, kind="stable")[..., :k].astype(np.int64)


def grid_knn_shape(N: int, k: int) -> tuple[int, int]:
    """Grid side G and cell capacity M -- ``src/kernels/prescore_selection.py:87-101``:
    about ``max(2, k)`` agents per cell, capacity mean + 3 sqrt(mean) + 2."""
    occ = max(2, k)
    G = max(1, int((N / occ) ** 0.5))
    mean = N / (G * G)
    return G, int(mean + 3 * mean ** 0.5 + 2)


def grid_cells(pos: np.ndarray, G: int) -> np.ndarray:
    """Cell coordinates ``[B, N, 2]`` -- ``prescore_selection.py:134-136``:
    per-batch fp32 normalisation, ``* G``, truncation, clamp to ``[0, G-1]``."""
    pos = np.asarray(pos, np.float32)
    lo = pos.min(axis=1, keepdims=True)
    span = np.maximum(pos.max(axis=1, keepdims=True) - lo, np.float32(1e-6))
    c = ((pos - lo) / span * np.float32(G)).astype(np.int64)
    return np.clip(c, 0, G - 1)


def select_grid_knn(pos: np.ndarray, k: int, slot_order: bool = False) -> np.ndarray:
    """k nearest peers among the 3x3 cells around each agent --
    ``src/kernels/prescore_selection.py:107-164``.

    Agents sorted by cell ``x*G + y`` (equal cells by agent index: the
    reference's ``argsort`` is not stable); for each neighbour column
    ``x-1..x+1`` a run of at most ``L = 3M`` sorted agents from cell
    ``(x', max(y-1, 0))`` to the end of cell ``(x', min(y+1, G-1))``; slots
    past the run, of a column outside the grid, or holding the agent itself
    are at +inf. The k smallest slots by (distance, slot) are kept, so a
    query with fewer than k valid candidates keeps the first invalid slots,
    whose agents are what the reference's gather reads there. Falls back to
    :func:`select_radius_knn` when ``3L >= N`` (``:127-128``).
    Returns int64 ``[B, N, k]``, nearest first (in ascending slot with
    ``slot_order``; ascending agent index on the all-pairs route).
    """
    pos = np.asarray(pos, np.float32)
    B, N, _ = pos.shape
    G, M = grid_knn_shape(N, k)
    L = 3 * M
    if 3 * L >= N:
        out = select_radius_knn(pos, k)
        return np.sort(out, -1) if slot_order else out
    cxy = grid_cells(pos, G)
    cell = cxy[..., 0] * G + cxy[..., 1]
    order = np.argsort(cell, axis=1, kind="stable")
    start = np.zeros((B, G * G + 1), np.int64)
    for b in range(B):
        start[b, 1:] = np.cumsum(np.bincount(cell[b], minlength=G * G))
    x = cxy[..., 0][..., None] + np.arange(-1, 2)
    y = cxy[..., 1][..., None]
    ok_col = (x >= 0) & (x < G)
    xc = np.clip(x, 0, G - 1)
    c_lo = xc * G + np.maximum(y - 1, 0)
    c_hi = xc * G + np.minimum(y + 1, G - 1) + 1
    s_lo = np.take_along_axis(start, c_lo.reshape(B, -1), 1).reshape(B, N, 3)
    s_hi = np.take_along_axis(start, c_hi.reshape(B, -1), 1).reshape(B, N, 3)
    s_hi = np.minimum(s_hi, s_lo + L)
    idx = s_lo[..., None] + np.arange(L)
    valid = (idx < s_hi[..., None]) & ok_col[..., None]
    cand = np.take_along_axis(order, np.minimum(idx, N - 1).reshape(B, -1), 1).reshape(B, N, 3 * L)
    valid = valid.reshape(B, N, 3 * L) & (cand != np.arange(N)[None, :, None])
    pc = np.take_along_axis(pos, cand.reshape(B, -1, 1), 1).reshape(B, N, 3 * L, 2)
    d2 = pair_d2(pos[:, :, None, :], pc)
    d2 = np.where(valid, d2, np.float32(np.inf))
    j = np.argsort(d2, axis=-1, kind="stable")[..., :k]
    if slot_order:
        j = np.sort(j, -1)
    return np.take_along_axis(cand, j, -1).astype(np.int64)


def prescore_attention(q, k, v, idx):
    """Attention over a given peer set -- ``src/kernels/prescore_selection.py:184-195``
    (gather K and V rows, k scores divided by sqrt(d), softmax, contract); the
    same function as ``src/kernels/fused_prescore_attention.py:27-114``."""
    d = q.shape[-1]
    kg = gather_rows(k, idx)
    vg = gather_rows(v, idx)
    s = np.einsum("bnd,bnkd->bnk", q, kg) / q.dtype.type(np.sqrt(d))
    return np.einsum("bnk,bnkd->bnd", softmax(s), vg)


def zorder_attention(q, k, v, pos, topk, bits=10):
    """``prescore_attention(select_morton_window(pos, k))`` --
    ``src/agents/mappo.py:265-292``; ``scripts/bench_prescore.py:253-257``."""
    idx = select_morton_window(pos, topk, bits)
    return prescore_attention(q, k, v, idx), idx


def near_tie_rows(s: np.ndarray, topk: int, eps: np.ndarray | float) -> np.ndarray:
    """Rows whose k-th and (k+1)-th largest scores are within ``eps``.

    On these rows the retained set legitimately depends on the rounding of the
    scores (the reference attributes such rows in
    ``scripts/verify_all_configurations.py:160-213``)."""
    srt = -np.sort(-s, axis=-1)
    if topk >= s.shape[-1]:
        return np.zeros(s.shape[:-1], dtype=bool)
    gap = srt[..., topk - 1] - srt[..., topk]
    return gap <= eps


def entmax_bisect(s: np.ndarray, alpha: float, iters: int = 24) -> np.ndarray:
    """alpha-entmax weights over the last axis by threshold bisection, the
    reference's ``_forward_entmax`` (``src/agents/mappo.py:294-330``): z =
    (alpha - 1) s, tau bracketed in [max z - 1, max z] and halved ``iters``
    times on sum_j [z_j - tau]_+^(1/(alpha-1)) > 1, then the weights at the
    midpoint, renormalised. -inf scores (the self pair) get weight 0."""
    z = np.where(np.isneginf(s), -np.inf, s * (alpha - 1.0))
    power = 1.0 / (alpha - 1.0)
    hi = z.max(-1, keepdims=True)
    lo = hi - 1.0
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        above = (np.maximum(z - mid, 0.0) ** power).sum(-1, keepdims=True) > 1.0
        lo = np.where(above, mid, lo)
        hi = np.where(above, hi, mid)
    p = np.maximum(z - 0.5 * (lo + hi), 0.0) ** power
    return p / np.maximum(p.sum(-1, keepdims=True), 1e-8)


def entmax15_exact(s: np.ndarray) -> np.ndarray:
    """Exact 1.5-entmax over the last axis (sort-based closed form; Peters,
    Niculae and Martins, 2019): with z = s / 2 sorted descending, the support
    is the largest k whose threshold tau_k = mean_k - sqrt(mean_k^2 -
    (sumsq_k - 1) / k) stays at or below z_(k); weights [z - tau]_+^2."""
    z = np.where(np.isneginf(s), -np.inf, s / 2.0)
    out = np.zeros_like(z, dtype=np.float64)
    flat_z = z.reshape(-1, z.shape[-1])
    flat_o = out.reshape(-1, z.shape[-1])
    for r in range(flat_z.shape[0]):
        zs = np.sort(flat_z[r][np.isfinite(flat_z[r])])[::-1]
        tau = None
        for k in range(1, len(zs) + 1):
            m = zs[:k].mean()
            disc = m * m - ((zs[:k] ** 2).sum() - 1.0) / k
            t = m - np.sqrt(max(disc, 0.0))
            if t <= zs[k - 1]:
                tau = t
        flat_o[r] = np.maximum(flat_z[r] - tau, 0.0) ** 2
        flat_o[r][~np.isfinite(flat_z[r])] = 0.0
    return out


def score_error_bound(q, k) -> np.ndarray:
    """Twice the forward error bound of one canonical fp32 score, ``[B, N, N]``:
    ``2 * gamma_{d+2} * sum_c |q_c k_c| / sqrt(d)`` with
    ``gamma_m = m u / (1 - m u)``, ``u = 2^-24``. One score is the fmaf chain
    (d roundings, each at most u times the running partial, which is at most
    ``sum_c |q_c k_c|``) times fp32(1/sqrt(d)) (the constant's own rounding
    and the product's: two more). Twice that bounds how far two scores' order
    can move, so rows whose k-th and (k+1)-th scores are closer are the ones
    where the fp32 selection may legitimately differ from exact arithmetic."""
    d = q.shape[-1]
    u = 2.0 ** -24
    g = (d + 2) * u / (1 - (d + 2) * u)
    a = np.matmul(np.abs(q.astype(np.float64)), np.abs(np.swapaxes(k, -1, -2)).astype(np.float64))
    return 2 * g * a / np.sqrt(d)


# ---------------------------------------------------------------------------
# canonical-order C oracle (bit-exact twin of the HIP score rounding)
# ---------------------------------------------------------------------------

_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = _HERE / "_build" / "libtarmac_oracle.so"
        if not path.exists():
            build()
        _LIB = ctypes.CDLL(str(path))
        f = ctypes.c_void_p
        i = ctypes.c_int
        _LIB.or_canon_scores.argtypes = [f, f, i, i, i, f]
        _LIB.or_canon_topk.argtypes = [f, f, f, i, i, i, i, f, f]
        _LIB.or_morton_codes.argtypes = [f, i, i, i, f]
        _LIB.or_morton_window.argtypes = [f, i, i, i, i, f]
        _LIB.or_fixedset.argtypes = [f, f, f, f, i, i, i, i, f]
        _LIB.or_dense.argtypes = [f, f, f, i, i, i, f]
        for fn in (_LIB.or_canon_scores, _LIB.or_canon_topk, _LIB.or_morton_codes,
                   _LIB.or_morton_window, _LIB.or_fixedset, _LIB.or_dense):
            fn.restype = ctypes.c_int
    return _LIB


def build() -> None:
    """Compile ``tarmac_oracle.c`` with gcc (no contraction, explicit fmaf)."""
    import subprocess
    out = _HERE / "_build"
    out.mkdir(exist_ok=True)
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    assert (out / "libtarmac_oracle.so").exists()


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def canon_scores(q, k) -> np.ndarray:
    """fp32 scores in the HIP kernels' rounding order, ``[B, N, N]``, -inf diagonal."""
    q, k = _f32(q), _f32(k)
    B, N, d = q.shape
    s = np.empty((B, N, N), np.float32)
    rc = _lib().or_canon_scores(_ptr(q), _ptr(k), B, N, d, _ptr(s))
    assert rc == 0, rc
    return s


def canon_topk(q, k, v, topk):
    """Canonical fp32 selection + float64 aggregation. Returns (out f64, idx i32)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, N, d = q.shape
    kk = k_eff(topk, N)
    out = np.empty((B, N, d), np.float64)
    idx = np.empty((B, N, kk), np.int32)
    rc = _lib().or_canon_topk(_ptr(q), _ptr(k), _ptr(v), B, N, d, kk, _ptr(out), _ptr(idx))
    assert rc == 0, rc
    return out, idx


def canon_morton_codes(pos, bits) -> np.ndarray:
    pos = _f32(pos)
    B, N, _ = pos.shape
    codes = np.empty((B, N), np.int64)
    rc = _lib().or_morton_codes(_ptr(pos), B, N, bits, _ptr(codes))
    assert rc == 0, rc
    return codes


def canon_morton_window(pos, k, bits) -> np.ndarray:
    pos = _f32(pos)
    B, N, _ = pos.shape
    idx = np.empty((B, N, k), np.int64)
    rc = _lib().or_morton_window(_ptr(pos), B, N, k, bits, _ptr(idx))
    assert rc == 0, rc
    return idx


def canon_fixedset(q, k, v, idx):
    q, k, v = _f32(q), _f32(k), _f32(v)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    B, N, d = q.shape
    kk = idx.shape[-1]
    out = np.empty((B, N, d), np.float64)
    rc = _lib().or_fixedset(_ptr(q), _ptr(k), _ptr(v), _ptr(idx), kk, B, N, d, _ptr(out))
    assert rc == 0, rc
    return out


def canon_dense(q, k, v):
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, N, d = q.shape
    out = np.empty((B, N, d), np.float64)
    rc = _lib().or_dense(_ptr(q), _ptr(k), _ptr(v), B, N, d, _ptr(out))
    assert rc == 0, rc
    return out


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 (round to nearest even) -> float32, as ``Tensor.to(bf16)``."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


__all__ = [n for n in dir() if not n.startswith("_")]
del os
