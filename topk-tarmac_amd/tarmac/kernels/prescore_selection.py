"""Positional (select-before-scoring) peer selection and its attention (HIP).

Drop-in for ``src/kernels/prescore_selection.py``:

* ``select_radius_knn`` (``:35-42``): the k nearest peers over all pairs,
  squared fp32 distances, ties by agent index; emitted in ascending agent
  index (the reference's ``topk(sorted=False)`` leaves the order open).
* ``grid_knn_shape`` (``:87-101``) and ``select_grid_knn`` (``:107-164``):
  the k nearest among the 3x3 cells around each agent, with the reference's
  capacity cut and its all-pairs route when the block would hold N or more;
  agents with equal cells are ordered by index (the reference's ``argsort``
  is not stable); emitted in slot order.
* ``grid_knn_recall`` (``:167-172``).

* ``select_morton_window`` (``:71-84``) and ``_morton_code`` (``:62-68``):
  one workgroup per batch row computes the codes, sorts (code, agent) in LDS
  and emits each agent's k curve neighbours. ``bits`` defaults to the
  reference's 10; equal codes are ordered by agent index (the reference's
  ``argsort`` leaves them unordered).
* ``prescore_attention`` (``:184-195``): attention over a given set -- the
  same function as ``fused_prescore_attention``.
* ``zorder_attention``: selector and attention in one launch (the
  "select+attend" total of ``scripts/bench_prescore.py:253-257``).
"""

from __future__ import annotations

import ctypes

import torch

from .. import _launch, _lib
from .fused_prescore_attention import fused_prescore_attention


def _pos(pos: torch.Tensor) -> torch.Tensor:
    if pos.dim() != 3 or pos.shape[-1] != 2:
        raise ValueError(f"pos must be [B, N, 2], got {tuple(pos.shape)}")
    _launch.on_gpu(pos)
    return _launch.ready(pos.float(), 8)


def _morton_code(pos: torch.Tensor, bits: int = 10) -> torch.Tensor:
    """Interleave the bits of quantised 2-D coordinates. pos: (B, N, 2) -> int64 (B, N)."""
    pos = _pos(pos)
    B, N, _ = pos.shape
    codes = torch.empty(B, N, device=pos.device, dtype=torch.int64)
    if B == 0:  # an empty batch: nothing to launch
        return codes
    with torch.cuda.device(pos.device):
        _lib.check(_lib.LIB.tarmac_morton_window(
            _launch.ptr(pos), _launch.ptr(None), _lib.IDX_I64, _launch.ptr(codes),
            B, N, 1, int(bits), _launch.stream(pos)))
    return codes


def select_morton_window(pos: torch.Tensor, k: int, bits: int = 10) -> torch.Tensor:
    """k peers adjacent along a Z-order curve. (B, N, 2) -> int64 (B, N, k)."""
    pos = _pos(pos)
    B, N, _ = pos.shape
    idx = torch.empty(B, N, k, device=pos.device, dtype=torch.int64)
    if B == 0:
        return idx
    with torch.cuda.device(pos.device):
        _lib.check(_lib.LIB.tarmac_morton_window(
            _launch.ptr(pos), _launch.ptr(idx), _lib.IDX_I64, _launch.ptr(None),
            B, N, int(k), int(bits), _launch.stream(pos)))
    return idx


def _knn(fn, pos: torch.Tensor, k: int) -> torch.Tensor:
    pos = _pos(pos)
    B, N, _ = pos.shape
    idx = torch.empty(B, N, int(k), device=pos.device, dtype=torch.int64)
    if B == 0:
        return idx
    with torch.cuda.device(pos.device):
        _lib.check(fn(_launch.ptr(pos), _launch.ptr(idx), _lib.IDX_I64, B, N, int(k),
                      _launch.stream(pos)))
    return idx


def select_radius_knn(pos: torch.Tensor, k: int) -> torch.Tensor:
    """k spatially nearest peers per agent. pos: (B, N, 2) -> (B, N, k) int64."""
    return _knn(_lib.LIB.tarmac_knn_radius, pos, k)


def grid_knn_shape(N: int, k: int) -> tuple[int, int]:
    """Grid side G and per-cell capacity M for select_grid_knn (the library's
    own computation, the one its grid kernel uses)."""
    G, M = ctypes.c_int(), ctypes.c_int()
    _lib.check(_lib.LIB.tarmac_grid_knn_shape(int(N), int(k), ctypes.byref(G), ctypes.byref(M)))
    return G.value, M.value


def select_grid_knn(pos: torch.Tensor, k: int) -> torch.Tensor:
    """k nearest peers among the 3x3 grid cells around each agent.
    (B, N, 2) -> (B, N, k) int64."""
    return _knn(_lib.LIB.tarmac_knn_grid, pos, k)


def grid_knn_recall(pos: torch.Tensor, k: int) -> float:
    """Fraction of retained peers that exact kNN would also retain."""
    got = select_grid_knn(pos, k)
    ref = select_radius_knn(pos, k)
    hit = (got.unsqueeze(-1) == ref.unsqueeze(-2)).any(-1)
    return hit.float().mean().item()


def prescore_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       idx: torch.Tensor) -> torch.Tensor:
    """Score only the retained pairs. q,k,v: (B,N,d); idx: (B,N,kk)."""
    return fused_prescore_attention(q, k, v, idx)


@_launch.half_on_f32
def zorder_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor,
                     topk: int, bits: int = 10, return_indices: bool = False):
    """``prescore_attention(q, k, v, select_morton_window(pos, topk, bits))`` in
    one launch. Optionally returns the int32 peer indices."""
    q, k, v = _launch.core(q, k, v)
    pos = _pos(pos)
    B, N, d = q.shape
    if pos.shape[:2] != (B, N):
        raise ValueError("pos must be [B, N, 2] matching q")
    out = torch.empty_like(q)
    idx = torch.empty(B, N, topk, device=q.device, dtype=torch.int32) if return_indices else None
    if B == 0:
        return (out, idx) if return_indices else out
    with torch.cuda.device(q.device):
        _lib.check(_lib.LIB.tarmac_zorder_fwd(
            _launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(pos), _launch.ptr(out),
            _launch.ptr(idx), B, N, d, int(topk), int(bits), _launch.dtype_code(q),
            _launch.stream(q)))
    return (out, idx) if return_indices else out


def prescore_full(q, k, v, pos, kk: int, selector: str) -> torch.Tensor:
    return prescore_attention(q, k, v, SELECTORS[selector](pos, kk))


SELECTORS = {"radius_knn": select_radius_knn,
             "grid_knn": select_grid_knn,
             "morton_window": select_morton_window}
