"""Positional (select-before-scoring) peer selection and its attention (HIP).

Drop-in for the Z-order parts of ``src/kernels/prescore_selection.py``:

* ``select_morton_window`` (``:71-84``) and ``_morton_code`` (``:62-68``):
  one workgroup per batch row computes the codes, sorts (code, agent) in LDS
  and emits each agent's k curve neighbours. ``bits`` defaults to the
  reference's 10; equal codes are ordered by agent index (the reference's
  ``argsort`` leaves them unordered).
* ``prescore_attention`` (``:184-195``): attention over a given set -- the
  same function as ``fused_prescore_attention``.
* ``zorder_attention``: selector and attention in one launch (the
  "select+attend" total of ``scripts/bench_prescore.py:253-257``).

``select_radius_knn`` and ``select_grid_knn`` are outside this build.
"""

from __future__ import annotations

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
    with torch.cuda.device(pos.device):
        _lib.check(_lib.LIB.tarmac_morton_window(
            _launch.ptr(pos), _launch.ptr(idx), _lib.IDX_I64, _launch.ptr(None),
            B, N, int(k), int(bits), _launch.stream(pos)))
    return idx


def prescore_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       idx: torch.Tensor) -> torch.Tensor:
    """Score only the retained pairs. q,k,v: (B,N,d); idx: (B,N,kk)."""
    return fused_prescore_attention(q, k, v, idx)


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
    with torch.cuda.device(q.device):
        _lib.check(_lib.LIB.tarmac_zorder_fwd(
            _launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(pos), _launch.ptr(out),
            _launch.ptr(idx), B, N, d, int(topk), int(bits), _launch.dtype_code(q),
            _launch.stream(q)))
    return (out, idx) if return_indices else out


def prescore_full(q, k, v, pos, kk: int, selector: str) -> torch.Tensor:
    return prescore_attention(q, k, v, SELECTORS[selector](pos, kk))


SELECTORS = {"morton_window": select_morton_window}
