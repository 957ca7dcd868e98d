"""Attention over a pre-chosen peer set, fused (HIP).

Drop-in for ``src/kernels/fused_prescore_attention.py:88-114``: for each query,
the k named key and value rows are read straight from HBM/L2, scored, softmaxed
online and accumulated; no gathered tensor exists.
"""

from __future__ import annotations

import torch

from .. import _launch, _lib


@_launch.half_on_f32
def fused_prescore_attention(q: torch.Tensor, k: torch.Tensor,
                             v: torch.Tensor, idx: torch.Tensor,
                             block_m: int | None = None) -> torch.Tensor:
    """Attention over the peers named by ``idx``, with nothing intermediate
    written. q, k, v: (B, N, d); idx: (B, N, kk) int64 or int32. Query rows
    naming an out-of-range peer come out NaN (the index is never followed).
    ``block_m`` is a Triton knob, accepted for signature compatibility."""
    q, k, v = _launch.core(q, k, v)
    B, N, d = q.shape
    if idx.dim() != 3 or idx.shape[:2] != (B, N):
        raise ValueError(f"idx must be [B, N, kk] = [{B}, {N}, kk], got {tuple(idx.shape)}")
    _launch.on_gpu(idx)
    if idx.dtype == torch.int64:
        code = _lib.IDX_I64
    elif idx.dtype == torch.int32:
        code = _lib.IDX_I32
    else:
        idx, code = idx.to(torch.int32), _lib.IDX_I32
    idx = _launch.ready(idx, 8)
    out = torch.empty_like(q)
    if B == 0:  # an empty batch: nothing to launch
        return out
    with torch.cuda.device(q.device):
        _lib.check(_lib.LIB.tarmac_fixedset_fwd(
            _launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(idx), code,
            idx.shape[-1], _launch.ptr(out), B, N, d, _launch.dtype_code(q), _launch.stream(q)))
    return out
