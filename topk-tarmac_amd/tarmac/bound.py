"""Pre-bound launches: arguments, outputs and stream resolved once, so each
call is a single C-ABI call with no allocation and no Python tensor checks.

Meant for serving loops and timed regions, where the per-call wrapper cost
(shape checks, ``torch.empty_like``, stream lookup) would otherwise be
comparable to a kernel of a few microseconds. Outputs are overwritten on every
call; the stream is the one current when the call was bound.
"""

from __future__ import annotations

import torch

from . import _launch, _lib


class Bound:
    """A libtarmac entry point with its arguments fixed."""

    def __init__(self, fn, args, out, idx=None, keep=()):
        self._fn = fn
        self._args = args
        self.out = out
        self.idx = idx
        self._keep = keep  # tensors whose memory the bound pointers refer to

    def __call__(self) -> torch.Tensor:
        rc = self._fn(*self._args)
        if rc:
            _lib.check(rc)
        return self.out


def topk(q, k, v, topk: int, key_chunk: int | None = None, with_idx: bool = False) -> Bound:
    q, k, v = _launch.core(q, k, v)
    B, N, d = q.shape
    kk = max(1, min(int(topk), N - 1))
    out = torch.empty_like(q)
    idx = torch.empty(B, N, kk, device=q.device, dtype=torch.int32) if with_idx else None
    st = _launch.stream(q)
    if key_chunk is None:
        fn = _lib.LIB.tarmac_topk_fused_fwd
        args = (_launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(out),
                _launch.ptr(idx), B, N, d, kk, _launch.dtype_code(q), st)
    else:
        fn = _lib.LIB.tarmac_topk_stream_fwd
        args = (_launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(out),
                _launch.ptr(idx), B, N, d, kk, _launch.dtype_code(q), int(key_chunk), st)
    return Bound(fn, args, out, idx, keep=(q, k, v))


def dense(q, k, v, key_chunk: int = 0) -> Bound:
    q, k, v = _launch.core(q, k, v)
    B, N, d = q.shape
    out = torch.empty_like(q)
    args = (_launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(out), B, N, d,
            _launch.dtype_code(q), int(key_chunk), _launch.stream(q))
    return Bound(_lib.LIB.tarmac_dense_fwd, args, out, keep=(q, k, v))


def fixedset(q, k, v, idx: torch.Tensor) -> Bound:
    q, k, v = _launch.core(q, k, v)
    B, N, d = q.shape
    code = _lib.IDX_I64 if idx.dtype == torch.int64 else _lib.IDX_I32
    idx = _launch.ready(idx if idx.dtype in (torch.int64, torch.int32) else idx.int(), 8)
    out = torch.empty_like(q)
    args = (_launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(idx), code,
            idx.shape[-1], _launch.ptr(out), B, N, d, _launch.dtype_code(q), _launch.stream(q))
    return Bound(_lib.LIB.tarmac_fixedset_fwd, args, out, keep=(q, k, v, idx))


def zorder(q, k, v, pos, topk: int, bits: int = 16, with_idx: bool = False) -> Bound:
    q, k, v = _launch.core(q, k, v)
    pos = _launch.ready(pos.float(), 8)
    B, N, d = q.shape
    out = torch.empty_like(q)
    idx = torch.empty(B, N, topk, device=q.device, dtype=torch.int32) if with_idx else None
    args = (_launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(pos), _launch.ptr(out),
            _launch.ptr(idx), B, N, d, int(topk), int(bits), _launch.dtype_code(q),
            _launch.stream(q))
    return Bound(_lib.LIB.tarmac_zorder_fwd, args, out, idx, keep=(q, k, v, pos))


def noop(device) -> Bound:
    t = torch.zeros(1, device=device)
    return Bound(_lib.LIB.tarmac_noop, (_launch.ptr(t), _launch.stream(t)), t, keep=(t,))
