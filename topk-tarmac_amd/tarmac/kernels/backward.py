"""Backward passes of the attention core (HIP, fp32 arithmetic).

The reference's Triton kernels are forward-only
(``scripts/bench_attention_core.py:172-176``); in training it differentiates
its PyTorch composition with autograd (``src/agents/mappo.py:192-231`` gather
path, ``:361-372`` dense path). These wrappers compute the same gradients on
the GPU:

* ``fixedset_attention_backward`` -- attention over a given peer set: the
  top-k core with the set its forward retained (gradients flow only through
  the retained scores and value rows, as for ``torch.topk``'s gather), the
  Z-order core with its selector's set, and prescore attention.
* ``dense_attention_backward`` -- the dense core (self pair excluded).

bf16 and float16 heads are differentiated in fp32: every operand is copied to
fp32 (exactly: bf16 and float16 values are fp32 values), the fp32 kernels run,
and the gradients come back rounded once to the heads' dtype -- the gradient
of the attention function at the given inputs, with fp32 accumulation, where
autograd through the reference's half-precision composition would round its
intermediates as well.
"""

from __future__ import annotations

import functools

import torch

from .. import _launch, _lib


def _f32(*ts):
    for t in ts:
        if t.dtype != torch.float32:
            raise TypeError(f"q, out and dout must share the heads' dtype, got {t.dtype}")


def _grads_on_f32(fn):
    """Run a backward ``fn(q, k, v, ...) -> (dq, dk, dv)`` for bf16 / float16
    heads on fp32 copies of its floating-point operands; gradients are
    returned in the heads' dtype."""

    @functools.wraps(fn)
    def wrapper(q, k, v, *args, **kwargs):
        dt = q.dtype
        if dt == torch.float32:
            return fn(q, k, v, *args, **kwargs)
        if dt not in (torch.bfloat16, torch.float16):
            raise TypeError(f"the backward takes float32, bfloat16 or float16 heads, got {dt}")

        def up(t):
            if isinstance(t, torch.Tensor) and t.is_floating_point() and t.dtype == dt:
                return t.float()
            return t

        grads = fn(up(q), up(k), up(v), *map(up, args), **{n: up(a) for n, a in kwargs.items()})
        return tuple(g.to(dt) for g in grads)

    return wrapper


@_grads_on_f32
def fixedset_attention_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                idx: torch.Tensor, dout: torch.Tensor):
    """Gradients (dq, dk, dv) of ``softmax(q k_S^T / sqrt(d)) v_S`` over the
    peer sets ``idx`` ([B, N, kk], int32 or int64)."""
    q, k, v = _launch.core(q, k, v)
    _f32(q, dout)
    dout = dout.contiguous()
    if dout.shape != q.shape:
        raise ValueError(f"dout shape {tuple(dout.shape)} != {tuple(q.shape)}")
    idx = idx.contiguous()
    B, N, d = q.shape
    if idx.dim() != 3 or idx.shape[:2] != (B, N):
        raise ValueError(f"idx must be [B, N, kk], got {tuple(idx.shape)}")
    if idx.dtype not in (torch.int32, torch.int64):
        raise ValueError("idx must be int32 or int64")
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    if B == 0:  # an empty batch: nothing to launch
        return dq, dk, dv
    with torch.cuda.device(q.device):
        rc = _lib.LIB.tarmac_fixedset_bwd(
            _launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(dout), _launch.ptr(idx),
            _lib.IDX_I64 if idx.dtype == torch.int64 else _lib.IDX_I32, idx.shape[-1],
            _launch.ptr(dq), _launch.ptr(dk), _launch.ptr(dv), B, N, d, _launch.stream(q))
        _lib.check(rc)
    return dq, dk, dv


def dense_attention_forward_stats(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """Dense attention (fp32) that also returns the per-query statistics its
    backward needs: ``(out, stats)``, stats ``[B, 2, N]`` with plane 0 the
    log2-domain logsumexp of the scaled scores."""
    q, k, v = _launch.core(q, k, v)
    if q.dtype != torch.float32:
        raise NotImplementedError(
            "dense_attention_forward_stats takes fp32 heads; a bf16 / float16 forward is "
            "fused_dense_attention, and dense_attention_backward without stats recomputes them")
    B, N, d = q.shape
    out = torch.empty_like(q)
    stats = torch.empty(B, 2, N, device=q.device, dtype=torch.float32)
    if B == 0:
        return out, stats
    with torch.cuda.device(q.device):
        _lib.check(_lib.LIB.tarmac_dense_fwd_stats(
            _launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(out), _launch.ptr(stats),
            B, N, d, _launch.stream(q)))
    return out, stats


@_grads_on_f32
def dense_attention_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                             out: torch.Tensor, dout: torch.Tensor,
                             stats: torch.Tensor | None = None):
    """Gradients (dq, dk, dv) of dense attention with the self pair excluded,
    given its forward output ``out`` (and, optionally, the ``stats`` returned
    with it by :func:`dense_attention_forward_stats`, which saves recomputing
    the logsumexp)."""
    q, k, v = _launch.core(q, k, v)
    _f32(q, out, dout)
    out, dout = out.contiguous(), dout.contiguous()
    if out.shape != q.shape or dout.shape != q.shape:
        raise ValueError("out and dout must match q's shape")
    B, N, d = q.shape
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ready = stats is not None
    if ready:
        if stats.shape != (B, 2, N) or stats.dtype != torch.float32 or not stats.is_contiguous():
            raise ValueError("stats must be the contiguous fp32 [B, 2, N] tensor of the forward")
    else:
        stats = torch.empty(B, 2, N, device=q.device, dtype=torch.float32)
    if B == 0:
        return dq, dk, dv
    with torch.cuda.device(q.device):
        rc = _lib.LIB.tarmac_dense_bwd(
            _launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(out), _launch.ptr(dout),
            _launch.ptr(dq), _launch.ptr(dk), _launch.ptr(dv), _launch.ptr(stats), int(ready),
            B, N, d, _launch.stream(q))
        _lib.check(rc)
    return dq, dk, dv
