"""Fused score-then-select top-k attention (HIP).

Drop-in for ``src/kernels/fused_topk_attention.py``: every candidate is scored
(MFMA), the k best are selected in registers (ties keep the lower agent
index), softmaxed, and the k value rows gathered -- in one launch, with no
score row, index tensor or gathered tensor written to HBM.

* ``fused_topk_attention`` / ``fused_topk_attention_tiled``
  (``fused_topk_attention.py:296-355``): both are this kernel; the reference's
  two differ only in Triton tiling.
* ``fused_topk_attention_masked`` (``:127-208,358-387``): the
  threshold-bisection kernel, emulated step for step on the integer score
  keys. Its retained set is "every peer at or above the threshold", which
  equals exact top-k except on an exact tie at the k-th score, where it keeps
  every tied peer (or a superset when ``bisect`` < 32).
* ``fused_topk_attention_sort`` (``:405-540``): sort-based selection whose
  tie rule keeps the higher index.
* ``reference_topk_attention`` (``:390-402``): the composed PyTorch gather
  path, kept as the baseline it is in the reference.
"""

from __future__ import annotations

import math

import torch

from .. import _launch, _lib


def _check_precision(precision: str) -> None:
    if precision != "ieee":
        raise ValueError(f"precision={precision!r}: gfx950 has no TF32 mode; use 'ieee'")


@_launch.half_on_f32
def topk_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, topk: int,
                   return_indices: bool = False, key_chunk: int | None = None):
    """Exact top-k attention. ``topk`` is clamped to [1, N-1]. With
    ``return_indices`` also returns int32 [B, N, k] (score desc, index asc for
    k <= 8; ascending index above). ``key_chunk`` selects the streamed kernel
    with that many keys per LDS pass; ``None`` keeps the key row resident."""
    q, k, v = _launch.core(q, k, v)
    B, N, d = q.shape
    kk = max(1, min(int(topk), N - 1))
    out = torch.empty_like(q)
    idx = torch.empty(B, N, kk, device=q.device, dtype=torch.int32) if return_indices else None
    if B == 0:  # an empty batch: nothing to launch
        return (out, idx) if return_indices else out
    with torch.cuda.device(q.device):
        if key_chunk is None:
            rc = _lib.LIB.tarmac_topk_fused_fwd(
                _launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(out),
                _launch.ptr(idx), B, N, d, kk, _launch.dtype_code(q), _launch.stream(q))
        else:
            rc = _lib.LIB.tarmac_topk_stream_fwd(
                _launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(out),
                _launch.ptr(idx), B, N, d, kk, _launch.dtype_code(q), int(key_chunk),
                _launch.stream(q))
        _lib.check(rc)
    return (out, idx) if return_indices else out


def fused_topk_attention_tiled(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, topk: int,
                               block_m: int | None = None,
                               block_dc: int | None = None,
                               num_warps: int = 4,
                               num_stages: int | None = None,
                               precision: str = "ieee") -> torch.Tensor:
    """Tiled fused top-k attention (the reference's ``topk_fused_gather``).

    ``block_m``, ``block_dc``, ``num_warps`` and ``num_stages`` are Triton
    tiling knobs, accepted for signature compatibility; the HIP kernel fixes
    16 queries per wavefront and stages the whole key row in LDS.
    """
    B, N, d = q.shape
    assert N <= 1024
    _check_precision(precision)
    return topk_attention(q, k, v, topk)


def fused_topk_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         topk: int) -> torch.Tensor:
    """Fused score-then-select top-k attention. q, k, v: (B, N, d)."""
    B, N, d = q.shape
    assert k.shape == v.shape == q.shape
    assert N <= 1024, "single-block variant; N > 1024 needs a two-pass kernel"
    return topk_attention(q, k, v, topk)


@_launch.half_on_f32
def topk_variant_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, topk: int,
                           variant: int, bisect: int = 34,
                           return_indices: bool = False):
    """The reference's other two resident selection rules (one HIP launch):
    ``_lib.VARIANT_MASKED`` (threshold bisection) or ``_lib.VARIANT_SORT``
    (ties keep the higher index). ``topk`` is clamped to [1, N-1].

    bf16 heads whose rule the fp32 register-list kernel serves (sort, or
    masked with ``bisect`` >= 32; k <= 8; N <= 1024) run it on fp32 copies:
    bf16 values widen exactly, so the kept sets are the rules' sets on the
    canonical fp32 scores of the inputs, as the bf16 kernels define them, and
    the output is the fp32 result rounded once to bf16."""
    B, N = q.shape[0], q.shape[1]
    kk = max(1, min(int(topk), N - 1))
    if (q.dtype == torch.bfloat16 and k.dtype == v.dtype == torch.bfloat16 and kk <= 8
            and N <= 1024 and (variant == _lib.VARIANT_SORT or int(bisect) >= 32)):
        res = topk_variant_attention(q.float(), k.float(), v.float(), topk, variant, bisect,
                                     return_indices)
        if return_indices:
            return res[0].to(torch.bfloat16), res[1]
        return res.to(torch.bfloat16)
    q, k, v = _launch.core(q, k, v)
    B, N, d = q.shape
    out = torch.empty_like(q)
    idx = torch.empty(B, N, kk, device=q.device, dtype=torch.int32) if return_indices else None
    if B == 0:
        return (out, idx) if return_indices else out
    with torch.cuda.device(q.device):
        rc = _lib.LIB.tarmac_topk_variant_fwd(
            _launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(out), _launch.ptr(idx),
            B, N, d, kk, int(variant), int(bisect), _launch.dtype_code(q), _launch.stream(q))
        _lib.check(rc)
    return (out, idx) if return_indices else out


def fused_topk_attention_masked(q: torch.Tensor, k: torch.Tensor,
                                v: torch.Tensor, topk: int,
                                bisect: int = 34) -> torch.Tensor:
    """Threshold top-k: every peer whose score key is at or above the
    threshold left by ``bisect`` halvings of the integer bisection -- exact
    top-k plus every peer tied at the k-th score once ``bisect`` >= 32, a
    superset for fewer halvings, as the reference's kernel computes it."""
    B, N, d = q.shape
    assert N <= 1024
    return topk_variant_attention(q, k, v, topk, _lib.VARIANT_MASKED, bisect)


def fused_topk_attention_sort(q: torch.Tensor, k: torch.Tensor,
                              v: torch.Tensor, topk: int,
                              block_m: int | None = None) -> torch.Tensor:
    """Sort-based selection; an exact tie at the k-th score keeps the higher
    index, as the reference's descending sort of (key << 32 | index) does.
    ``block_m`` is a Triton tiling knob, accepted for signature compatibility."""
    B, N, d = q.shape
    assert N <= 1024
    return topk_variant_attention(q, k, v, topk, _lib.VARIANT_SORT)


def reference_topk_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                             topk: int) -> torch.Tensor:
    """The composed PyTorch score-then-select path the reference times as its
    baseline (``fused_topk_attention.py:390-402``): all N x N scores, the
    self pair masked, ``topk`` (unsorted), softmax over the kept scores, and
    the kept value rows gathered and contracted. Each query's kept rows are
    read through flat row numbers ``b * N + j`` of ``v`` viewed as
    ``[B * N, d]``. Not a fallback: the fused entry points above never call it."""
    n_batch, n_agents, dim = q.shape
    keep = max(1, min(int(topk), n_agents - 1))
    logits = torch.bmm(q, k.transpose(1, 2).contiguous()) / math.sqrt(dim)
    logits.diagonal(dim1=1, dim2=2).fill_(float("-inf"))
    kept, which = torch.topk(logits, keep, dim=2, sorted=False)
    weights = torch.softmax(kept, dim=2)
    base = torch.arange(n_batch, device=q.device).view(n_batch, 1, 1) * n_agents
    rows = v.reshape(n_batch * n_agents, dim)[which + base]   # [B, N, keep, d]
    return (weights.unsqueeze(3) * rows).sum(dim=2)
