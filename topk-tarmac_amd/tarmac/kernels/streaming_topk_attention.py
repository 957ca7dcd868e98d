"""Streaming exact top-k attention (HIP): keys pass through LDS in chunks, so
the N-wide score row is never resident and N is not capped.

Drop-in for ``src/kernels/streaming_topk_attention.py:206-258``. The retained
set is the first k under (score descending, index ascending), the reference's
rule (``:37-44``). Per chunk, every lane of a wavefront updates a register list
of its query's best k; the lists of the four lanes sharing a query are merged
once at the end, then the k value rows are gathered.
"""

from __future__ import annotations

import torch

from .fused_topk_attention import topk_attention

#: 0 = the largest chunk the LDS budget holds (the reference's ``tuned=True``
#: picks its key tile per shape, ``:191-203``)
DEFAULT_KEY_CHUNK = 0


def streaming_topk_attention(q: torch.Tensor, k: torch.Tensor,
                             v: torch.Tensor, topk: int,
                             block_m: int | None = None,
                             block_n: int | None = None,
                             num_warps: int | None = None,
                             num_stages: int | None = None,
                             tuned: bool = True,
                             bitonic: bool | None = None,
                             early_exit: bool | None = None,
                             precision: str = "ieee",
                             return_indices: bool = False):
    """Exact top-k attention with streamed keys. q, k, v: (B, N, d).

    With ``return_indices`` also returns the retained peer indices (B, N, k)
    int32, ordered by score (descending) then index. ``block_n`` is the number
    of keys staged per LDS pass (rounded up to 16; default: the largest chunk
    that fits LDS, e.g. 576 keys at d=16 fp32). ``block_m``,
    ``num_warps``, ``num_stages``, ``tuned``, ``bitonic`` and ``early_exit``
    select Triton tilings and merge schemes in the reference and are accepted
    for signature compatibility; the result does not depend on them there
    either.
    """
    B, N, d = q.shape
    assert k.shape == v.shape == q.shape
    topk = max(1, min(topk, N - 1))
    assert topk <= 8, "register candidate buffer is sized for small k"
    if precision != "ieee":
        raise ValueError(f"precision={precision!r}: gfx950 has no TF32 mode; use 'ieee'")
    chunk = DEFAULT_KEY_CHUNK if block_n is None else -(-int(block_n) // 16) * 16
    chunk = chunk if chunk > 0 else 0
    return topk_attention(q, k, v, topk, return_indices=return_indices, key_chunk=chunk)
