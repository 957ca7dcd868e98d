"""Dense attention with the self-diagonal masked, as one HIP kernel.

Drop-in for ``src/kernels/fused_dense_attention.py:106-152``
(``fused_dense_attention``). The kernel is flash-style (online softmax over key
blocks staged in LDS, MFMA for both contractions), so no score matrix reaches
HBM. It is also the function of the composed dense paths
``scripts/bench_attention_core.py:74-82`` and ``src/agents/mappo.py:174-190``.
"""

from __future__ import annotations

import torch

from .. import _launch, _lib


@_launch.half_on_f32
def fused_dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          block_m: int | None = None,
                          block_kn: int | None = None,
                          num_warps: int | None = None,
                          num_stages: int | None = None,
                          precision: str = "ieee") -> torch.Tensor:
    """Streaming dense self-attention with the diagonal masked. q, k, v: [B, N, d].

    ``precision="ieee"`` is the only fp32 mode: CDNA4's fp32 MFMA is full
    fp32, and gfx950 has no TF32 path. ``block_kn`` sets the keys staged per
    LDS pass (rounded up to 16); ``block_m``, ``num_warps`` and ``num_stages``
    are Triton tiling knobs of the reference and are accepted for signature
    compatibility only.
    """
    if precision != "ieee":
        raise ValueError(f"precision={precision!r}: gfx950 has no TF32 mode; use 'ieee'")
    q, k, v = _launch.core(q, k, v)
    B, N, d = q.shape
    out = torch.empty_like(q)
    chunk = 0 if block_kn is None else -(-int(block_kn) // 16) * 16
    if B == 0:  # an empty batch: nothing to launch
        return out
    with torch.cuda.device(q.device):
        _lib.check(_lib.LIB.tarmac_dense_fwd(
            _launch.ptr(q), _launch.ptr(k), _launch.ptr(v), _launch.ptr(out),
            B, N, d, _launch.dtype_code(q), chunk, _launch.stream(q)))
    return out
