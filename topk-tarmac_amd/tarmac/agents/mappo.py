"""``AttentionComm`` -- the TarMAC communication block, with its attention core
on the HIP kernels of :mod:`tarmac.kernels`.

Drop-in for ``src/agents/mappo.py:31-86`` (``MAPPOConfig``) and
``src/agents/mappo.py:138-420`` (``AttentionComm``): same constructor, same
parameters and initialisation, same ``forward(x, pos=None) -> (msg, info)``
contract, same errors. The qkv and output projections stay ``nn.Linear``
(hipBLASLt); the core between them -- the part the reference times -- is one
HIP launch per call:

=============  ==========================================================
attn_mode      core
=============  ==========================================================
dense          ``tarmac_dense_fwd``
dense_sdpa     ``tarmac_dense_fwd`` (the same function, ``mappo.py:174-190``)
topk           ``tarmac_topk_fused_fwd`` (masked top-k is the same function
               as the gathered one, ``mappo.py:374-382``)
topk_gather    ``tarmac_topk_fused_fwd``
zorder_k       ``tarmac_zorder_fwd`` (selector + attend in one launch)
=============  ==========================================================

The training-study arms ``random_k``, ``entmax`` and ``adaptive_topk`` are
not part of the timed core and are not provided here.

The reference's Triton kernels are forward-only
(``scripts/bench_attention_core.py:172-176``) and its training differentiates
the PyTorch composition; here the core's backward runs on HIP kernels too
(:mod:`tarmac.kernels.backward`, fp32): gradients reach q, k, v through the
retained set of the top-k and Z-order cores, and through every pair of the
dense core.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels.backward import (dense_attention_backward, dense_attention_forward_stats,
                                fixedset_attention_backward)
from ..kernels.fused_dense_attention import fused_dense_attention
from ..kernels.fused_topk_attention import topk_attention
from ..kernels.prescore_selection import zorder_attention

#: Morton bits per axis of the zorder_k selector (``select_morton_window``'s
#: default, ``src/kernels/prescore_selection.py:62``).
ZORDER_BITS = 10

HIP_MODES = ("dense", "dense_sdpa", "topk", "topk_gather", "zorder_k")
REFERENCE_ONLY_MODES = ("random_k", "entmax", "adaptive_topk")


@dataclass
class MAPPOConfig:
    """Field-for-field ``src/agents/mappo.py:31-86``."""
    obs_dim: int
    n_actions: int
    n_agents: int
    hidden: int = 64
    use_orthogonal_init: bool = True
    use_comm: bool = False
    msg_dim: int = 16
    n_heads: int = 1
    attn_mode: str = "dense"
    topk: int = 0
    entmax_alpha: float = 1.5


def _ortho_init(layer: nn.Linear, gain: float = np.sqrt(2.0)) -> None:
    nn.init.orthogonal_(layer.weight, gain=gain)
    nn.init.zeros_(layer.bias)


class _DenseCore(torch.autograd.Function):
    """Dense core with the HIP backward (fp32)."""

    @staticmethod
    def forward(ctx, q, k, v):
        if q.dtype == torch.float32:
            out, stats = dense_attention_forward_stats(q, k, v)
        else:  # the backward raises for bf16; nothing to keep
            out, stats = fused_dense_attention(q, k, v), None
        ctx.save_for_backward(q, k, v, out, stats)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, stats = ctx.saved_tensors
        return dense_attention_backward(q, k, v, out, dout, stats)


class _SetCore(torch.autograd.Function):
    """A core that attends over a peer set it chooses itself (top-k,
    Z-order); the HIP backward treats that set as fixed, as autograd through
    ``torch.topk``'s gather does. ``fn`` returns (out, idx)."""

    @staticmethod
    def forward(ctx, fn, q, k, v, *extra):
        out, idx = fn(q, k, v, *extra)
        ctx.mark_non_differentiable(idx)
        ctx.save_for_backward(q, k, v, idx)
        ctx.n_extra = len(extra)
        return out, idx

    @staticmethod
    def backward(ctx, dout, _didx):
        q, k, v, idx = ctx.saved_tensors
        dq, dk, dv = fixedset_attention_backward(q, k, v, idx, dout)
        return (None, dq, dk, dv) + (None,) * ctx.n_extra


def _tracks_grad(*ts: torch.Tensor) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for t in ts)


def _entropy(w: torch.Tensor) -> float:
    w = w.clamp_min(1e-12)
    return float((-(w * w.log()).sum(-1)).mean().item())


class AttentionComm(nn.Module):
    """Inter-agent attention communication block (``src/agents/mappo.py:138-420``).

    Inputs (B, N, D_in) -> messages (B, N, msg_dim). ``collect_info`` gates the
    diagnostics that synchronise the device (entropy via ``.item()``); timed
    callers must set it False, as in the reference.
    """

    def __init__(self, cfg: MAPPOConfig, in_dim: int) -> None:
        super().__init__()
        self.cfg = cfg
        self.collect_info = True
        self.qkv = nn.Linear(in_dim, 3 * cfg.msg_dim)
        self.proj = nn.Linear(cfg.msg_dim, cfg.msg_dim)
        self.k_bins = max(cfg.n_agents - 1, 1)
        self.k_gate = nn.Linear(in_dim, self.k_bins)
        if cfg.use_orthogonal_init:
            for layer in (self.qkv, self.proj, self.k_gate):
                _ortho_init(layer)

    def _k_eff(self, N: int) -> int:
        return min(max(self.cfg.topk, 1), N - 1)

    # -- diagnostics (only with collect_info) --------------------------------
    @staticmethod
    def _dense_weights(q, k) -> torch.Tensor:
        N = q.shape[1]
        s = torch.matmul(q.float(), k.float().transpose(-1, -2)) / (q.shape[-1] ** 0.5)
        eye = torch.eye(N, device=q.device, dtype=torch.bool).unsqueeze(0)
        return torch.softmax(s.masked_fill(eye, float("-inf")), -1)

    @staticmethod
    def _set_weights(q, k, idx) -> torch.Tensor:
        B, N, d = q.shape
        kk = idx.shape[-1]
        flat = idx.long().reshape(B, N * kk, 1).expand(B, N * kk, d)
        kg = k.float().gather(1, flat).view(B, N, kk, d)
        s = torch.matmul(q.float().unsqueeze(-2), kg.transpose(-1, -2)).squeeze(-2) / d ** 0.5
        return torch.softmax(s, -1)

    # -- forward -------------------------------------------------------------
    def forward(self, x: torch.Tensor,
                pos: torch.Tensor | None = None) -> tuple[torch.Tensor, dict]:
        B, N, _ = x.shape
        mode = self.cfg.attn_mode
        qkv = self.qkv(x)
        q, k, v = (t.contiguous() for t in qkv.chunk(3, dim=-1))
        info: dict = {}

        if mode == "zorder_k":
            if pos is None:
                raise ValueError("attn_mode='zorder_k' needs agent positions")
            kk = self._k_eff(N)
            if _tracks_grad(q, k, v):
                msg, idx = _SetCore.apply(
                    lambda a, b, c, p: zorder_attention(a, b, c, p, kk, ZORDER_BITS,
                                                        return_indices=True),
                    q, k, v, pos)
            else:
                res = zorder_attention(q, k, v, pos, kk, ZORDER_BITS,
                                       return_indices=self.collect_info)
                msg, idx = res if self.collect_info else (res, None)
            info["effective_k"] = float(kk)
            if self.collect_info:
                info["mean_attn_entropy"] = _entropy(self._set_weights(q, k, idx))
            return self.proj(F.gelu(msg)), info

        if mode in ("dense", "dense_sdpa"):
            msg = (_DenseCore.apply(q, k, v) if _tracks_grad(q, k, v)
                   else fused_dense_attention(q, k, v))
            if mode == "dense" and self.collect_info:
                info["mean_attn_entropy"] = _entropy(self._dense_weights(q, k))
            return self.proj(F.gelu(msg)), info

        if mode in ("topk", "topk_gather"):
            kk = self._k_eff(N)
            if _tracks_grad(q, k, v):
                msg, idx = _SetCore.apply(
                    lambda a, b, c: topk_attention(a, b, c, kk, return_indices=True), q, k, v)
            else:
                want_idx = self.collect_info and mode == "topk_gather"
                res = topk_attention(q, k, v, kk, return_indices=want_idx)
                msg, idx = res if want_idx else (res, None)
            if mode == "topk":
                if self.collect_info:
                    info["mean_attn_entropy"] = _entropy(self._dense_weights(q, k))
                info["effective_k"] = float(kk)
            else:
                if self.collect_info:
                    info["effective_k"] = float(kk)
                    info["mean_attn_entropy"] = _entropy(self._set_weights(q, k, idx))
            return self.proj(F.gelu(msg)), info

        if mode in REFERENCE_ONLY_MODES:
            raise NotImplementedError(
                f"attn_mode={mode!r} is a training-study arm outside the HIP attention core")
        raise ValueError(f"unknown attn_mode {mode!r}")
