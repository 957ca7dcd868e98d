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
random_k       k peers drawn uniformly without the self pair, exactly as
               ``mappo.py:233-263`` draws them (the same ``torch.rand``
               call), then ``tarmac_fixedset_fwd`` over that set
entmax         alpha-entmax over all peers by the reference's 24-step
               threshold bisection (``mappo.py:294-330``), dense torch ops
adaptive_topk  the Gumbel-softmax k gate over dense weights
               (``mappo.py:383-414``), dense torch ops
=============  ==========================================================

``entmax`` and ``adaptive_topk`` are training-study arms outside the timed
core; their dense (B, N, N) formulations run as torch operations on the
device, as in the reference. Any ``msg_dim`` up to 128 works: heads whose
width the kernels do not take (fp32: 8, 16, 32, 64, 128; bf16: 16, 32, 64,
128) are zero-padded to the next width, with q pre-scaled by
sqrt(width / msg_dim) so that scores keep the 1/sqrt(msg_dim) scale; that
padding and scaling happen
in fp32 (bf16 heads are widened first, exactly), so the only perturbation of
the scores is fp32 rounding. float16 heads run the fp32 kernels on exact
fp32 copies. Messages return in the heads' dtype.

The reference's Triton kernels are forward-only
(``scripts/bench_attention_core.py:172-176``) and its training differentiates
the PyTorch composition; here the core's backward runs on HIP kernels too
(:mod:`tarmac.kernels.backward`, fp32 arithmetic for every head dtype):
gradients reach q, k, v through the retained set of the top-k and Z-order
cores, and through every pair of the dense core.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels.backward import (dense_attention_backward, dense_attention_forward_stats,
                                fixedset_attention_backward)
from ..kernels.fused_dense_attention import fused_dense_attention
from ..kernels.fused_prescore_attention import fused_prescore_attention
from ..kernels.fused_topk_attention import topk_attention
from ..kernels.prescore_selection import zorder_attention

#: Morton bits per axis of the zorder_k selector (``select_morton_window``'s
#: default, ``src/kernels/prescore_selection.py:62``).
ZORDER_BITS = 10

HIP_MODES = ("dense", "dense_sdpa", "topk", "topk_gather", "zorder_k", "random_k")
TORCH_MODES = ("entmax", "adaptive_topk")

#: Head widths the HIP kernels take, per dtype.
_WIDTHS = {torch.float32: (8, 16, 32, 64, 128), torch.bfloat16: (16, 32, 64, 128),
           torch.float16: (8, 16, 32, 64, 128)}


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
    """Dense core with the HIP backward (fp32 arithmetic)."""

    @staticmethod
    def forward(ctx, q, k, v):
        if q.dtype == torch.float32:
            out, stats = dense_attention_forward_stats(q, k, v)
        else:  # bf16 / float16: the backward recomputes the statistics in fp32
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


def _kernel_width(d: int, dtype: torch.dtype) -> int:
    for w in _WIDTHS.get(dtype, ()):
        if w >= d:
            return w
    raise NotImplementedError(
        f"msg_dim={d} ({dtype}): the HIP attention core takes head widths up to 128")


def _to_width(q, k, v):
    """Zero-pad the heads to a width the kernels take; q is scaled so that
    q'.k' / sqrt(width) = q.k / sqrt(d). Padded heads are fp32 (bf16 and
    float16 values widen exactly, so the scaling rounds once, at fp32).
    Returns (q', k', v', d)."""
    d = q.shape[-1]
    w = _kernel_width(d, q.dtype)
    if w == d:
        return q, k, v, d
    q, k, v = q.float(), k.float(), v.float()
    pad = (0, w - d)
    return (F.pad(q * math.sqrt(w / d), pad), F.pad(k, pad), F.pad(v, pad), d)


def _random_peers(B: int, N: int, kk: int, device) -> torch.Tensor:
    """k peers per agent uniformly without replacement, self excluded: the
    reference ranks uniform noise with self pushed to +inf and keeps the k
    smallest (``mappo.py:250-255``); the same draw gives the same sets."""
    noise = torch.rand(B, N, N, device=device)
    eye = torch.eye(N, device=device, dtype=torch.bool).unsqueeze(0)
    noise = noise.masked_fill(eye, float("inf"))
    return noise.topk(kk, dim=-1, largest=False, sorted=False).indices


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

    # -- the torch-composed arms (outside the timed core) ---------------------
    def _entmax(self, q, k, v, N: int) -> tuple[torch.Tensor, dict]:
        """alpha-entmax over all peers (``mappo.py:294-330``): threshold tau
        found by 24 bisection steps on sum_j [(alpha-1) s_j - tau]_+^(1/(alpha-1)) = 1,
        starting from [max - 1, max]; the self pair sits far below any threshold."""
        alpha = self.cfg.entmax_alpha
        z = (torch.matmul(q, k.transpose(-1, -2).contiguous()) / math.sqrt(q.shape[-1])) * (alpha - 1.0)
        z.diagonal(dim1=-2, dim2=-1).fill_(torch.finfo(z.dtype).min / 4)
        power = 1.0 / (alpha - 1.0)
        hi = z.amax(dim=-1, keepdim=True)
        lo = hi - 1.0
        for _ in range(24):
            mid = 0.5 * (lo + hi)
            above = (z - mid).clamp_min(0).pow(power).sum(-1, keepdim=True) > 1.0
            lo = torch.where(above, mid, lo)
            hi = torch.where(above, hi, mid)
        p = (z - 0.5 * (lo + hi)).clamp_min(0).pow(power)
        p = p / p.sum(-1, keepdim=True).clamp_min(1e-8)
        info: dict = {}
        if self.collect_info:
            info["effective_k"] = float((p > 0).sum(-1).float().mean().item())
        return torch.matmul(p, v), info

    def _adaptive_topk(self, x, q, k, v, N: int) -> tuple[torch.Tensor, dict]:
        """Per-agent k from a hard Gumbel-softmax gate over k = 1..N-1, applied
        to the dense weights (``mappo.py:383-414``): the weights outside each
        row's chosen top k are zeroed and the rest renormalised; ``expected_k``
        stays a differentiable tensor."""
        w = self._dense_weights_like(q, k)
        info: dict = {}
        if self.collect_info:
            info["mean_attn_entropy"] = _entropy(w)
        gate = F.gumbel_softmax(self.k_gate(x), tau=1.0, hard=True)          # (B, N, K)
        ranked, order = w.sort(dim=-1, descending=True)
        # prefix[m, j] = 1 when rank j is within the first m + 1 ranks
        ranks = torch.arange(N, device=x.device)
        prefix = (ranks.view(1, N) <= torch.arange(self.k_bins, device=x.device).view(-1, 1))
        keep_ranked = torch.matmul(gate, prefix.to(w.dtype))                  # (B, N, N)
        keep = torch.zeros_like(w).scatter_(-1, order, keep_ranked)
        attn = w * keep
        attn = attn / attn.sum(-1, keepdim=True).clamp_min(1e-8)
        ks = torch.arange(1, self.k_bins + 1, device=x.device, dtype=gate.dtype)
        info["expected_k"] = (gate * ks).sum(-1).mean()
        if self.collect_info:
            info["mean_k"] = float(info["expected_k"].item())
        return torch.matmul(attn, v), info

    @staticmethod
    def _dense_weights_like(q, k) -> torch.Tensor:
        """softmax(q k^T / sqrt(d)) with the self pair masked, in q's dtype."""
        N = q.shape[1]
        s = torch.matmul(q, k.transpose(-1, -2).contiguous()) / math.sqrt(q.shape[-1])
        s = s.masked_fill(torch.eye(N, device=q.device, dtype=torch.bool).unsqueeze(0),
                          float("-inf"))
        return torch.softmax(s, -1)

    # -- forward -------------------------------------------------------------
    def forward(self, x: torch.Tensor,
                pos: torch.Tensor | None = None) -> tuple[torch.Tensor, dict]:
        B, N, _ = x.shape
        mode = self.cfg.attn_mode
        qkv = self.qkv(x)
        # one copy into a [3, B, N, m] buffer: q, k and v are then contiguous
        # views (three .contiguous() chunks would be three launches)
        m = qkv.shape[-1] // 3
        q, k, v = qkv.view(B, N, 3, m).permute(2, 0, 1, 3).contiguous().unbind(0)

        if mode == "entmax":
            msg, info = self._entmax(q, k, v, N)
            return self.proj(F.gelu(msg)), info
        if mode == "adaptive_topk":
            msg, info = self._adaptive_topk(x, q, k, v, N)
            return self.proj(F.gelu(msg)), info
        if mode not in HIP_MODES:
            raise ValueError(f"unknown attn_mode {mode!r}")
        if mode == "zorder_k" and pos is None:
            raise ValueError("attn_mode='zorder_k' needs agent positions")
        qw, kw, vw, d = _to_width(q, k, v)
        msg, info = self._core(mode, q, k, qw, kw, vw, pos, B, N)
        return self.proj(F.gelu(msg[..., :d].to(q.dtype))), info

    def _core(self, mode, q, k, qw, kw, vw, pos, B: int, N: int) -> tuple[torch.Tensor, dict]:
        """The HIP core on kernel-width heads (qw, kw, vw); q, k are the
        unpadded heads for the diagnostics."""
        info: dict = {}
        grad = _tracks_grad(qw, kw, vw)
        if mode == "zorder_k":
            kk = self._k_eff(N)
            if grad:
                msg, idx = _SetCore.apply(
                    lambda a, b, c, p: zorder_attention(a, b, c, p, kk, ZORDER_BITS,
                                                        return_indices=True),
                    qw, kw, vw, pos)
            else:
                res = zorder_attention(qw, kw, vw, pos, kk, ZORDER_BITS,
                                       return_indices=self.collect_info)
                msg, idx = res if self.collect_info else (res, None)
            info["effective_k"] = float(kk)
            if self.collect_info:
                info["mean_attn_entropy"] = _entropy(self._set_weights(q, k, idx))
            return msg, info

        if mode == "random_k":
            kk = self._k_eff(N)
            peers = _random_peers(B, N, kk, qw.device)
            if grad:
                msg, _ = _SetCore.apply(
                    lambda a, b, c, ix: (fused_prescore_attention(a, b, c, ix), ix),
                    qw, kw, vw, peers)
            else:
                msg = fused_prescore_attention(qw, kw, vw, peers)
            info["effective_k"] = float(kk)
            return msg, info

        if mode in ("dense", "dense_sdpa"):
            msg = _DenseCore.apply(qw, kw, vw) if grad else fused_dense_attention(qw, kw, vw)
            if mode == "dense" and self.collect_info:
                info["mean_attn_entropy"] = _entropy(self._dense_weights(q, k))
            return msg, info

        kk = self._k_eff(N)  # topk, topk_gather
        if grad:
            msg, idx = _SetCore.apply(
                lambda a, b, c: topk_attention(a, b, c, kk, return_indices=True), qw, kw, vw)
        else:
            want_idx = self.collect_info and mode == "topk_gather"
            res = topk_attention(qw, kw, vw, kk, return_indices=want_idx)
            msg, idx = res if want_idx else (res, None)
        if mode == "topk":
            if self.collect_info:
                info["mean_attn_entropy"] = _entropy(self._dense_weights(q, k))
            info["effective_k"] = float(kk)
        else:
            if self.collect_info:
                info["effective_k"] = float(kk)
                info["mean_attn_entropy"] = _entropy(self._set_weights(q, k, idx))
        return msg, info
