"""Backward kernels against torch autograd in float64 (CPU).

The reference's Triton kernels are forward-only; its training differentiates
the PyTorch composition (src/agents/mappo.py:192-231 gather path, :361-372
dense). Here torch autograd of that composition, in float64 on the CPU, is
the reference gradient; the fixed-set composition uses the kernel's own
retained sets. Bar: 1e-4 of the largest |ref| gradient entry (normwise).

The fixed-set backward sums each key's dk, dv over the queries that retain
it in ascending query order (bitwise reproducible), except where a set names
a peer twice, the row's bitmask does not fit LDS (N above about 1100 at
d = 16) or d = 128: those rows are summed with fp32 atomics.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import qkv

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _ref_set(q, k, v, idx, g):
    t = [torch.from_numpy(np.asarray(x, np.float64)).requires_grad_(True) for x in (q, k, v)]
    qt, kt, vt = t
    B, N, d = qt.shape
    ix = torch.from_numpy(idx).long()
    kk = ix.shape[-1]
    kg = torch.gather(kt.unsqueeze(1).expand(B, N, N, d), 2, ix.unsqueeze(-1).expand(B, N, kk, d))
    vg = torch.gather(vt.unsqueeze(1).expand(B, N, N, d), 2, ix.unsqueeze(-1).expand(B, N, kk, d))
    s = (qt.unsqueeze(-2) * kg).sum(-1) / d ** 0.5
    out = (torch.softmax(s, -1).unsqueeze(-1) * vg).sum(-2)
    (out * torch.from_numpy(g.astype(np.float64))).sum().backward()
    return [x.grad.numpy() for x in t]


def _ref_dense(q, k, v, g):
    t = [torch.from_numpy(np.asarray(x, np.float64)).requires_grad_(True) for x in (q, k, v)]
    qt, kt, vt = t
    N, d = qt.shape[1], qt.shape[2]
    s = (qt @ kt.transpose(-1, -2) / d ** 0.5).masked_fill(torch.eye(N, dtype=torch.bool), float("-inf"))
    out = torch.softmax(s, -1) @ vt
    (out * torch.from_numpy(g.astype(np.float64))).sum().backward()
    return [x.grad.numpy() for x in t]


def _close(got, want):
    # normwise against the largest of the three gradients: one of them can be
    # exactly zero (N = 2: each query's single peer has weight 1, so dq = 0)
    scale = max(np.abs(b).max() for b in want)
    for a, b in zip(got, want):
        assert np.abs(a.cpu().numpy() - b).max() <= TOL * scale


def _dev(*xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in xs]


@pytest.mark.parametrize("N,d,kk", [(6, 16, 2), (24, 8, 5), (100, 16, 3), (256, 16, 2),
                                    (256, 32, 4), (300, 64, 12), (512, 16, 8), (96, 16, 23),
                                    (384, 16, 95), (384, 32, 95), (300, 8, 30), (1000, 16, 40),
                                    (1500, 8, 3), (100, 128, 3), (300, 128, 12)])
def test_topk_backward(N, d, kk):
    from tarmac.kernels import fixedset_attention_backward, topk_attention
    B = 3
    q, k, v = qkv(31 * N + kk, B, N, d)
    g = np.random.default_rng(N).standard_normal(q.shape).astype(np.float32)
    qd, kd, vd, gd = _dev(q, k, v, g)
    _, idx = topk_attention(qd, kd, vd, kk, return_indices=True)
    got = fixedset_attention_backward(qd, kd, vd, idx, gd)
    torch.cuda.synchronize()
    _close(got, _ref_set(q, k, v, idx.cpu().numpy(), g))


@pytest.mark.parametrize("N,d,kk", [(40, 16, 6), (300, 16, 30), (300, 8, 7), (200, 128, 9)])
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
def test_fixedset_backward_any_sets(idx_dtype, N, d, kk):
    """Arbitrary peer sets, repeated peers and the self pair included (rows
    of 300 take lane pairs per query in the per-query pass, the repeated-peer
    path quads)."""
    from tarmac.kernels import fixedset_attention_backward
    B = 2
    q, k, v = qkv(9, B, N, d)
    g = np.random.default_rng(2).standard_normal(q.shape).astype(np.float32)
    idx = np.random.default_rng(3).integers(0, N, size=(B, N, kk))
    qd, kd, vd, gd = _dev(q, k, v, g)
    got = fixedset_attention_backward(qd, kd, vd, torch.from_numpy(idx).to(idx_dtype).cuda(), gd)
    torch.cuda.synchronize()
    _close(got, _ref_set(q, k, v, idx, g))


@pytest.mark.parametrize("N,d,kk", [(40, 16, 6), (384, 16, 95), (1000, 16, 9)])
def test_fixedset_backward_is_reproducible(N, d, kk):
    """Sets without repeats: dq, dk, dv the same bit for bit on a second
    call; with every set's slots permuted, within the bar of the float64
    reference (a query's softmax sums run in slot order)."""
    from tarmac.kernels import fixedset_attention_backward
    B = 2
    q, k, v = qkv(17 * N + kk, B, N, d)
    g = np.random.default_rng(5).standard_normal(q.shape).astype(np.float32)
    r = np.random.default_rng(6)
    idx = np.stack([np.stack([r.permutation(N)[:kk] for _ in range(N)]) for _ in range(B)])
    perm = np.stack([np.stack([r.permutation(kk) for _ in range(N)]) for _ in range(B)])
    shuffled = np.take_along_axis(idx, perm, axis=-1)
    qd, kd, vd, gd = _dev(q, k, v, g)
    a = fixedset_attention_backward(qd, kd, vd, torch.from_numpy(idx).int().cuda(), gd)
    b = fixedset_attention_backward(qd, kd, vd, torch.from_numpy(idx).int().cuda(), gd)
    c = fixedset_attention_backward(qd, kd, vd, torch.from_numpy(shuffled).int().cuda(), gd)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    _close(a, _ref_set(q, k, v, idx, g))
    _close(c, _ref_set(q, k, v, shuffled, g))


@pytest.mark.parametrize("N,d", [(2, 16), (6, 16), (24, 8), (100, 32), (129, 8), (256, 16), (300, 64),
                                 (700, 16), (1000, 32), (6, 128), (100, 128), (300, 128)])
def test_dense_backward(N, d):
    from tarmac.kernels import dense_attention_backward, fused_dense_attention
    B = 2
    q, k, v = qkv(5 * N + d, B, N, d)
    g = np.random.default_rng(N + 1).standard_normal(q.shape).astype(np.float32)
    qd, kd, vd, gd = _dev(q, k, v, g)
    out = fused_dense_attention(qd, kd, vd)
    got = dense_attention_backward(qd, kd, vd, out, gd)
    torch.cuda.synchronize()
    _close(got, _ref_dense(q, k, v, g))


HALF_TOL = {torch.bfloat16: 1e-2, torch.float16: 2e-3}


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N,d,kk", [(6, 16, 2), (256, 16, 2), (300, 64, 12), (384, 32, 95),
                                    (256, 128, 4)])
def test_half_backward(dt, N, d, kk):
    """bf16 / float16 heads: gradients (computed in fp32 on exact copies,
    returned in the heads' dtype) against float64 autograd on the same
    half-precision inputs, for the dense core (given the half-precision
    forward output) and the top-k core (over the kernel's own retained
    set). Bar: 1e-2 (bf16) / 2e-3 (float16) of the largest |ref| entry."""
    from tarmac.kernels import (dense_attention_backward, fixedset_attention_backward,
                                fused_dense_attention, topk_attention)
    B = 2
    q, k, v = qkv(13 * N + d, B, N, d)
    g = np.random.default_rng(N + 7).standard_normal(q.shape).astype(np.float32)
    qd, kd, vd, gd = (t.to(dt) for t in _dev(q, k, v, g))
    q, k, v, g = (t.float().cpu().numpy() for t in (qd, kd, vd, gd))
    out = fused_dense_attention(qd, kd, vd)
    dense = dense_attention_backward(qd, kd, vd, out, gd)
    _, idx = topk_attention(qd, kd, vd, kk, return_indices=True)
    sets = fixedset_attention_backward(qd, kd, vd, idx, gd)
    torch.cuda.synchronize()
    assert all(x.dtype == dt for x in dense + sets)
    for got, want in ((dense, _ref_dense(q, k, v, g)),
                      (sets, _ref_set(q, k, v, idx.cpu().numpy(), g))):
        scale = max(np.abs(b).max() for b in want)
        for a, b in zip(got, want):
            assert np.abs(a.float().cpu().numpy() - b).max() <= HALF_TOL[dt] * scale


def test_backward_rejects_mixed_dtypes():
    from tarmac.kernels import dense_attention_backward
    q, k, v = _dev(*qkv(1, 2, 16, 16))
    with pytest.raises(TypeError):
        dense_attention_backward(q, k, v, q, q.to(torch.bfloat16))


@pytest.mark.parametrize("N,d", [(6, 16), (256, 16), (300, 64), (700, 16), (300, 128)])
def test_dense_forward_stats_and_saved_backward(N, d):
    """tarmac_dense_fwd_stats: the same output as the plain forward, plane 0
    of stats the log2-domain logsumexp of the scaled scores (float64
    reference), and a backward from those stats equal to one that recomputes
    them."""
    from tarmac.kernels import (dense_attention_backward, dense_attention_forward_stats,
                                fused_dense_attention)
    B = 2
    q, k, v = qkv(7 * N + d, B, N, d)
    g = np.random.default_rng(N + 3).standard_normal(q.shape).astype(np.float32)
    qd, kd, vd, gd = _dev(q, k, v, g)
    out, stats = dense_attention_forward_stats(qd, kd, vd)
    plain = fused_dense_attention(qd, kd, vd)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    s = np.einsum("bnd,bmd->bnm", q.astype(np.float64), k.astype(np.float64)) / np.sqrt(d)
    s[:, np.arange(N), np.arange(N)] = -np.inf
    mx = s.max(-1, keepdims=True)
    lse2 = (mx[..., 0] + np.log(np.exp(s - mx).sum(-1))) / np.log(2.0)
    assert np.abs(stats[:, 0].cpu().numpy() - lse2).max() <= 1e-5 * max(1.0, np.abs(lse2).max())
    saved = dense_attention_backward(qd, kd, vd, out, gd, stats.clone())
    fresh = dense_attention_backward(qd, kd, vd, out, gd)
    torch.cuda.synchronize()
    _close(saved, [x.cpu().numpy().astype(np.float64) for x in fresh])
    _close(saved, _ref_dense(q, k, v, g))
