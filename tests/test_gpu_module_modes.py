"""``AttentionComm`` modes beyond the timed core, and message widths the
kernels do not take directly, on the GPU.

* ``entmax`` (src/agents/mappo.py:294-330) is deterministic: checked against
  a float64 restatement of the module whose entmax is the oracle's exact
  1.5-entmax (1e-4 of max|ref|; the arm bisects in fp32).
* ``random_k`` (:233-263) draws its peers with the reference's own
  ``torch.rand`` call: re-drawing from the same seed gives the set, and the
  output equals float64 attention over that set (1e-5); the sets exclude
  self, hold k distinct peers and are uniform.
* ``adaptive_topk`` (:383-414) is random through its Gumbel gate: with the
  gate forced to one bin it must equal top-k attention at that k, and
  ``expected_k`` must carry gradient to the gate.
* ``msg_dim`` 12, 24, 40, 100 (heads zero-padded to 16, 32, 64, 128) and
  128: forward against
  float64 with the kernel's own retained sets (1e-5), backward against float64
  autograd (1e-4); the retained sets against the exact top k of the unpadded
  scores off near-ties, fp32 and bf16 heads.
* bf16 and float16 modules: forward against float64 on the module's own
  weights and heads, backward to the projections.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import tarmac_oracle as O

pytestmark = pytest.mark.gpu


def _module(mode, k, n_agents, msg_dim, seed=0, in_dim=32):
    from tarmac.agents import AttentionComm, MAPPOConfig
    torch.manual_seed(seed)
    cfg = MAPPOConfig(obs_dim=18, n_actions=5, n_agents=n_agents, hidden=32, use_comm=True,
                      msg_dim=msg_dim, attn_mode=mode, topk=k)
    return AttentionComm(cfg, in_dim=in_dim).cuda()


def _x(B, N, in_dim=32, seed=1):
    g = np.random.default_rng(seed)
    return torch.from_numpy(g.standard_normal((B, N, in_dim)).astype(np.float32)).cuda()


def _heads64(mod, x):
    """float64 CPU q, k, v of the module's qkv projection."""
    W = mod.qkv.weight.detach().double().cpu()
    b = mod.qkv.bias.detach().double().cpu()
    qkv = x.detach().double().cpu() @ W.T + b
    return [t.numpy() for t in qkv.chunk(3, dim=-1)]


def _finish64(mod, msg):
    """gelu then the output projection, float64."""
    m = F.gelu(torch.from_numpy(msg))
    out = m @ mod.proj.weight.detach().double().cpu().T + mod.proj.bias.detach().double().cpu()
    return out.numpy()


@pytest.mark.parametrize("n_agents,msg_dim", [(6, 16), (24, 16), (24, 12)])
def test_entmax_matches_exact_entmax(n_agents, msg_dim):
    mod = _module("entmax", 0, n_agents, msg_dim)
    x = _x(4, n_agents)
    with torch.no_grad():
        out, info = mod(x)
    q, k, v = _heads64(mod, x)
    w = O.entmax15_exact(O.scores(q, k))
    ref = _finish64(mod, w @ v)
    assert np.abs(out.cpu().numpy() - ref).max() <= 1e-4 * np.abs(ref).max()
    support = (w > 0).sum(-1).mean()
    assert abs(info["effective_k"] - support) <= 0.05 * support


@pytest.mark.parametrize("n_agents,msg_dim,k", [(6, 16, 2), (24, 16, 5), (24, 24, 3)])
def test_random_k_attends_over_the_drawn_set(n_agents, msg_dim, k):
    from tarmac.agents.mappo import _random_peers
    mod = _module("random_k", k, n_agents, msg_dim)
    mod.collect_info = False
    x = _x(8, n_agents)
    torch.manual_seed(123)
    with torch.no_grad():
        out, info = mod(x)
    torch.manual_seed(123)
    peers = _random_peers(8, n_agents, k, "cuda").cpu().numpy()
    assert info["effective_k"] == float(k)
    assert not np.any(peers == np.arange(n_agents)[None, :, None])
    assert all(len(set(r)) == k for r in peers.reshape(-1, k).tolist())
    q, kh, v = _heads64(mod, x)
    ref = _finish64(mod, O.prescore_attention(q, kh, v, peers))
    assert np.abs(out.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()


def test_random_k_sets_are_uniform():
    from tarmac.agents.mappo import _random_peers
    torch.manual_seed(7)
    N, k, B = 6, 2, 4000
    peers = _random_peers(B, N, k, "cuda").cpu().numpy()
    counts = np.zeros((N, N))
    for i in range(N):
        np.add.at(counts[i], peers[:, i].ravel(), 1)
    assert np.all(counts[np.arange(N), np.arange(N)] == 0)
    freq = counts / (B * k)
    off = ~np.eye(N, dtype=bool)
    assert np.abs(freq[off] - 1.0 / (N - 1)).max() < 0.02


def test_random_k_trains():
    mod = _module("random_k", 3, 12, 16).train()
    mod.collect_info = False
    x = _x(4, 12).requires_grad_(True)
    out, _ = mod(x)
    out.square().sum().backward()
    assert torch.isfinite(x.grad).all() and mod.qkv.weight.grad.abs().sum() > 0


@pytest.mark.parametrize("bin_", [0, 2])
def test_adaptive_topk_with_a_forced_gate_is_topk(bin_):
    n_agents, msg_dim = 8, 16
    mod = _module("adaptive_topk", 0, n_agents, msg_dim)
    with torch.no_grad():
        mod.k_gate.weight.zero_()
        mod.k_gate.bias.fill_(-100.0)
        mod.k_gate.bias[bin_] = 100.0
    x = _x(4, n_agents)
    out, info = mod(x)
    assert abs(info["expected_k"].item() - (bin_ + 1)) < 1e-6
    assert 0.0 <= info["mean_attn_entropy"] <= np.log(n_agents - 1) + 1e-5
    ref_mod = _module("topk", bin_ + 1, n_agents, msg_dim)
    ref_mod.load_state_dict(mod.state_dict())
    with torch.no_grad():
        ref, _ = ref_mod(x)
    assert (out.detach() - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()


def test_adaptive_topk_expected_k_reaches_the_gate():
    mod = _module("adaptive_topk", 0, 10, 16).train()
    mod.collect_info = False
    out, info = mod(_x(4, 10))
    assert "mean_k" not in info and info["expected_k"].requires_grad
    (out.sum() + info["expected_k"]).backward()
    assert mod.k_gate.weight.grad is not None and mod.k_gate.weight.grad.abs().sum() > 0


@pytest.mark.parametrize("msg_dim", [12, 24, 40, 100, 128])
@pytest.mark.parametrize("mode,k", [("dense", 0), ("topk_gather", 2), ("zorder_k", 2),
                                    ("random_k", 2)])
def test_any_msg_dim(msg_dim, mode, k):
    from tarmac.agents.mappo import _random_peers, _to_width
    from tarmac.kernels import topk_attention, zorder_attention
    n_agents = 16
    mod = _module(mode, k, n_agents, msg_dim)
    mod.collect_info = False
    x = _x(6, n_agents)
    pos = torch.from_numpy(np.random.default_rng(2).random((6, n_agents, 2)).astype(np.float32)).cuda()
    torch.manual_seed(9)
    with torch.no_grad():
        out, _ = mod(x, pos if mode == "zorder_k" else None)
        q, kh, v = (t.contiguous() for t in mod.qkv(x).chunk(3, dim=-1))
        qw, kw, vw, _ = _to_width(q, kh, v)
        assert qw.shape[-1] in (16, 32, 64, 128)
        if mode == "topk_gather":
            peers = topk_attention(qw, kw, vw, k, return_indices=True)[1]
        elif mode == "zorder_k":
            peers = zorder_attention(qw, kw, vw, pos, k, 10, return_indices=True)[1]
        elif mode == "random_k":
            torch.manual_seed(9)
            peers = _random_peers(6, n_agents, k, "cuda")
    q64, k64, v64 = _heads64(mod, x)
    if mode == "dense":
        msg = O.dense_unfused(q64, k64, v64)
    else:
        msg = O.prescore_attention(q64, k64, v64, peers.cpu().numpy().astype(np.int64))
    ref = _finish64(mod, msg)
    assert np.abs(out.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("msg_dim", [12, 24, 40, 100])
def test_padded_width_selects_on_unpadded_scores(msg_dim, dt):
    """The top-k peers the module takes on padded, pre-scaled heads are the
    exact top k of q.k / sqrt(msg_dim) on the unpadded heads (float64 over
    the heads' own values), on every row whose k-th and (k+1)-th scores are
    further apart than four times the fp32 score error bound; bf16 heads are
    padded and scaled in fp32, so the bound is the same."""
    from tarmac.agents.mappo import _to_width
    from tarmac.kernels import topk_attention
    n_agents, k = 48, 3
    mod = _module("topk_gather", k, n_agents, msg_dim).to(dt)
    x = _x(8, n_agents).to(dt)
    with torch.no_grad():
        q, kh, v = (t.contiguous() for t in mod.qkv(x).chunk(3, dim=-1))
        qw, kw, vw, _ = _to_width(q, kh, v)
        assert qw.dtype == torch.float32
        peers = topk_attention(qw, kw, vw, k, return_indices=True)[1].cpu().numpy()
    q64, k64 = (t.double().cpu().numpy() for t in (q, kh))
    s = O.scores(q64, k64)
    want = O.topk_indices(s, k)
    far = ~O.near_tie_rows(s, k, 4 * O.score_error_bound(q64, k64).max(-1))
    assert far.mean() > 0.9
    assert np.array_equal(np.sort(peers, -1)[far], np.sort(want, -1)[far])


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("msg_dim", [12, 16, 128])
@pytest.mark.parametrize("mode,k", [("dense", 0), ("topk_gather", 2), ("zorder_k", 2)])
def test_half_precision_module(mode, k, msg_dim, dt):
    """bf16 and float16 modules (the reference's half-precision arms): the
    forward against a float64 evaluation of the same module (its own weights
    and heads, the kernel's own retained set) within the dtype's rounding
    (3e-2 bf16, 4e-3 float16, of max|ref|), and a backward that reaches the
    projections with finite gradients."""
    from tarmac.agents.mappo import _to_width
    from tarmac.kernels import topk_attention
    n_agents = 24
    g = np.random.default_rng(2)
    pos = torch.from_numpy(g.random((4, n_agents, 2)).astype(np.float32)).cuda()
    mod = _module(mode, k, n_agents, msg_dim).to(dt).train()
    mod.collect_info = False
    x = _x(4, n_agents).to(dt)
    out, _ = mod(x, pos if mode == "zorder_k" else None)
    assert out.dtype == dt
    with torch.no_grad():
        q, kh, v = (t.contiguous() for t in mod.qkv(x).chunk(3, dim=-1))
        q64, k64, v64 = (t.double().cpu().numpy() for t in (q, kh, v))
        if mode == "dense":
            msg = O.dense_unfused(q64, k64, v64)
        else:
            if mode == "topk_gather":
                qw, kw, vw, _ = _to_width(q, kh, v)
                peers = topk_attention(qw, kw, vw, k, return_indices=True)[1].cpu().numpy()
            else:
                peers = O.canon_morton_window(pos.cpu().numpy(), k, 10)
            msg = O.prescore_attention(q64, k64, v64, peers.astype(np.int64))
    ref = _finish64(mod, msg)
    tol = 3e-2 if dt == torch.bfloat16 else 4e-3
    err = np.abs(out.detach().double().cpu().numpy() - ref).max()
    assert err <= tol * np.abs(ref).max(), err
    out.float().square().sum().backward()
    for name in ("qkv.weight", "proj.weight"):
        grad = mod.get_parameter(name).grad
        assert grad is not None and torch.isfinite(grad).all() and grad.abs().sum() > 0, name


@pytest.mark.parametrize("msg_dim", [12, 100])
def test_padded_width_backward_matches_float64_autograd(msg_dim):
    """msg_dim 12 and 100 (padded to 16 and 128): gradients of the whole
    module through the dense HIP core and the padding, against float64
    autograd."""
    mod = _module("dense", 0, 10, msg_dim).train()
    mod.collect_info = False
    x = _x(3, 10).requires_grad_(True)
    out, _ = mod(x)
    g = torch.from_numpy(np.random.default_rng(4).standard_normal(out.shape).astype(np.float32)).cuda()
    (out * g).sum().backward()
    W = {n: p.detach().double().cpu().requires_grad_(True) for n, p in mod.named_parameters()}
    xr = x.detach().double().cpu().requires_grad_(True)
    q, k, v = (xr @ W["qkv.weight"].T + W["qkv.bias"]).chunk(3, dim=-1)
    s = q @ k.transpose(-1, -2) / msg_dim ** 0.5
    s = s.masked_fill(torch.eye(10, dtype=torch.bool), float("-inf"))
    ref = F.gelu(torch.softmax(s, -1) @ v) @ W["proj.weight"].T + W["proj.bias"]
    (ref * g.double().cpu()).sum().backward()
    assert np.abs(x.grad.cpu().numpy() - xr.grad.numpy()).max() <= 1e-4 * xr.grad.abs().max().item()
    for name in ("qkv.weight", "proj.weight"):
        got, want = mod.get_parameter(name).grad.cpu().numpy(), W[name].grad.numpy()
        assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max(), name


def test_wide_messages_are_refused():
    mod = _module("dense", 0, 6, 160)
    with pytest.raises(NotImplementedError, match="up to 128"):
        mod(_x(2, 6))
