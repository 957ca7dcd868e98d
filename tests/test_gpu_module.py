"""``AttentionComm`` on the GPU against the reference module's own outputs.

tests/golden/make_golden.py ran the reference's ``AttentionComm.forward``
(src/agents/mappo.py:332-420) on the CPU with fixed weights and inputs; here
the same weights drive this package's module, whose core runs on the HIP
kernels. Bar: within 1e-5 of max|ref| (normwise relative), fp32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MODES = [("dense", 0), ("dense_sdpa", 0), ("topk", 2), ("topk_gather", 1),
         ("topk_gather", 2), ("topk_gather", 3), ("zorder_k", 2), ("zorder_k", 1)]


def _module(mode, k, n_agents, msg_dim, golden, tag):
    from tarmac.agents import AttentionComm, MAPPOConfig
    cfg = MAPPOConfig(obs_dim=18, n_actions=5, n_agents=n_agents, hidden=32, use_comm=True,
                      msg_dim=msg_dim, attn_mode=mode, topk=k)
    mod = AttentionComm(cfg, in_dim=32)
    with torch.no_grad():
        for name in ("qkv.weight", "qkv.bias", "proj.weight", "proj.bias"):
            mod.get_parameter(name).copy_(torch.from_numpy(golden[f"{tag}_w_{name}"]))
    return mod.cuda().eval()


@pytest.mark.parametrize("n_agents", [6, 24])
@pytest.mark.parametrize("msg_dim", [8, 16])
@pytest.mark.parametrize("mode,k", MODES)
def test_module_matches_reference_outputs(golden, n_agents, msg_dim, mode, k):
    tag = f"comm_n{n_agents}_d{msg_dim}"
    mod = _module(mode, k, n_agents, msg_dim, golden, tag)
    mod.collect_info = False
    x = torch.from_numpy(golden[f"{tag}_x"]).cuda()
    pos = torch.from_numpy(golden[f"{tag}_pos"]).cuda()
    with torch.no_grad():
        out, info = mod(x, pos if mode == "zorder_k" else None)
    ref = golden[f"{tag}_{mode}_k{k}_out"]
    got = out.cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max(), mode
    assert "mean_attn_entropy" not in info


def test_module_info_and_errors(golden):
    tag = "comm_n6_d16"
    x = torch.from_numpy(golden[f"{tag}_x"]).cuda()
    mod = _module("topk_gather", 2, 6, 16, golden, tag)
    with torch.no_grad():
        _, info = mod(x)
    assert info["effective_k"] == 2.0 and 0.0 <= info["mean_attn_entropy"] <= np.log(2) + 1e-6
    zmod = _module("zorder_k", 2, 6, 16, golden, tag)
    with pytest.raises(ValueError):
        zmod(x)
    bad = _module("dense", 0, 6, 16, golden, tag)
    bad.cfg.attn_mode = "nonsense"
    with pytest.raises(ValueError):
        bad(x)


def _torch_module_ref(mod, x, pos, mode, k, idx=None):
    """float64 CPU restatement of the module (qkv split, core, gelu, proj) in
    torch, with the given peer sets for the set-based modes; autograd gives
    the reference gradients."""
    import torch.nn.functional as F
    W = {n: p.detach().double().cpu().requires_grad_(True) for n, p in mod.named_parameters()}
    xr = x.detach().double().cpu().requires_grad_(True)
    qkv = xr @ W["qkv.weight"].T + W["qkv.bias"]
    q, kk_, v = qkv.chunk(3, dim=-1)
    B, N, d = q.shape
    s = q @ kk_.transpose(-1, -2) / d ** 0.5
    if mode in ("dense", "dense_sdpa"):
        s = s.masked_fill(torch.eye(N, dtype=torch.bool), float("-inf"))
        msg = torch.softmax(s, -1) @ v
    else:
        ix = torch.from_numpy(idx).long()
        sg = torch.gather(s, -1, ix)
        w = torch.softmax(sg, -1)
        vg = torch.gather(v.unsqueeze(1).expand(B, N, N, d), 2, ix.unsqueeze(-1).expand(B, N, ix.shape[-1], d))
        msg = (w.unsqueeze(-1) * vg).sum(-2)
    out = F.gelu(msg) @ W["proj.weight"].T + W["proj.bias"]
    return out, xr, W


@pytest.mark.parametrize("mode,k", [("dense", 0), ("topk_gather", 2), ("topk", 3), ("zorder_k", 2)])
def test_module_backward_matches_torch_autograd(golden, mode, k):
    """Forward + backward of the whole module: the HIP core's gradients
    (through the retained set for top-k / Z-order) against torch autograd of
    the same composition in float64."""
    tag = "comm_n24_d16"
    mod = _module(mode, k, 24, 16, golden, tag)
    mod.collect_info = False
    x = torch.from_numpy(golden[f"{tag}_x"]).cuda().requires_grad_(True)
    pos = torch.from_numpy(golden[f"{tag}_pos"]).cuda()
    out, _ = mod(x, pos if mode == "zorder_k" else None)
    g = torch.from_numpy(np.random.default_rng(5).standard_normal(out.shape).astype(np.float32)).cuda()
    (out * g).sum().backward()
    idx = None
    if mode != "dense":
        from tarmac.kernels import topk_attention, zorder_attention
        with torch.no_grad():
            q, kk_, v = (t.contiguous() for t in mod.qkv(x).chunk(3, dim=-1))
            kk = min(max(k, 1), 23)
            idx = (zorder_attention(q, kk_, v, pos, kk, 10, return_indices=True)[1]
                   if mode == "zorder_k" else topk_attention(q, kk_, v, kk, return_indices=True)[1])
        idx = idx.cpu().numpy()
    ref, xr, W = _torch_module_ref(mod, x, pos, mode, k, idx)
    assert np.abs(out.detach().cpu().numpy() - ref.detach().numpy()).max() <= 1e-5 * ref.abs().max().item()
    (ref * g.double().cpu()).sum().backward()
    for name, p in mod.named_parameters():
        if name.startswith("k_gate"):
            continue
        got, want = p.grad.cpu().numpy(), W[name].grad.numpy()
        assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max(), name
    assert np.abs(x.grad.cpu().numpy() - xr.grad.numpy()).max() <= 1e-4 * xr.grad.abs().max().item()


@pytest.mark.parametrize("mode,k", [("dense", 0), ("topk_gather", 2), ("zorder_k", 2)])
def test_module_empty_batch(golden, mode, k):
    """An empty batch of episodes passes through the module (forward and
    backward) with correctly shaped empty results."""
    tag = "comm_n6_d16"
    mod = _module(mode, k, 6, 16, golden, tag).train()
    mod.collect_info = False
    x = torch.zeros(0, 6, 32, device="cuda", requires_grad=True)
    pos = torch.zeros(0, 6, 2, device="cuda")
    out, _ = mod(x, pos if mode == "zorder_k" else None)
    assert out.shape[:2] == (0, 6)
    out.sum().backward()
    assert x.grad.shape == (0, 6, 32)
