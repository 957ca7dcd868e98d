"""Dense, fixed-set and Z-order paths on the GPU against the oracle.

Bars: fp32 outputs within 1e-5 of max|ref| (normwise relative) against the
float64 restatements; bf16 within 1e-2 against float64 evaluation of the
bf16-rounded inputs; Morton codes and window indices bit-exact against the
reference's golden vectors and the C oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import tarmac_oracle as O
from conftest import qkv

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 1e-2


def dev(*xs, dtype=torch.float32):
    return [torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(dtype) for x in xs]


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def normwise(got, ref):
    return np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)


# ---------------------------------------------------------------------------
# dense
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,d", [(2, 16), (6, 16), (6, 8), (17, 16), (64, 32), (100, 16),
                                 (128, 64), (256, 16), (384, 16), (512, 32), (1024, 16),
                                 (1024, 64), (32, 64), (40, 8), (33, 32), (64, 16), (48, 64),
                                 (6, 128), (100, 128), (256, 128), (1024, 128)])
def test_dense_f32(N, d):
    from tarmac.kernels import fused_dense_attention
    B = max(2, min(16, 4096 // N))
    q, k, v = qkv(N * 131 + d * 17, B, N, d)
    out = host(fused_dense_attention(*dev(q, k, v)))
    ref = O.canon_dense(q, k, v)
    assert normwise(out, ref) <= F32_TOL


@pytest.mark.parametrize("N,d,chunk", [(256, 16, 64), (1000, 16, 128), (512, 64, 64), (64, 16, 32),
                                       (300, 128, 64)])
def test_dense_streamed_chunks(N, d, chunk):
    from tarmac.kernels import fused_dense_attention
    q, k, v = qkv(N + chunk, 3, N, d)
    out = host(fused_dense_attention(*dev(q, k, v), block_kn=chunk))
    assert normwise(out, O.canon_dense(q, k, v)) <= F32_TOL


@pytest.mark.parametrize("N,d", [(64, 16), (256, 16), (256, 32), (512, 64), (100, 16), (300, 128)])
def test_dense_bf16(N, d):
    from tarmac.kernels import fused_dense_attention
    q, k, v = qkv(77 + N + d, 8, N, d)
    qb, kb, vb = (O.bf16_round(x) for x in (q, k, v))
    out = host(fused_dense_attention(*dev(q, k, v, dtype=torch.bfloat16)))
    ref = O.canon_dense(qb, kb, vb)
    assert normwise(out, ref) <= BF16_TOL


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("B,N", [(4, 256), (128, 256), (64, 100), (1024, 256)])
@pytest.mark.parametrize("spread", [0.0, 15.0, 60.0])
def test_dense_loose_offset_bound(dtype, B, N, spread):
    """A row staged in one chunk takes its exponent offset from |q| max|k|
    instead of a running maximum. Keys with a large component orthogonal to
    the queries (`spread`) push that bound far above the true maximum: at 15
    the terms shrink by about 2^-40 and stay normal; at 60 they underflow,
    the query's sum falls below 2^-64 and the wave reruns the row with the
    running maximum. Every other query carries the large component, so waves
    mix rows that need the rerun with rows that do not; one, two and (bf16)
    four query tiles per wave (B = 4 / 128 / 1024 at N = 256)."""
    from tarmac.kernels import fused_dense_attention
    d = 16
    g = np.random.default_rng(int(spread) + B + N)
    q = g.standard_normal((B, N, d)).astype(np.float32) * 0.1
    k = g.standard_normal((B, N, d)).astype(np.float32) * 0.1
    v = g.standard_normal((B, N, d)).astype(np.float32)
    q[:, ::2, 0] = 8.0
    q[:, 1::2, 0] = g.standard_normal((B, N // 2)).astype(np.float32)
    k[..., 0] = g.standard_normal((B, N)).astype(np.float32)
    k[..., 1] = spread
    if dtype == "bf16":
        q, k, v = (O.bf16_round(x) for x in (q, k, v))
        out = host(fused_dense_attention(*dev(q, k, v, dtype=torch.bfloat16)))
        tol = BF16_TOL
    else:
        out = host(fused_dense_attention(*dev(q, k, v)))
        tol = F32_TOL
    rows = np.arange(B) if B <= 128 else np.random.default_rng(B).choice(B, 24, replace=False)
    ref = O.canon_dense(q[rows], k[rows], v[rows])
    assert np.isfinite(out).all()
    assert normwise(out[rows], ref) <= tol


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("where", ["all", "late"])
@pytest.mark.parametrize("spread", [0.0, 15.0, 60.0])
def test_dense_loose_offset_bound_chunked(dtype, where, spread):
    """Rows in four 64-key chunks: the offset is the bound over the keys
    staged so far and rises with a chunk that holds a longer key. `late` puts
    the long keys in the last two chunks only, so the first chunks' terms are
    rescaled by 2^-(rise) (about 2^-33 at spread 15; at 60 they vanish and the
    workgroup reruns the row online)."""
    from tarmac.kernels import fused_dense_attention
    B, N, d = 128, 256, 16
    g = np.random.default_rng(int(spread) + (7 if where == "late" else 0))
    q = g.standard_normal((B, N, d)).astype(np.float32) * 0.1
    k = g.standard_normal((B, N, d)).astype(np.float32) * 0.1
    v = g.standard_normal((B, N, d)).astype(np.float32)
    q[:, ::2, 0] = 8.0
    q[:, 1::2, 0] = g.standard_normal((B, N // 2)).astype(np.float32)
    k[..., 0] = g.standard_normal((B, N)).astype(np.float32)
    if where == "all":
        k[..., 1] = spread
    else:
        k[:, N // 2:, 1] = spread
    if dtype == "bf16":
        q, k, v = (O.bf16_round(x) for x in (q, k, v))
        out = host(fused_dense_attention(*dev(q, k, v, dtype=torch.bfloat16), block_kn=64))
        tol = BF16_TOL
    else:
        out = host(fused_dense_attention(*dev(q, k, v), block_kn=64))
        tol = F32_TOL
    rows = np.random.default_rng(3).choice(B, 24, replace=False)
    assert np.isfinite(out).all()
    assert normwise(out[rows], O.canon_dense(q[rows], k[rows], v[rows])) <= tol


@pytest.mark.parametrize("B,N,d", [(1024, 256, 16), (4096, 256, 16), (512, 512, 16), (1024, 256, 32),
                                   (2048, 256, 32), (256, 512, 32), (256, 256, 64)])
def test_dense_bf16_large_batch(B, N, d):
    """The launch shapes the bench times (two and four query tiles per wave;
    rows of 512 keys at d = 32 staged whole in 80 KB, of 256 keys at d = 64
    in two chunks) on sampled rows against float64 evaluation of the bf16
    inputs."""
    from tarmac.kernels import fused_dense_attention
    q, k, v = qkv(5 * B + N + d, B, N, d)
    qb, kb, vb = (O.bf16_round(x) for x in (q, k, v))
    out = host(fused_dense_attention(*dev(q, k, v, dtype=torch.bfloat16)))
    rows = np.random.default_rng(B + N).choice(B, 16, replace=False)
    assert np.isfinite(out).all()
    assert normwise(out[rows], O.canon_dense(qb[rows], kb[rows], vb[rows])) <= BF16_TOL


def test_dense_headline_shape():
    from tarmac.kernels import fused_dense_attention
    B, N, d = 1024, 256, 16
    q, k, v = qkv(1234 + 7 * N + d, B, N, d)
    out = host(fused_dense_attention(*dev(q, k, v)))
    rows = np.random.default_rng(1).choice(B, 32, replace=False)
    assert normwise(out[rows], O.canon_dense(q[rows], k[rows], v[rows])) <= F32_TOL
    assert np.isfinite(out).all()


# ---------------------------------------------------------------------------
# fixed set
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,d,kk,itype", [(6, 16, 2, torch.int64), (64, 8, 3, torch.int32),
                                          (512, 16, 2, torch.int64), (200, 64, 7, torch.int32),
                                          (33, 32, 1, torch.int64), (300, 128, 5, torch.int32)])
def test_fixedset_f32(N, d, kk, itype):
    from tarmac.kernels import fused_prescore_attention
    B = 6
    q, k, v = qkv(N * 977 + kk, B, N, d)
    idx = np.random.default_rng(N).integers(0, N, (B, N, kk))  # repeats and self allowed
    out = host(fused_prescore_attention(*dev(q, k, v), torch.from_numpy(idx).to("cuda", itype)))
    assert normwise(out, O.canon_fixedset(q, k, v, idx)) <= F32_TOL


@pytest.mark.parametrize("d", [32, 128])
def test_fixedset_bf16(d):
    from tarmac.kernels import fused_prescore_attention
    B, N, kk = 4, 128, 4
    q, k, v = qkv(3, B, N, d)
    idx = np.random.default_rng(3).integers(0, N, (B, N, kk))
    out = host(fused_prescore_attention(*dev(q, k, v, dtype=torch.bfloat16),
                                        torch.from_numpy(idx).cuda()))
    ref = O.canon_fixedset(*(O.bf16_round(x) for x in (q, k, v)), idx)
    assert normwise(out, ref) <= BF16_TOL


def test_fixedset_out_of_range_rows_are_nan():
    from tarmac.kernels import fused_prescore_attention
    B, N, d = 2, 16, 16
    q, k, v = qkv(4, B, N, d)
    idx = np.random.default_rng(4).integers(0, N, (B, N, 2))
    idx[0, 3, 1] = N
    idx[1, 5, 0] = -1
    out = host(fused_prescore_attention(*dev(q, k, v), torch.from_numpy(idx).cuda()))
    assert np.isnan(out[0, 3]).all() and np.isnan(out[1, 5]).all()
    good = np.ones((B, N), bool); good[0, 3] = good[1, 5] = False
    ref = O.canon_fixedset(q, k, v, np.clip(idx, 0, N - 1))
    assert np.abs(out[good] - ref[good]).max() <= F32_TOL * np.abs(ref).max()


# ---------------------------------------------------------------------------
# Z-order
# ---------------------------------------------------------------------------

def test_morton_codes_golden(golden):
    from tarmac.kernels import _morton_code
    for name in ("m6", "m64", "m512", "mgrid", "mflat", "mline"):
        pos = torch.from_numpy(golden[f"{name}_pos"]).cuda()
        for bits in (10, 16):
            got = _morton_code(pos, bits).cpu().numpy()
            assert np.array_equal(got, golden[f"{name}_code{bits}"].astype(np.int64)), (name, bits)


def test_morton_window_golden(golden):
    from tarmac.kernels import select_morton_window
    for name in ("m6", "m64", "m512", "mgrid"):
        pos = torch.from_numpy(golden[f"{name}_pos"]).cuda()
        distinct = golden[f"{name}_distinct10"]
        for kk in (1, 2, 3, 4):
            key = f"{name}_win{kk}"
            if key not in golden:
                continue
            got = select_morton_window(pos, kk).cpu().numpy()
            assert got.dtype == np.int64
            ref = golden[key].astype(np.int64)
            assert np.array_equal(got[distinct], ref[distinct]), (name, kk)


@pytest.mark.parametrize("B,N,kk,bits", [(8, 6, 2, 10), (4, 512, 2, 16), (4, 512, 4, 10),
                                         (2, 1000, 3, 16), (3, 64, 63, 16), (2, 4000, 2, 16),
                                         (64, 17, 5, 4)])
def test_morton_window_vs_oracle(B, N, kk, bits):
    """Bit-exact, ties included (few bits force equal codes; both sides order
    equal codes by agent index)."""
    from tarmac.kernels import _morton_code, select_morton_window
    pos = np.random.default_rng(N + bits).random((B, N, 2)).astype(np.float32)
    pd = torch.from_numpy(pos).cuda()
    assert np.array_equal(_morton_code(pd, bits).cpu().numpy(), O.canon_morton_codes(pos, bits))
    got = select_morton_window(pd, kk, bits).cpu().numpy()
    assert np.array_equal(got, O.canon_morton_window(pos, kk, bits))


@pytest.mark.parametrize("B,N,d,kk,bits", [(8, 6, 16, 2, 10), (16, 512, 16, 2, 16),
                                           (4, 512, 32, 4, 16), (4, 100, 8, 3, 10),
                                           (2, 2048, 64, 1, 16), (4, 300, 128, 3, 10)])
def test_zorder_fused_f32(B, N, d, kk, bits):
    from tarmac.kernels import zorder_attention
    q, k, v = qkv(4242 + N, B, N, d)
    pos = np.random.default_rng(4242 + N).random((B, N, 2)).astype(np.float32)
    out, idx = zorder_attention(*dev(q, k, v), torch.from_numpy(pos).cuda(), kk, bits,
                                return_indices=True)
    out, idx = host(out), idx.cpu().numpy()
    want_idx = O.canon_morton_window(pos, kk, bits)
    assert np.array_equal(idx, want_idx)
    ref = O.prescore_attention(q.astype(np.float64), k.astype(np.float64),
                               v.astype(np.float64), want_idx)
    assert normwise(out, ref) <= F32_TOL


@pytest.mark.parametrize("d", [16, 128])
def test_zorder_fused_bf16(d):
    from tarmac.kernels import zorder_attention
    B, N, kk = 4, 512, 2
    q, k, v = qkv(9, B, N, d)
    pos = np.random.default_rng(9).random((B, N, 2)).astype(np.float32)
    out = host(zorder_attention(*dev(q, k, v, dtype=torch.bfloat16),
                                torch.from_numpy(pos).cuda(), kk, 16))
    idx = O.canon_morton_window(pos, kk, 16)
    ref = O.prescore_attention(*(O.bf16_round(x).astype(np.float64) for x in (q, k, v)), idx)
    assert normwise(out, ref) <= BF16_TOL


def test_zorder_headline_shape():
    """C5: B=1024, N=512, d=16, k=2, 16-bit codes; sample rows vs the oracle."""
    from tarmac.kernels import zorder_attention
    B, N, d, kk = 1024, 512, 16, 2
    q, k, v = qkv(4242 + N, B, N, d)
    pos = np.random.default_rng(5).random((B, N, 2)).astype(np.float32)
    out, idx = zorder_attention(*dev(q, k, v), torch.from_numpy(pos).cuda(), kk, 16,
                                return_indices=True)
    out, idx = host(out), idx.cpu().numpy()
    rows = np.random.default_rng(2).choice(B, 32, replace=False)
    want = O.canon_morton_window(pos[rows], kk, 16)
    assert np.array_equal(idx[rows], want)
    ref = O.prescore_attention(*(x[rows].astype(np.float64) for x in (q, k, v)), want)
    assert normwise(out[rows], ref) <= F32_TOL


def test_noop():
    from tarmac import _lib
    from tarmac._launch import ptr, stream
    t = torch.zeros(1, device="cuda")
    _lib.check(_lib.LIB.tarmac_noop(ptr(t), stream(t)))
    assert t.item() == 1.0
