"""Fused and streaming top-k on the GPU against the oracle.

fp32 bar: retained indices bit-exact against the canonical-order C oracle
(same score rounding as the kernel), in the same (score desc, index asc) order
for k <= 8; outputs within 1e-5 of max|ref| (normwise relative) against the
float64 restatement of the reference's gather path wherever the k-th score is
not a near-tie. bf16 bar: retained indices bit-exact against the
canonical-order C oracle on the bf16-rounded inputs (the exact top k of the
fp32 scores of the converted inputs, ties to the lower index) on every path
and launch shape, and outputs within 1e-2 of max|ref| against a float64
evaluation over that set.
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


def run_topk(q, k, v, kk, chunk=None):
    from tarmac.kernels import topk_attention
    qd, kd, vd = dev(q, k, v)
    out, idx = topk_attention(qd, kd, vd, kk, return_indices=True, key_chunk=chunk)
    torch.cuda.synchronize()
    return out.cpu().numpy(), idx.cpu().numpy()


def check_f32(q, k, v, kk, out, idx, exact_order=True):
    out_c, idx_c = O.canon_topk(q, k, v, kk)
    if exact_order:
        assert np.array_equal(idx, idx_c), "retained indices differ from the canonical oracle"
    else:
        assert np.array_equal(np.sort(idx, -1), np.sort(idx_c, -1))
    scale = max(np.abs(out_c).max(), 1e-30)
    assert np.abs(out - out_c).max() <= F32_TOL * scale
    # against the float64 reference path, off near-ties
    out_r, idx_r = O.topk_gather(q.astype(np.float64), k.astype(np.float64),
                                 v.astype(np.float64), kk)
    s64 = O.scores(q.astype(np.float64), k.astype(np.float64))
    amb = O.near_tie_rows(s64, kk, O.score_error_bound(q, k).max(-1))
    same = np.all(np.sort(idx, -1) == np.sort(idx_r, -1), -1)
    assert np.all(same | amb)
    if same.any():
        assert np.abs(out - out_r)[same].max() <= F32_TOL * max(np.abs(out_r).max(), 1e-30)


def _set_filter(mode: int) -> int:
    """0 = packed pass (fp32 MFMA scores), 1 = automatic, 2 = split-bf16
    filter-and-verify wherever supported, 3 = register-list pass (fp32),
    4 = packed pass on split-bf16 scores (fp32, d = 16), 5 = the same on
    32 x 32 score tiles (fp32, d = 16, k <= 4, N <= 1024)."""
    from tarmac import _lib
    return _lib.LIB.tarmac_set_topk_filter(mode)


@pytest.fixture
def filter_always():
    prev = _set_filter(2)
    yield
    _set_filter(prev)



CASES = [
    (6, 16, 2), (6, 16, 1), (6, 8, 5), (2, 16, 1), (17, 16, 3), (32, 16, 1), (32, 16, 4),
    (64, 8, 2), (64, 32, 2), (100, 16, 2), (128, 64, 1), (256, 16, 1), (256, 16, 2),
    (256, 16, 4), (256, 32, 4), (384, 16, 2), (512, 16, 8), (512, 64, 3), (1024, 16, 2),
    (1024, 16, 7), (6, 128, 1), (64, 128, 2), (256, 128, 4), (300, 128, 8), (1024, 128, 1),
]


@pytest.mark.parametrize("mode", [0, 2, 3, 4, 5], ids=["packed", "filter", "lists", "split", "split32"])
@pytest.mark.parametrize("N,d,kk", CASES)
def test_fused_topk_f32_parity(N, d, kk, mode):
    B = max(2, min(16, 4096 // N))
    q, k, v = qkv(N * 131 + d * 17 + kk, B, N, d)
    prev = _set_filter(mode)
    try:
        out, idx = run_topk(q, k, v, kk)
    finally:
        _set_filter(prev)
    check_f32(q, k, v, kk, out, idx)


@pytest.mark.parametrize("tiles", [1, 2], ids=["one_tile", "two_tiles"])
@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("N,chunk", [(256, None), (1100, None), (700, 128)])
def test_d128_launch_shapes(N, chunk, dtype, tiles):
    """Head width 128 (msg_dim 65 .. 128 after the module's zero padding)
    under both query-tile launch shapes (forced: the automatic choice
    depends on the batch), on resident and streamed rows and rows of more
    than 1024 keys (several packing segments): indices bit-exact against the
    canonical oracle for k = 1, 2, 4, 8."""
    from tarmac import _lib
    B = 2
    q, k, v = qkv(13 * N + tiles, B, N, 128)
    prev = _lib.LIB.tarmac_set_query_tiles(tiles)
    try:
        for kk in (1, 2, 4, 8):
            if dtype == "fp32":
                out, idx = run_topk(q, k, v, kk, chunk)
                check_f32(q, k, v, kk, out, idx)
            else:
                out, idx = run_topk_bf16(q, k, v, kk, chunk)
                check_bf16_exact(q, k, v, kk, out, idx)
    finally:
        _lib.LIB.tarmac_set_query_tiles(prev)


@pytest.mark.parametrize("N,d,kk,chunk", [(256, 16, 2, 16), (256, 16, 4, 64), (300, 32, 1, 128),
                                          (1024, 16, 2, 256), (2048, 16, 1, 256), (300, 128, 2, 64),
                                          (1024, 128, 4, 128)])
def test_streaming_topk_matches_fused_bitwise(N, d, kk, chunk):
    B = 4
    q, k, v = qkv(7 * N + kk, B, N, d)
    out_s, idx_s = run_topk(q, k, v, kk, chunk=chunk)
    out_f, idx_f = run_topk(q, k, v, kk)
    assert np.array_equal(idx_s, idx_f)
    assert np.array_equal(out_s, out_f)
    check_f32(q, k, v, kk, out_s, idx_s)


@pytest.mark.parametrize("N,kk,chunk", [(256, 2, 16), (256, 4, 64), (256, 1, 128), (200, 3, 48),
                                        (256, 2, 80)])
def test_split32_streamed_matches_resident_bitwise(N, kk, chunk):
    """The 32 x 32 kernel (mode 5) over key chunks that start at any multiple
    of 16 keys (the self pair then straddles two 32-key tiles, and rows end
    inside a tile): identical indices and outputs to the resident row, and
    to the oracle."""
    B = 3
    q, k, v = qkv(11 * N + kk + chunk, B, N, 16)
    prev = _set_filter(5)
    try:
        out_s, idx_s = run_topk(q, k, v, kk, chunk=chunk)
        out_f, idx_f = run_topk(q, k, v, kk)
    finally:
        _set_filter(prev)
    assert np.array_equal(idx_s, idx_f)
    assert np.array_equal(out_s, out_f)
    check_f32(q, k, v, kk, out_s, idx_s)


@pytest.mark.parametrize("N,d,kk", [(12, 16, 11), (24, 8, 23), (64, 16, 9), (200, 32, 40),
                                    (300, 16, 299), (200, 128, 40), (600, 128, 12)])
def test_wide_k_parity(N, d, kk):
    q, k, v = qkv(N + 3 * kk, 3, N, d)
    out, idx = run_topk(q, k, v, kk)
    check_f32(q, k, v, kk, out, idx, exact_order=False)
    assert np.all(np.diff(idx, axis=-1) > 0)  # ascending index order above k = 8


def test_k_equal_n_minus_1_is_dense():
    from tarmac.kernels import fused_dense_attention, fused_topk_attention
    for N in (3, 6, 12, 24):
        q, k, v = qkv(N, 3, N, 16)
        qd, kd, vd = dev(q, k, v)
        a = fused_topk_attention(qd, kd, vd, N - 1)
        b = fused_dense_attention(qd, kd, vd)
        assert (a - b).abs().max().item() < 1e-6


def test_exact_ties_keep_lower_index():
    """Duplicate key rows give bit-identical scores; zero queries tie everything."""
    B, N, d = 4, 64, 16
    q, k, v = qkv(5, B, N, d)
    k[:, 1::2] = k[:, 0::2]        # keys 2j and 2j+1 identical
    q[:, 0] = 0.0                  # query 0: all scores +0 -> lowest indices 1, 2, ...
    for kk in (1, 2, 3, 4, 8):
        out, idx = run_topk(q, k, v, kk)
        check_f32(q, k, v, kk, out, idx)
        assert idx[:, 0].tolist() == [list(range(1, kk + 1))] * B


@pytest.mark.parametrize("N,d", [(256, 32), (300, 64), (200, 8), (256, 128)])
def test_exact_ties_fp32_wide_heads(N, d):
    """fp32 at d = 8, 32, 64 (the packed pass on fp32 MFMA scores for k >= 3):
    duplicated keys and zero queries leave the packed proof unsettled, and
    the per-query exact pass (key rows from the LDS copy) must return the
    canonical sets, ties to the lower index."""
    B = 3
    q, k, v = qkv(31 + N + d, B, N, d)
    k[:, 1::2] = k[:, 0::2]
    q[:, :6] = 0.0
    for kk in (3, 4, 8):
        out, idx = run_topk(q, k, v, kk)
        check_f32(q, k, v, kk, out, idx)
        assert idx[:, 0].tolist() == [list(range(1, kk + 1))] * B


def test_topk_clamp_and_default_tiling():
    from tarmac.kernels import (fused_topk_attention, fused_topk_attention_tiled,
                                streaming_topk_attention)
    q, k, v = qkv(11, 2, 6, 16)
    qd, kd, vd = dev(q, k, v)
    a = fused_topk_attention(qd, kd, vd, 99)     # clamped to N-1
    b = fused_topk_attention_tiled(qd, kd, vd, 5)
    c = fused_topk_attention(qd, kd, vd, 0)      # clamped to 1
    d_ = streaming_topk_attention(qd, kd, vd, 1)
    assert torch.equal(a, b) and torch.equal(c, d_)
    out, idx = streaming_topk_attention(qd, kd, vd, 2, return_indices=True)
    assert idx.dtype == torch.int32 and idx.shape == (2, 6, 2)


def test_headline_shape_properties():
    """B=1024, N=256, d=16, k=2 (the metric point): full-size properties, and
    a sample of batch rows against the canonical oracle."""
    B, N, d, kk = 1024, 256, 16, 2
    q, k, v = qkv(1234 + 7 * N + d, B, N, d)
    out, idx = run_topk(q, k, v, kk)
    assert np.isfinite(out).all()
    assert not np.any(idx == np.arange(N)[None, :, None])
    assert np.all(idx[..., 0] != idx[..., 1])
    rows = np.random.default_rng(0).choice(B, 48, replace=False)
    check_f32(q[rows], k[rows], v[rows], kk, out[rows], idx[rows])


@pytest.mark.parametrize("N,d,kk", [(64, 16, 1), (256, 16, 2), (256, 32, 4), (512, 64, 2),
                                    (100, 16, 3), (1024, 16, 1), (256, 64, 12), (6, 16, 2),
                                    (32, 16, 5), (17, 16, 8), (48, 16, 2), (256, 128, 2),
                                    (512, 128, 8), (64, 128, 12)])
def test_topk_bf16(N, d, kk):
    from tarmac.kernels import topk_attention
    B = 8
    q, k, v = qkv(77 + N + d, B, N, d)
    qb, kb, vb = (O.bf16_round(x) for x in (q, k, v))
    qd, kd, vd = dev(q, k, v, dtype=torch.bfloat16)
    out, idx = topk_attention(qd, kd, vd, kk, return_indices=True)
    torch.cuda.synchronize()
    out = out.float().cpu().numpy()
    idx = idx.cpu().numpy()
    check_bf16_exact(q, k, v, kk, out, idx)
    ref = O.prescore_attention(qb.astype(np.float64), kb.astype(np.float64),
                               vb.astype(np.float64), idx.astype(np.int64))
    assert np.abs(out - ref).max() <= BF16_TOL * np.abs(ref).max()


def run_topk_bf16(q, k, v, kk, chunk=None):
    from tarmac.kernels import topk_attention
    qd, kd, vd = dev(q, k, v, dtype=torch.bfloat16)
    out, idx = topk_attention(qd, kd, vd, kk, return_indices=True, key_chunk=chunk)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), idx.cpu().numpy()


def check_bf16_exact(q, k, v, kk, out, idx):
    """bf16 top-k selects the exact top k of the canonical fp32 scores of the
    inputs converted to fp32: indices bit-exact against the C oracle on the
    bf16-rounded inputs, outputs within 1e-2."""
    qb, kb, vb = (O.bf16_round(x) for x in (q, k, v))
    out_c, idx_c = O.canon_topk(qb, kb, vb, kk)
    if kk > 8:  # the large-k kernels emit ascending index order
        idx_c = np.sort(idx_c, -1)
    assert np.array_equal(idx, idx_c), "bf16 retained indices differ from the canonical oracle"
    assert np.abs(out - out_c).max() <= BF16_TOL * max(np.abs(out_c).max(), 1e-30)


@pytest.mark.parametrize("N,d", [(64, 16), (256, 32), (300, 64), (32, 16), (24, 16), (256, 128)])
def test_topk_bf16_exact_with_ties(N, d):
    """bf16 with exact ties (duplicated keys, zero and repeated queries): the
    retained set and its order are the canonical oracle's, ties to the lower
    index, on every k <= 8."""
    B = 4
    q, k, v = (O.bf16_round(x) for x in qkv(500 + N + d, B, N, d))
    k[:, 1::2] = k[:, 0::2]
    q[:, :5] = 0.0
    q[:, 5:10] = q[:, 5:6]
    for kk in (1, 2, 3, 4, 8):
        out, idx = run_topk_bf16(q, k, v, kk)
        check_bf16_exact(q, k, v, kk, out, idx)
        # zero queries tie every peer at +0: the lowest indices win
        assert idx[:, 0].tolist() == [list(range(1, kk + 1))] * B


CONFIGS2 = [(N, d, kk) for N in (64, 256, 512) for d in (16, 32, 64) for kk in (1, 2, 4)]


@pytest.mark.parametrize("N,d,kk", CONFIGS2)
def test_topk_bf16_configs2_exact(N, d, kk):
    """Every (N, d, k) cell of the bf16 grid: the retained set is the exact top
    k of the canonical fp32 scores of the bf16 inputs (bit-exact indices and
    order), outputs within 1e-2."""
    B = 8
    q, k, v = qkv(77 + N + d, B, N, d)
    out, idx = run_topk_bf16(q, k, v, kk)
    check_bf16_exact(q, k, v, kk, out, idx)


@pytest.mark.parametrize("N,d,kk,chunk", [(256, 16, 1, 64), (256, 16, 2, 16), (512, 32, 2, 128),
                                          (1024, 64, 2, 256), (700, 16, 3, 128), (1500, 16, 4, 256),
                                          (64, 16, 2, 16), (32, 16, 4, 16), (64, 32, 2, 32),
                                          (40, 64, 3, 16), (512, 128, 2, 128), (300, 128, 4, 64)])
def test_streaming_topk_bf16_matches_fused_bitwise(N, d, kk, chunk):
    """bf16: the streamed kernel (key chunks) returns exactly the resident
    kernel's indices and outputs, on every bf16 selection path."""
    B = 3
    q, k, v = qkv(5 * N + d + kk, B, N, d)
    out_s, idx_s = run_topk_bf16(q, k, v, kk, chunk)
    out_f, idx_f = run_topk_bf16(q, k, v, kk)
    assert np.array_equal(idx_s, idx_f)
    assert np.array_equal(out_s, out_f)


@pytest.mark.parametrize("N,kk,chunk", [(6, 2, None), (33, 4, None), (128, 1, None), (200, 3, None),
                                        (256, 2, None), (256, 4, None), (256, 2, 80), (256, 4, 16),
                                        (130, 3, 64), (256, 1, 128), (512, 4, None), (1024, 2, None),
                                        (1024, 4, 256), (700, 3, None)])
def test_bf16_split32_exact(N, kk, chunk):
    """bf16 heads at d = 16 on the 32 x 32 kernel (mode 5: one bf16 MFMA per
    tile, the bf16 accumulation bound in the proof): indices bit-exact against
    the canonical oracle on the bf16 inputs, resident and streamed (a
    streamed row equals the resident one bitwise), outputs within 1e-2."""
    B = 4
    q, k, v = qkv(71 * N + kk + (chunk or 0), B, N, 16)
    prev = _set_filter(5)
    try:
        out, idx = run_topk_bf16(q, k, v, kk, chunk)
        out_r, idx_r = run_topk_bf16(q, k, v, kk)
    finally:
        _set_filter(prev)
    check_bf16_exact(q, k, v, kk, out, idx)
    assert np.array_equal(idx, idx_r) and np.array_equal(out, out_r)


@pytest.mark.parametrize("N", [64, 256])
def test_bf16_split32_exact_with_ties(N):
    """The 32 x 32 bf16 kernel on exact ties (duplicated keys, zero and
    repeated queries): the canonical order, ties to the lower index."""
    B = 4
    q, k, v = (O.bf16_round(x) for x in qkv(900 + N, B, N, 16))
    k[:, 1::2] = k[:, 0::2]
    q[:, :5] = 0.0
    q[:, 5:10] = q[:, 5:6]
    prev = _set_filter(5)
    try:
        for kk in (1, 2, 3, 4):
            out, idx = run_topk_bf16(q, k, v, kk)
            check_bf16_exact(q, k, v, kk, out, idx)
            assert idx[:, 0].tolist() == [list(range(1, kk + 1))] * B
    finally:
        _set_filter(prev)


@pytest.mark.parametrize("N,kk,chunk", [(256, 4, None), (256, 8, None), (512, 5, None),
                                        (1024, 4, None), (700, 6, 128), (1500, 4, 256)])
def test_topk_bf16_filter_exact(N, kk, chunk):
    """bf16, d = 16, k >= 4, N >= 256 runs filter-and-verify by default: exact."""
    B = 4
    q, k, v = qkv(91 + 3 * N + kk, B, N, 16)
    out, idx = run_topk_bf16(q, k, v, kk, chunk)
    check_bf16_exact(q, k, v, kk, out, idx)


@pytest.mark.parametrize("N", [6, 64, 256, 1024])
def test_topk_bf16_filter_forced_exact_with_ties(N, filter_always):
    """Forced for every k at d = 16 (k <= 2 included), with duplicated keys,
    zero and repeated queries and near-tied key clusters: still exact."""
    B = 3
    q, k, v = (O.bf16_round(x) for x in qkv(300 + N, B, N, 16))
    k[:, 1::2] = k[:, 0::2]
    q[:, :8] = 0.0
    q[:, 8:16] = q[:, 8:9]
    rng = np.random.default_rng(N)
    for c0 in range(2, N - 20, 61):
        k[:, c0 + 1:c0 + 12] = O.bf16_round(k[:, c0:c0 + 1] * (1.0 + 2.0 ** -7 *
                                            rng.integers(-1, 2, (B, 11, 16))))
    for kk in (1, 2, 4, 8):
        if kk < N:
            out, idx = run_topk_bf16(q, k, v, kk)
            check_bf16_exact(q, k, v, kk, out, idx)


@pytest.mark.parametrize("N,d,kk,chunk", [(256, 16, 1, None), (256, 16, 2, None), (384, 32, 4, None),
                                          (512, 64, 8, None), (100, 16, 3, None),
                                          (1024, 16, 2, 256), (700, 32, 5, 128)])
def test_filter_path_matches_plain_fp32_path_bitwise(N, d, kk, chunk, filter_always):
    """The split-bf16 filter with exact verification returns exactly what the
    plain fp32 scoring pass returns (and both equal the canonical oracle)."""
    B = 6
    q, k, v = qkv(17 * N + kk, B, N, d)
    _set_filter(0)
    try:
        out_p, idx_p = run_topk(q, k, v, kk, chunk=chunk)
    finally:
        _set_filter(2)
    out_f, idx_f = run_topk(q, k, v, kk, chunk=chunk)
    assert np.array_equal(idx_f, idx_p)
    assert np.array_equal(out_f, out_p)
    check_f32(q, k, v, kk, out_f, idx_f)


@pytest.mark.parametrize("mode", [0, 2, 4], ids=["packed", "filter", "split"])
@pytest.mark.parametrize("N,chunk", [(256, None), (700, 128), (2048, None)])
def test_filter_fallback_on_ties(N, chunk, mode):
    """Duplicated keys and constant queries defeat the filter's proof; the
    fallback must still return the canonical answer (single-segment lists,
    chunked lists and lists spanning several 1024-key segments)."""
    B, d = 3, 16
    q, k, v = qkv(23 + N, B, N, d)
    k[:, 1::2] = k[:, 0::2]
    q[:, :40] = 0.0
    q[:, 40:80] = q[:, 40:41]
    prev = _set_filter(mode)
    try:
        for kk in (1, 2, 4, 8):
            out, idx = run_topk(q, k, v, kk, chunk=chunk)
            check_f32(q, k, v, kk, out, idx)
    finally:
        _set_filter(prev)


@pytest.mark.parametrize("mode", [0, 2, 4], ids=["packed", "filter", "split"])
@pytest.mark.parametrize("N,kk,chunk", [(256, 2, None), (512, 8, None), (1500, 3, 256)])
def test_filter_near_ties(N, kk, chunk, mode):
    """Clusters of keys whose scores agree to ~1e-6 relative: candidates that
    share their truncated filter score, lists that must be re-sorted after
    repacking, and proofs that fail on purpose."""
    B, d = 3, 16
    q, k, v = qkv(91 + N + kk, B, N, d)
    rng = np.random.default_rng(N)
    for c0 in range(0, N - 40, 97):
        k[:, c0 + 1:c0 + 40] = k[:, c0:c0 + 1] * 3.0 + 1e-6 * rng.standard_normal((B, 39, d))
    prev = _set_filter(mode)
    try:
        out, idx = run_topk(q, k, v, kk, chunk=chunk)
    finally:
        _set_filter(prev)
    check_f32(q, k, v, kk, out, idx)


# ---------------------------------------------------------------------------
# the reference's other resident selection rules (masked bisection, sort)
# ---------------------------------------------------------------------------

def _variant_inputs(seed, B, N, d, ties):
    q, k, v = qkv(seed, B, N, d)
    if ties:
        k[:, 1::2] = k[:, 0:2 * (N // 2):2]  # every score tied in pairs
        q[:, :N // 4] = 0.0              # and whole rows of +0 scores
    return q, k, v


@pytest.mark.parametrize("N,d,kk,ties", [(6, 16, 2, False), (24, 16, 3, True), (100, 32, 4, False),
                                         (256, 16, 2, True), (256, 64, 8, False), (513, 16, 5, True),
                                         (1024, 16, 1, True), (1024, 64, 7, True), (300, 128, 4, True)])
@pytest.mark.parametrize("bisect", [34, 32, 20, 5, 0])
def test_masked_variant_matches_bisection_oracle(N, d, kk, ties, bisect):
    """fused_topk_attention_masked: the kept set is the reference's bisection
    step for step (on the canonical fp32 scores), so outputs match the float64
    softmax over exactly that set."""
    from tarmac.kernels import fused_topk_attention_masked
    B = 3
    q, k, v = _variant_inputs(N + kk + bisect, B, N, d, ties)
    qd, kd, vd = dev(q, k, v)
    out = fused_topk_attention_masked(qd, kd, vd, kk, bisect=bisect)
    torch.cuda.synchronize()
    s = O.canon_scores(q, k)
    keep = O.masked_threshold_keep(s, kk, bisect)
    ref = O.weights_attention(s, keep, v)
    assert np.abs(out.cpu().numpy() - ref).max() <= F32_TOL * np.abs(ref).max()


@pytest.mark.parametrize("N,d,kk,ties", [(6, 16, 2, True), (24, 8, 5, True), (100, 32, 4, False),
                                         (256, 16, 2, True), (256, 64, 8, True), (300, 16, 12, True),
                                         (1024, 16, 3, True), (1024, 32, 8, True), (300, 128, 6, True)])
def test_sort_variant_keeps_higher_index_on_ties(N, d, kk, ties):
    from tarmac.kernels import fused_topk_attention_sort, topk_variant_attention
    from tarmac import _lib
    B = 3
    q, k, v = _variant_inputs(7 * N + kk, B, N, d, ties)
    qd, kd, vd = dev(q, k, v)
    out, idx = topk_variant_attention(qd, kd, vd, kk, _lib.VARIANT_SORT, return_indices=True)
    out2 = fused_topk_attention_sort(qd, kd, vd, kk)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    s = O.canon_scores(q, k)
    want = O.sort_select(s, kk)
    assert np.array_equal(idx.cpu().numpy(), np.sort(want, -1))
    keep = np.zeros_like(s, dtype=bool)
    np.put_along_axis(keep, want, True, -1)
    ref = O.weights_attention(s, keep, v)
    assert np.abs(out.cpu().numpy() - ref).max() <= F32_TOL * np.abs(ref).max()
    if ties:  # the tie rule is visible: rows of +0 scores keep the top indices
        assert np.all(idx.cpu().numpy()[:, 0] == np.arange(N - kk, N))


@pytest.mark.parametrize("N,d,kk,ties", [(6, 16, 2, False), (24, 16, 3, True), (256, 16, 2, True),
                                         (256, 64, 8, False), (300, 32, 12, True),
                                         (1024, 16, 4, True), (256, 128, 3, True)])
@pytest.mark.parametrize("rule", ["masked34", "masked32", "masked20", "masked5", "sort"])
def test_bf16_variants_match_oracle(N, d, kk, ties, rule):
    """bf16 heads: the masked and sort rules on the canonical fp32 scores of
    the bf16 values (the list kernel on widened copies for sort / masked with
    >= 32 halvings at k <= 8, the wide kernels otherwise), outputs within 1e-2
    of the float64 softmax over the oracle's kept set; sort indices
    bit-exact."""
    from tarmac import _lib
    from tarmac.kernels import topk_variant_attention
    B = 3
    q, k, v = (O.bf16_round(x) for x in _variant_inputs(5 * N + kk, B, N, d, ties))
    qd, kd, vd = dev(q, k, v, dtype=torch.bfloat16)
    s = O.canon_scores(q, k)
    if rule == "sort":
        out, idx = topk_variant_attention(qd, kd, vd, kk, _lib.VARIANT_SORT, return_indices=True)
        want = O.sort_select(s, kk)
        assert np.array_equal(idx.cpu().numpy(), np.sort(want, -1))
        keep = np.zeros_like(s, dtype=bool)
        np.put_along_axis(keep, want, True, -1)
    else:
        bis = int(rule[6:])
        out = topk_variant_attention(qd, kd, vd, kk, _lib.VARIANT_MASKED, bis)
        keep = O.masked_threshold_keep(s, kk, bis)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    ref = O.weights_attention(s, keep, v)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= BF16_TOL * np.abs(ref).max()


@pytest.mark.parametrize("variant", ["masked", "sort"])
def test_variants_nonfinite_inputs(variant):
    """An infinite key element (batch row 0) and an infinite query element
    (batch row 1): scores of +-inf, no NaN (each infinite element is the first
    of its fmaf chain). The rules rank them by integer key like any score;
    kept sets bit-exact (sort indices), NaN rows where an infinite score is
    kept (inf - inf in the softmax), the other rows within 1e-5."""
    from tarmac.kernels import topk_variant_attention
    from tarmac import _lib
    B, N, d, kk = 2, 256, 16, 3
    q, k, v = qkv(91, B, N, d)
    k[0, 37, 0] = np.inf
    q[1, 9, 0] = -np.inf
    qd, kd, vd = dev(q, k, v)
    s = O.canon_scores(q, k)
    assert not np.isnan(s).any()
    if variant == "sort":
        out, idx = topk_variant_attention(qd, kd, vd, kk, _lib.VARIANT_SORT, return_indices=True)
        want = O.sort_select(s, kk)
        assert np.array_equal(idx.cpu().numpy(), np.sort(want, -1))
        keep = np.zeros_like(s, dtype=bool)
        np.put_along_axis(keep, want, True, -1)
    else:
        out = topk_variant_attention(qd, kd, vd, kk, _lib.VARIANT_MASKED)
        keep = O.masked_threshold_keep(s, kk, 34)
    with np.errstate(invalid="ignore"):
        ref = O.weights_attention(s, keep, v)
    got = out.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.isnan(ref).any()
    fin = ~np.isnan(ref)
    assert np.abs(got[fin] - ref[fin]).max() <= F32_TOL * np.abs(ref[fin]).max()


def test_variants_equal_topk_without_ties():
    from tarmac.kernels import (fused_topk_attention, fused_topk_attention_masked,
                                fused_topk_attention_sort)
    q, k, v = qkv(4321, 4, 128, 16)
    qd, kd, vd = dev(q, k, v)
    for kk in (1, 2, 4):
        a = fused_topk_attention(qd, kd, vd, kk)
        b = fused_topk_attention_masked(qd, kd, vd, kk)
        c = fused_topk_attention_sort(qd, kd, vd, kk)
        assert (a - b).abs().max().item() <= 1e-6 and (a - c).abs().max().item() <= 1e-6


def test_variant_argument_errors():
    from tarmac.kernels import topk_variant_attention
    from tarmac import _lib
    q, k, v = dev(*qkv(1, 2, 16, 16))
    with pytest.raises(ValueError, match="idx_out must be NULL"):
        topk_variant_attention(q, k, v, 2, _lib.VARIANT_MASKED, return_indices=True)
    with pytest.raises(ValueError, match="variant"):
        topk_variant_attention(q, k, v, 2, 7)
    with pytest.raises(ValueError, match="bisect"):
        topk_variant_attention(q, k, v, 2, _lib.VARIANT_MASKED, bisect=-1)


def test_empty_batch_returns_empty_outputs():
    """B = 0: every entry point returns correctly shaped empty outputs (as the
    reference's torch compositions do) without launching anything."""
    from tarmac.kernels import (fused_dense_attention, fused_prescore_attention,
                                fused_topk_attention_masked, fused_topk_attention_sort,
                                select_grid_knn, select_morton_window, select_radius_knn,
                                zorder_attention)
    from tarmac.kernels.backward import (dense_attention_backward,
                                         dense_attention_forward_stats,
                                         fixedset_attention_backward)
    from tarmac.kernels.prescore_selection import _morton_code
    q = torch.zeros(0, 6, 16, device="cuda")
    pos = torch.zeros(0, 6, 2, device="cuda")
    idx = torch.zeros(0, 6, 2, dtype=torch.int32, device="cuda")
    from tarmac.kernels import topk_attention
    out, ix = topk_attention(q, q, q, 2, return_indices=True)
    assert out.shape == (0, 6, 16) and ix.shape == (0, 6, 2)
    assert topk_attention(q, q, q, 2, key_chunk=64).shape == (0, 6, 16)
    assert fused_dense_attention(q, q, q).shape == (0, 6, 16)
    assert fused_topk_attention_masked(q, q, q, 2).shape == (0, 6, 16)
    assert fused_topk_attention_sort(q, q, q, 2).shape == (0, 6, 16)
    assert fused_prescore_attention(q, q, q, idx).shape == (0, 6, 16)
    assert zorder_attention(q, q, q, pos, 2, 16).shape == (0, 6, 16)
    assert select_morton_window(pos, 2).shape == (0, 6, 2)
    assert _morton_code(pos).shape == (0, 6)
    assert select_radius_knn(pos, 2).shape == (0, 6, 2)
    assert select_grid_knn(pos, 2).shape == (0, 6, 2)
    o, st = dense_attention_forward_stats(q, q, q)
    assert o.shape == (0, 6, 16) and st.shape == (0, 2, 6)
    assert all(t.shape == (0, 6, 16) for t in dense_attention_backward(q, q, q, o, q, st))
    assert all(t.shape == (0, 6, 16) for t in fixedset_attention_backward(q, q, q, idx, q))
    torch.cuda.synchronize()


@pytest.mark.parametrize("N,d,kk", [(6, 16, 2), (256, 16, 2), (300, 8, 4), (512, 64, 12), (96, 32, 23),
                                    (256, 128, 4)])
def test_float16_inputs(N, d, kk):
    """float16 heads run the fp32 kernels on exact fp32 copies: retained
    indices bit-exact against the canonical C oracle on the float16 values,
    outputs float16 within 2e-3 of max|ref| (one rounding of the fp32
    result), for top-k (resident and streamed), dense, fixed-set and
    Z-order."""
    from tarmac.kernels import (fused_dense_attention, fused_prescore_attention,
                                topk_attention, zorder_attention)
    B = 3
    q, k, v = (x.astype(np.float16).astype(np.float32) for x in qkv(N + 3 * d + kk, B, N, d))
    qd, kd, vd = dev(q, k, v, dtype=torch.float16)
    want, idx_c = O.canon_topk(q, k, v, kk)
    out, idx = topk_attention(qd, kd, vd, kk, return_indices=True)
    out_s, idx_s = topk_attention(qd, kd, vd, kk, return_indices=True, key_chunk=64)
    dense = fused_dense_attention(qd, kd, vd)
    fixed = fused_prescore_attention(qd, kd, vd, idx)
    pos = np.random.default_rng(N).random((B, N, 2)).astype(np.float32)
    zo, zidx = zorder_attention(qd, kd, vd, torch.from_numpy(pos).cuda(), kk, 10,
                                return_indices=True)
    torch.cuda.synchronize()
    assert all(t.dtype == torch.float16 for t in (out, out_s, dense, fixed, zo))
    if kk > 8:  # k > 8 returns each set in ascending index order
        idx_c = np.sort(idx_c, -1)
    assert np.array_equal(idx.cpu().numpy(), idx_c)
    assert np.array_equal(idx_s.cpu().numpy(), idx_c)

    def close(got, ref):
        assert np.abs(got.float().cpu().numpy() - ref).max() <= 2e-3 * np.abs(ref).max()

    close(out, want)
    close(out_s, want)
    close(fixed, want)
    close(dense, O.dense_unfused(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64)))
    zi = zidx.cpu().numpy()
    assert np.array_equal(zi, O.canon_morton_window(pos, kk, 10))
    close(zo, O.prescore_attention(q.astype(np.float64), k.astype(np.float64),
                                   v.astype(np.float64), zi.astype(np.int64)))
