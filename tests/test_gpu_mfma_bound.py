"""The accumulation bound the exact bf16 / split-bf16 top-k proofs rest on.

The packed and filter top-k kernels score on bf16 MFMA (exact products, fp32
accumulation) and prove their retained set against an error bound
E = eps(d) |q| max_j |k_j| (``packed_eps`` / ``filter_eps``: 2^-18 at d <= 32,
2^-17 at d = 64). E must cover, relative to sum_c |q_c k_c| <= |q| |k_j|:

* the MFMA's accumulation error, measured here on this device
  (``tarmac_mfma_bf16_probe``) against exact float64 sums, on random,
  same-sign, mixed-magnitude, cancelling and one-dominant-product operands,
  chained over one to four 16x16x32 instructions (d = 32, 64, 128 and the 96
  products of a split-bf16 score at d = 16 on 16 x 16 tiles) and one to six
  32x32x16 instructions (the 32 x 32 split kernel chains six): the bound
  asserted is 2^-20.25 (the worst case seen is about 2^-20.5, one dominant
  product among small ones);
* the canonical fmaf chain's error, at most d 2^-24 (one rounding per step);
* for split-bf16 scores, the dropped products (mid.lo, lo.mid, lo.lo, each
  at most 2^-24 of |q_c k_c|).

The margins (eps over the sum) are asserted too, and the top-k kernels are
run on inputs built like the worst accumulation case (one dominant
coordinate, the ranking decided by small products) with indices required
bit-exact against the canonical C oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import tarmac_oracle as O

pytestmark = pytest.mark.gpu

MFMA_ACC_BOUND = 2.0 ** -20.25  # relative to the sum of |products|
EPS = {16: 2.0 ** -18, 32: 2.0 ** -18, 64: 2.0 ** -17, 128: 2.0 ** -16}  # packed_eps / filter_eps


def _bf16_bits(x):
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def _bits_f64(b):
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _mfma_rel_error(Am, Bm, shape=16):
    """shape 16: Am [T, chain, 16, 32], Bm [T, chain, 32, 16]; shape 32:
    Am [T, chain, 32, 16], Bm [T, chain, 16, 32] (float32, rounded to bf16):
    max over outputs of |MFMA - exact| / sum |products|."""
    from tarmac import _lib
    T, chain = Am.shape[:2]
    M = Am.shape[2]  # 16 or 32 rows (= columns) of the result
    Ab, Bb = _bf16_bits(Am), _bf16_bits(Bm)
    la = np.zeros((T, chain, 64, 8), np.uint16)
    lb = np.zeros((T, chain, 64, 8), np.uint16)
    for lane in range(64):
        i, g = lane % M, lane // M
        la[:, :, lane, :] = Ab[:, :, i, 8 * g:8 * g + 8]
        lb[:, :, lane, :] = Bb[:, :, 8 * g:8 * g + 8, i]
    da = torch.from_numpy(la.view(np.int16)).cuda()
    db = torch.from_numpy(lb.view(np.int16)).cuda()
    per = 4 if shape == 16 else 16
    out = torch.zeros(T, 64, per, device="cuda")
    rc = _lib.LIB.tarmac_mfma_bf16_probe(da.data_ptr(), db.data_ptr(), out.data_ptr(), T, chain,
                                         shape, None)
    _lib.check(rc)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    got = np.zeros((T, M, M))
    for lane in range(64):
        j, g = lane % M, lane // M
        for r in range(per):
            row = 4 * g + r if shape == 16 else 8 * (r // 4) + 4 * g + r % 4
            got[:, row, j] = o[:, lane, r]
    Af, Bf = _bits_f64(Ab), _bits_f64(Bb)
    exact = np.einsum("tcik,tckj->tij", Af, Bf)
    mag = np.einsum("tcik,tckj->tij", np.abs(Af), np.abs(Bf))
    return float((np.abs(got - exact) / np.maximum(mag, 1e-300)).max())


PATTERNS = {
    "normal": lambda g, s: g.standard_normal(s),
    "same_sign": lambda g, s: 1.0 + g.random(s),
    "mixed_magnitude": lambda g, s: g.standard_normal(s) * 2.0 ** g.integers(-20, 20, s),
    "one_dominant": lambda g, s: np.where(g.random(s) < 0.03, 2.0 ** 12, 1.0 + g.random(s)),
    "cancelling": lambda g, s: np.where(g.random(s) < 0.5, 1.0, -1.0) * (1.0 + 2.0 ** -7 * g.integers(0, 128, s)),
}


@pytest.mark.parametrize("shape,chain", [(16, 1), (16, 2), (16, 3), (16, 4), (32, 1), (32, 2),
                                         (32, 6)])
@pytest.mark.parametrize("pattern", list(PATTERNS))
def test_mfma_accumulation_error_within_bound(pattern, shape, chain):
    g = np.random.default_rng(10 * list(PATTERNS).index(pattern) + chain + shape)
    T = 1024 if shape == 16 else 256
    rows, inner = (16, 32) if shape == 16 else (32, 16)
    Am = PATTERNS[pattern](g, (T, chain, rows, inner)).astype(np.float32)
    Bm = PATTERNS[pattern](g, (T, chain, inner, rows)).astype(np.float32)
    err = _mfma_rel_error(Am, Bm, shape)
    assert err <= MFMA_ACC_BOUND, f"MFMA accumulation error {err:.3e} above the bound"


def test_proof_margins_cover_the_error_sources():
    """eps(d) against the sum of the sources it must cover, with margin."""
    for d, eps in EPS.items():
        canonical = d * 2.0 ** -24
        assert canonical + MFMA_ACC_BOUND <= eps / 1.25, d
    # split-bf16 scores (fp32 inputs, d = 16): three instructions of products
    # whose magnitudes sum to at most 1 + 2^-7 times sum |q_c k_c|, and three
    # dropped products of at most 2^-24 each
    split = 16 * 2.0 ** -24 + MFMA_ACC_BOUND * (1 + 2.0 ** -7) + 3 * 2.0 ** -24
    assert split <= EPS[16] / 1.25


@pytest.mark.parametrize("mode", [1, 4, 5], ids=["auto", "split16", "split32"])
@pytest.mark.parametrize("d", [16, 32, 64, 128])
@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_topk_exact_on_one_dominant_coordinate(d, dtype, mode):
    """Every score carries one dominant product (q_0 k_0 = 4096) and the
    ranking is decided by the small ones: the accumulation pattern with the
    largest MFMA error. Retained indices bit-exact against the canonical
    oracle (bf16: on the bf16 inputs; fp32 d = 16 runs the split-bf16 pass
    on 16 x 16 tiles (mode 4) and on 32 x 32 tiles (mode 5), bf16 d = 16
    the 32 x 32 kernel's single-product form (mode 5))."""
    from tarmac import _lib
    from tarmac.kernels import topk_attention
    if dtype == "fp32" and d != 16:
        pytest.skip("split-bf16 scoring serves fp32 at d = 16")
    if mode == 4 and not (dtype == "fp32" and d == 16):
        pytest.skip("mode 4 selects the split-bf16 16 x 16 kernel (fp32, d = 16)")
    if mode == 5 and d != 16:
        pytest.skip("mode 5 selects the 32 x 32 kernel (d = 16)")
    B, N = 8, 256
    g = np.random.default_rng(d)
    q = g.standard_normal((B, N, d)).astype(np.float32) / 8
    k = g.standard_normal((B, N, d)).astype(np.float32) / 8
    v = g.standard_normal((B, N, d)).astype(np.float32)
    q[..., 0] = 64.0
    k[..., 0] = 64.0
    if dtype == "bf16":
        q, k, v = (O.bf16_round(x) for x in (q, k, v))
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    qd, kd, vd = (torch.from_numpy(x).cuda().to(tdt) for x in (q, k, v))
    prev = _lib.LIB.tarmac_set_topk_filter(mode)
    try:
        for kk in (1, 2, 4):
            out, idx = topk_attention(qd, kd, vd, kk, return_indices=True)
            torch.cuda.synchronize()
            _, idx_c = O.canon_topk(q, k, v, kk)
            assert np.array_equal(idx.cpu().numpy(), idx_c), f"k={kk}: indices differ from the oracle"
    finally:
        _lib.LIB.tarmac_set_topk_filter(prev)
