"""Pins for the serving-router oracle (oracle/route_oracle.py), CPU only.

The reference ships no tests or vectors for route_triton.py, so the oracle's
restatement of _entmax_kernel is checked against what the mathematics fixes:
* tau: the 24-step bisection lands within its resolution (2^-24 of the [-1, 0]
  interval, plus fp32 rounding) of the exact 1.5-entmax threshold from the
  sort-based closed form (Peters, Niculae & Martins 2019), computed here in
  pure Python;
* budget: with well separated z the active set is exactly the top-K by
  sorting; with a tie at the K-th / (K+1)-th place the bisection keeps only the
  values strictly above the tie (fewer than K);
* bias: mean over the active blocks is 0 and the spread scales with 1/sigma;
* packing: ascending block ids, -1 / 0 fill, slots >= M untouched;
* the page-mask fallback, window bounds, plans and the prefill row map by
  direct enumeration.
"""

import math

import numpy as np
import pytest

from oracle import route_oracle as RO


def _entmax_tau_exact(z):
    """Exact tau of sum max(z - tau, 0)^2 = 1 by the sorted closed form (pure Python)."""
    zs = sorted(z, reverse=True)
    for k in range(1, len(zs) + 1):
        m = sum(zs[:k]) / k
        ss = sum(v * v for v in zs[:k]) / k - m * m
        d = (1 - k * ss) / k
        if d < 0:
            break
        tau = m - math.sqrt(d)
        if k == len(zs) or zs[k] <= tau:
            if zs[k - 1] > tau:
                return tau
    raise AssertionError("no threshold")


def _z(s, idx_scale, cand):
    x = [v * idx_scale for v, c in zip(s, cand) if c]
    xm = max(x)
    return [(v - xm) * 0.5 for v in x]


@pytest.mark.parametrize("seed", range(6))
def test_tau_matches_closed_form(seed):
    rng = np.random.default_rng(seed)
    W = int(rng.integers(5, 300))
    s = rng.standard_normal(W).astype(np.float32) * np.float32(rng.uniform(0.1, 3))
    s[rng.random(W) < 0.3] = RO.SCORE_NEG
    s[0] = 0.5
    idx_scale = float(rng.uniform(0.2, 4))
    _, _, tau = RO.entmax_row(s, None, idx_scale, 1e-4, 1.0, K=W)
    cand = [v > -5e8 for v in s.tolist()]
    exact = _entmax_tau_exact(_z([float(v) for v in s], float(np.float32(idx_scale)), cand))
    assert abs(float(tau) - exact) <= 2.0 ** -23, (float(tau), exact)


def test_budget_is_top_k_and_ties_keep_fewer():
    rng = np.random.default_rng(7)
    W, K = 200, 12
    s = rng.permutation(W).astype(np.float32) * np.float32(0.01)        # distinct, well separated
    ids, _, _ = RO.entmax_row(s, None, 1.0, 1e-4, 1.0, K=K)
    assert ids.tolist() == sorted(np.argsort(-s)[:K].tolist())
    # the K-th and (K+1)-th values tied: only the values strictly above survive
    t = np.sort(s)[::-1].copy()
    s2 = s.copy()
    s2[s2 == t[K]] = t[K - 1]
    ids2, _, _ = RO.entmax_row(s2, None, 1.0, 1e-4, 1.0, K=K)
    assert ids2.tolist() == sorted(np.argsort(-s2)[:K - 1].tolist())
    # no more candidates than K: every candidate is active
    s3 = np.full(W, RO.SCORE_NEG)
    s3[[3, 50, 120]] = [1.0, 2.0, 3.0]
    ids3, _, _ = RO.entmax_row(s3, None, 1.0, 1e-4, 1.0, K=K)
    assert ids3.tolist() == [3, 50, 120]


def test_bias_centred_and_scaled_by_inverse_sigma():
    rng = np.random.default_rng(8)
    s = rng.standard_normal(64).astype(np.float32)
    _, b1, _ = RO.entmax_row(s, None, 2.0, 1e-3, 1.0, K=9)
    _, b2, _ = RO.entmax_row(s, None, 2.0, 1e-3, 1.0 / 0.4, K=9)
    assert abs(float(np.mean(b1.astype(np.float64)))) < 1e-5
    assert np.allclose(b2, b1 / 0.4, rtol=1e-5, atol=1e-6)
    # a floor above every prior makes every bias 0
    _, b3, _ = RO.entmax_row(s, None, 2.0, 2.0, 1.0, K=9)
    assert np.all(b3 == 0)


def test_page_mask_fallback_and_packing():
    W, M = 40, 8
    s = np.linspace(-1, 1, W).astype(np.float32)
    img = np.zeros((2, W), bool)
    img[0, [5, 7, 30]] = True              # row 0: three allowed candidates
    sc = np.stack([s, s])                  # row 1: mask empty -> every remote block
    out_i = np.full((2, M + 2), 77, np.int32)
    out_b = np.full((2, M + 2), 5.0, np.float32)
    RO.route_entmax(sc, img, out_i, out_b, idx_scale=1.0, prior_floor=1e-4, inv_sigma=1.0, K=6, M=M)
    assert out_i[0, :3].tolist() == [5, 7, 30] and (out_i[0, 3:M] == -1).all() and (out_b[0, 3:M] == 0).all()
    assert out_i[1, :6].tolist() == sorted(np.argsort(-s)[:6].tolist())
    assert (out_i[:, M:] == 77).all() and (out_b[:, M:] == 5.0).all()     # slots >= M untouched


def test_win_bounds_enumeration():
    allow = np.zeros((4, 50), np.int8)
    allow[0, [3, 9, 40]] = 1                      # 40 is past the remote bound
    seq = np.array([1000, 1000, 10, 0])
    lo, hi, fit = RO.win_bounds(allow, seq, max_block=48, block_size=32, local_blocks=4, dql=1, tile=4)
    # row 0: q_blk 31, remote <= 27: allowed {3, 9}
    assert (lo[0], hi[0], fit[0]) == (3, 10, 0)
    # row 1: nothing allowed -> the live remote width, min(48, ceil(1000 / 32) = 32)
    assert (lo[1], hi[1]) == (0, 32)
    # rows 2, 3: no remote block at all
    assert (lo[2], hi[2], fit[2]) == (0, 0, 1) and (lo[3], hi[3]) == (0, 0)


def test_plans_and_row_map():
    bt = np.arange(20).reshape(2, 10) + 100
    pages, tok = RO.tail_plan(bt, [70, 10], 32, 2)
    assert pages.tolist() == [102, 101, 110, 110] and tok.tolist() == [6, 32, 10, 10]
    pages, tok = RO.all_plan(bt, [70, 10], [40, 0], 32, 10, 40)
    assert pages.tolist() == [101, 102, 103, 110, 111, 112] and tok.tolist() == [32, 6, 0, 10, 0, 0]
    rq, pos = RO.prefill_rows([0, 2, 2, 5], [10, 7, 3])
    assert rq.tolist() == [0, 0, 2, 2, 2] and pos.tolist() == [10, 11, 3, 4, 5]
