"""Serving DASH router oracle -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/`` may import this module, as the checker.  It restates, on the
CPU in numpy fp32 arithmetic, the serving router of the reference's SGLang
backend (WHL!layers/attention/unlimited_dash_ops/route_triton.py, WHL!p:N =
``sglang/srt/p`` line N inside the reference's SGLang wheel):

* ``route_entmax``  -- ``_entmax_kernel`` (:129-221), literally: the 24-step
  tau bisection and the 40-step budget bisection that counts the candidates
  above each midpoint.  Sums the reference takes in fp64 are taken exactly
  (``math.fsum``) and rounded once to fp32, the value an fp64 sum approximates.
* ``win_bounds``    -- ``_win_bounds_kernel`` (:466-505).
* ``tail_plan`` / ``all_plan`` / ``row2req`` -- ``kbar_tail_plan`` (:681-703),
  ``kbar_all_plan`` (:575-601), ``prefill_row2req`` (:604-620).
* ``prefill_rows``  -- the row -> (request, position) map of
  ``_score_prefill_kernel`` (:541-549).

The scores themselves are ``srswa_oracle.kbar_scores`` and the summaries
``srswa_oracle.kbar_summaries``.  Pins: ``tests/test_route_pins.py`` (the tau
bisection against the sort-based closed form of 1.5-entmax, the budget against
sorting, the centring and 1/sigma of the bias, the packing).
"""

from __future__ import annotations

import math

import numpy as np

SCORE_NEG = np.float32(-1.0e9)
ENTMAX_NEG = np.float32(-1.0e4)
ENTMAX_ITERS = 24
ENTMAX_ITERS_CAP = 40
F32 = np.float32


def _fsum32(v) -> np.float32:
    """fp32 rounding of the exact sum of fp32 values."""
    return F32(math.fsum(np.asarray(v, np.float64).tolist()))


def entmax_row(s, img, idx_scale, prior_floor, inv_sigma, K):
    """One row of ``_entmax_kernel``: s fp32 [W] scores (SCORE_NEG = not a
    remote block), img [W] bool page mask or None.  Returns (active ids
    ascending, their fp32 biases, tau)."""
    s = np.asarray(s, np.float32)
    idx_scale, prior_floor, inv_sigma = F32(idx_scale), F32(prior_floor), F32(inv_sigma)
    with np.errstate(invalid="ignore"):
        remote = s > SCORE_NEG * F32(0.5)
    cand = remote
    if img is not None:
        ci = remote & (np.asarray(img) != 0)
        if ci.sum() > 0:
            cand = ci
    has_any = bool(cand.any())
    with np.errstate(invalid="ignore", over="ignore"):
        x = np.where(cand, s * idx_scale, ENTMAX_NEG).astype(np.float32)
    x = np.where(np.isnan(x), ENTMAX_NEG, x).astype(np.float32)
    xm = F32(x[cand].max()) if has_any else F32(0.0)
    z = ((x - xm) * F32(0.5)).astype(np.float32)

    lo, hi = F32(-1.0), F32(0.0)
    for _ in range(ENTMAX_ITERS):
        mid = F32((lo + hi) * F32(0.5))
        p = np.maximum(z - mid, F32(0.0)).astype(np.float32)
        ssum = _fsum32((p * p)[cand])
        if ssum > F32(1.0):
            lo = mid
        else:
            hi = mid
    tau = F32((lo + hi) * F32(0.5))
    prior = np.maximum(z - tau, F32(0.0)).astype(np.float32)
    prior = (prior * prior).astype(np.float32)

    active = cand
    if int(cand.sum()) > int(K):
        lo2 = F32(z[cand].min() - F32(1.0)) if has_any else F32(-1.0)
        hi2 = F32(0.0)
        for _ in range(ENTMAX_ITERS_CAP):
            mid = F32((lo2 + hi2) * F32(0.5))
            cnt = int((cand & (z > mid)).sum())
            if cnt > int(K):
                lo2 = mid
            else:
                hi2 = mid
        active = cand & (z > hi2)
    logp = np.log(np.maximum(prior, prior_floor)).astype(np.float32)
    cnt_a = max(int(active.sum()), 1)
    mu = F32(_fsum32(logp[active]) / F32(cnt_a))
    bias = ((logp - mu) * inv_sigma).astype(np.float32)
    ids = np.nonzero(active)[0]
    return ids, bias[ids], tau


def route_entmax(scores, img, out_idx, out_bias, *, idx_scale, prior_floor, inv_sigma, K, M):
    """All rows: writes the first M slots of out_idx (int32) / out_bias (fp32)
    in place (active ids ascending, -1 / 0 in the rest), as the kernel does;
    returns them."""
    scores = np.asarray(scores, np.float32)
    for r in range(scores.shape[0]):
        ids, b, _ = entmax_row(scores[r], None if img is None else img[r], idx_scale, prior_floor, inv_sigma, K)
        n = min(len(ids), M)
        out_idx[r, :M] = -1
        out_bias[r, :M] = 0.0
        out_idx[r, :n] = ids[:n]
        out_bias[r, :n] = b[:n]
    return out_idx, out_bias


def win_bounds(allow, seq_lens, *, max_block, block_size, local_blocks, dql, tile):
    """``_win_bounds_kernel``: per decode row (lo, hi, fit) of the allowed live
    remote blocks (numpy int arrays)."""
    allow = np.asarray(allow)
    nd, WQ = allow.shape
    W = int(max_block)
    lo = np.zeros(nd, np.int32)
    hi = np.zeros(nd, np.int32)
    fit = np.zeros(nd, np.int8)
    for row in range(nd):
        seq = int(seq_lens[row // dql])
        q_pos = seq - dql + row % dql
        q_blk = int(q_pos / block_size)                  # truncation, as the kernel's integer division
        keep = [j for j in range(min(W, WQ))
                if allow[row, j] != 0 and j <= q_blk - local_blocks and j * block_size < seq]
        if keep:
            lo_v, hi_v = keep[0], keep[-1] + 1
        else:
            n_blk = -(-seq // block_size) if seq > 0 else 0
            no_remote = seq <= 0 or q_blk - local_blocks < 0
            lo_v, hi_v = 0, (0 if no_remote else min(W, max(n_blk, 1)))
        lo[row], hi[row], fit[row] = lo_v, hi_v, int(hi_v - lo_v <= tile)
    return lo, hi, fit


def tail_plan(block_table, seq_lens, block_size, tail_pages):
    """``kbar_tail_plan``: (pages, tok) of each request's last tail_pages blocks."""
    pages, tok = [], []
    w = block_table.shape[1]
    for r in range(block_table.shape[0]):
        sl = int(seq_lens[r])
        last = max(-(-sl // block_size) - 1, 0)
        for t in range(tail_pages):
            b = max(last - t, 0)
            pages.append(int(block_table[r, min(b, w - 1)]))
            tok.append(min(max(sl - b * block_size, 0), block_size))
    return np.array(pages, np.int64), np.array(tok, np.int32)


def all_plan(block_table, seq_lens, context_lens, block_size, max_block, max_query_len):
    """``kbar_all_plan``: (pages, tok) from each request's first new block."""
    W = min(int(max_block), block_table.shape[1])
    width = min(W, -(-int(max_query_len) // block_size) + 1)
    pages, tok = [], []
    for r in range(block_table.shape[0]):
        p0 = int(context_lens[r]) // block_size
        for t in range(width):
            b = p0 + t
            pages.append(int(block_table[r, min(b, W - 1)]))
            tok.append(min(max(int(seq_lens[r]) - b * block_size, 0), block_size))
    return np.array(pages, np.int64), np.array(tok, np.int32)


def row2req(cu_seqlens_q):
    cu = [int(c) for c in cu_seqlens_q]
    return np.array([r for r in range(len(cu) - 1) for _ in range(cu[r + 1] - cu[r])], np.int32)


def prefill_rows(cu_seqlens_q, context_lens):
    """(request, position) of every prefill query row: pos = ctx[r] + (row - cu[r])."""
    rq = row2req(cu_seqlens_q)
    pos = np.array([int(context_lens[r]) + i - int(cu_seqlens_q[r]) for i, r in enumerate(rq)], np.int32)
    return rq, pos
