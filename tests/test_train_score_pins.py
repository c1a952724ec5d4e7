"""Pins of the DASH training block-scorer oracle (oracle/train_score_oracle.py)
by checks that do not restate it: a pure-Python brute force of both scorers
and of the block-max gradient, the mean-pool special case against the
separately pinned inference oracle, permutation invariance, the one-hot limit
of the head_cls summary, and float64 gradcheck."""

import math

import torch

from oracle import srswa_oracle as O
from oracle import train_score_oracle as T


def _inputs(seed, B, S, d, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, S, d, generator=g, dtype=dtype), torch.randn(B, S, d, generator=g, dtype=dtype),
            torch.randn(d, generator=g, dtype=dtype))


def _brute_headcls(q, k, hc, pos, nblk, bs, lb):
    """pure-Python restatement from the definition: weights = softmax over the
    block's real keys of clamp(k.hc / sqrt d), summary = weighted mean, score =
    clamp(q.summary / sqrt d) on remote blocks holding a key, else -1e9."""
    B, S, d = len(k), len(k[0]), len(k[0][0])
    isd = 1.0 / math.sqrt(d)
    out = [[[0.0] * nblk for _ in range(S)] for _ in range(B)]
    for b in range(B):
        kbar = []
        for c in range(nblk):
            keys = [k[b][t] for t in range(c * bs, min(c * bs + bs, S))]
            if not keys:
                kbar.append(None)
                continue
            aw = [max(-1e4, min(1e4, sum(x * y for x, y in zip(kt, hc)) * isd)) for kt in keys]
            m = max(aw)
            e = [math.exp(a - m) for a in aw]
            den = max(sum(e), 1e-6)
            kbar.append([sum(e[t] / den * keys[t][j] for t in range(len(keys))) for j in range(d)])
        for i in range(S):
            for c in range(nblk):
                if kbar[c] is not None and c <= pos[b][i] // bs - lb:
                    s = sum(x * y for x, y in zip(q[b][i], kbar[c])) * isd
                    out[b][i][c] = max(-1e4, min(1e4, s))
                else:
                    out[b][i][c] = -1e9
    return out


def test_headcls_matches_brute_force_and_meanpool_special_case():
    B, S, d, bs, lb = 2, 37, 4, 8, 1
    q, k, hc = _inputs(1, B, S, d)
    nblk = -(-S // bs)
    pos = torch.stack([torch.arange(S), torch.arange(S) + 5])
    got = T.headcls_scores(q, k, hc, pos, nblk, bs, lb)
    ref = torch.tensor(_brute_headcls(q.tolist(), k.tolist(), hc.tolist(), pos.tolist(), nblk, bs, lb),
                       dtype=torch.float64)
    assert torch.allclose(got, ref, rtol=1e-12, atol=1e-12)
    # head_cls = 0: uniform weights, i.e. the block mean -- the inference oracle's form
    z0 = T.headcls_scores(q, k, torch.zeros(d, dtype=torch.float64), pos, nblk, bs, lb)
    mp = O.meanpool_block_scores(q[:, None], k[:, None], pos, bs, lb)[:, 0]
    assert torch.allclose(z0, mp, rtol=1e-12, atol=1e-12)


def test_headcls_permutation_invariant_and_one_hot_limit():
    B, S, d, bs, lb = 1, 64, 8, 16, 1
    q, k, hc = _inputs(2, B, S, d)
    pos = torch.arange(S)[None] + 40
    nblk = S // bs
    z = T.headcls_scores(q, k, hc, pos, nblk, bs, lb)
    perm = torch.cat([torch.randperm(bs, generator=torch.Generator().manual_seed(c)) + c * bs for c in range(nblk)])
    zp = T.headcls_scores(q, k[:, perm], hc, pos, nblk, bs, lb)
    assert torch.allclose(z, zp, rtol=1e-12, atol=1e-12)
    # a head_cls far along one direction: the summary of block 0 becomes the
    # block's key with the largest projection on it
    u = k[0, 3] / k[0, 3].norm()
    j = int((k[0, :bs] @ u).argmax())
    kbar, _ = T.headcls_summary(k, u * 400.0, nblk, bs)
    assert torch.allclose(kbar[0, 0], k[0, j], atol=1e-6)


def test_headcls_gradcheck():
    B, S, d, bs, lb = 2, 21, 4, 4, 1
    q, k, hc = _inputs(3, B, S, d)
    q.requires_grad_()
    k.requires_grad_()
    hc.requires_grad_()
    pos = torch.stack([torch.arange(S), torch.arange(S) + 3])
    nblk = -(-S // bs)
    assert torch.autograd.gradcheck(lambda a, b, c: T.headcls_scores(a, b, c, pos, nblk, bs, lb), (q, k, hc))


def _brute_blockmax(q, k, pos, nblk, bs, lw, g):
    """scores and (dq, dk) for upstream g from the definition: per (row, block)
    the maximum of the clamped scores of the block's keys j with
    j <= pos - lw; the gradient goes to the keys attaining it, split evenly,
    and only to those whose unclamped score lies in [-1e4, 1e4]."""
    B, S, d = len(k), len(k[0]), len(k[0][0])
    out = [[[0.0] * nblk for _ in range(S)] for _ in range(B)]
    dq = [[[0.0] * d for _ in range(S)] for _ in range(B)]
    dk = [[[0.0] * d for _ in range(S)] for _ in range(B)]
    for b in range(B):
        for i in range(S):
            for c in range(nblk):
                keys = [j for j in range(c * bs, min(c * bs + bs, S)) if j <= pos[b][i] - lw]
                if not keys:
                    out[b][i][c] = -1e9
                    continue
                raw = {j: sum(x * y for x, y in zip(q[b][i], k[b][j])) for j in keys}
                cl = {j: max(-1e4, min(1e4, r)) for j, r in raw.items()}
                m = max(cl.values())
                out[b][i][c] = m
                tied = [j for j in keys if cl[j] == m]
                # the padded tail of a partial last block holds -1e9 entries that never tie
                w = g[b][i][c] / len(tied)
                for j in tied:
                    if -1e4 <= raw[j] <= 1e4:
                        for e in range(d):
                            dq[b][i][e] += w * k[b][j][e]
                            dk[b][j][e] += w * q[b][i][e]
    return out, dq, dk


def test_blockmax_matches_brute_force_with_ties_and_clamps():
    B, S, d, bs, lw = 2, 45, 3, 8, 10
    q, k, _ = _inputs(4, B, S, d)
    k[0, 9] = k[0, 12]                       # identical keys in one block: exact ties
    k[1, 17] = k[1, 16]
    q[1, 40] *= 1e4                          # scores beyond the clamp
    q.requires_grad_()
    k.requires_grad_()
    pos = torch.stack([torch.arange(S), torch.arange(S) + 7])
    nblk = -(-S // bs)
    z = T.blockmax_scores(q, k, pos, nblk, bs, lw)
    g = torch.randn(B, S, nblk, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    z.backward(g)
    ref, dq, dk = _brute_blockmax(q.tolist(), k.tolist(), pos.tolist(), nblk, bs, lw, g.tolist())
    assert torch.allclose(z, torch.tensor(ref, dtype=torch.float64), rtol=1e-12, atol=1e-9)
    assert torch.allclose(q.grad, torch.tensor(dq, dtype=torch.float64), rtol=1e-10, atol=1e-9)
    assert torch.allclose(k.grad, torch.tensor(dk, dtype=torch.float64), rtol=1e-10, atol=1e-9)
    # the ties were exercised
    assert (z[0, :, 1] > -1e8).any()


def test_blockmax_gradcheck_away_from_ties():
    B, S, d, bs, lw = 1, 30, 4, 6, 7
    q, k, _ = _inputs(6, B, S, d)
    q.requires_grad_()
    k.requires_grad_()
    pos = torch.arange(S)[None]
    nblk = S // bs
    assert torch.autograd.gradcheck(lambda a, b: T.blockmax_scores(a, b, pos, nblk, bs, lw), (q, k))


def test_sanitize_grad():
    g = torch.tensor([float("nan"), float("inf"), -float("inf"), 3e4, -2e4, 1.5])
    assert T.sanitize_grad(g).tolist() == [0.0, 0.0, 0.0, 1e4, -1e4, 1.5]
