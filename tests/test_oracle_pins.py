"""Pins for the CPU oracle (oracle/srswa_oracle.py), CPU only.

The reference ships no tests, golden vectors or fixtures for this path, so each
oracle function is checked here against something that does not retype its
formula: a pure-Python enumeration of the key SETS the reference's kernels
read (HF/sparse_gather_triton.py:78-111, HF/modeling_deepseekv2.py:454-481),
textbook routines (torch's scaled_dot_product_attention, sorting), closed
forms, invariants, and torch.autograd.gradcheck for the backward.  A plausible
mistake (window off by one, a dropped segment bound, a transposed head map,
bias on window keys, summed duplicates) fails at least one of them.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import srswa_oracle as O


@pytest.fixture(autouse=True)
def _fp64_default():
    """fp64 for every tensor this module creates; restored afterwards."""
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


# ---------------------------------------------------------------- brute force
def _dot(a, b):
    return sum(float(x) * float(y) for x, y in zip(a, b))


def _softmax_rows(logits, vals):
    m = max(logits)
    w = [math.exp(z - m) for z in logits]
    s = sum(w)
    d = len(vals[0])
    o = [sum(w[i] * float(vals[i][e]) for i in range(len(w))) / s for e in range(d)]
    return o, m + math.log(s)


def brute_gather(q, k, v, bi, pos, bs, scale, lw, bias_slots=None):
    """Set enumeration of window | remote keys per query (pure Python)."""
    B, HQ, T, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    HI = bi.shape[1]
    o = torch.zeros(B, HQ, T, v.shape[-1])
    lse = torch.zeros(B, HQ, T)
    for b in range(B):
        for t in range(T):
            qi = Sk - T + t
            seg = qi - int(pos[b, t])
            ls = max(qi - lw + 1, seg)
            window = list(range(ls, qi + 1))
            for h in range(HQ):
                ih, kh = h // (HQ // HI), h // (HQ // Hkv)
                seen = []
                remote = {}
                for si, s in enumerate(bi[b, ih, t].tolist()):
                    if s < 0 or s * bs >= Sk or s in seen:
                        continue
                    seen.append(s)
                    bval = 0.0 if bias_slots is None else float(bias_slots[b, t, si])
                    for j in range(s * bs, min((s + 1) * bs, Sk)):
                        if seg <= j < ls and j <= qi:
                            remote[j] = bval
                keys = window + sorted(remote)
                logits = [scale * _dot(q[b, h, t], k[b, kh, j]) + (remote.get(j, 0.0)) for j in keys]
                oo, l = _softmax_rows(logits, [v[b, kh, j] for j in keys])
                o[b, h, t] = torch.tensor(oo)
                lse[b, h, t] = l
    return o, lse


def brute_decode(q, k, v, topi, bias, valid, q_pos, bs, lw, scale):
    """_decode_attend semantics by enumeration; topi/bias/valid [B,HI,Lq,K]."""
    B, H, Lq, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    HI = topi.shape[1]
    out = torch.zeros(B, H, Lq, v.shape[-1])
    for b in range(B):
        for r in range(Lq):
            qp = int(q_pos[b, r])
            win = [j for j in range(S) if qp - lw < j <= qp]
            for h in range(H):
                ih, kh = h // (H // HI), h // (H // Hkv)
                rem = {}
                for si in range(topi.shape[-1]):
                    s = int(topi[b, ih, r, si])
                    if not bool(valid[b, ih, r, si]) or s < 0:
                        continue
                    for j in range(s * bs, min((s + 1) * bs, S)):
                        if j <= qp - lw and j not in rem:     # an earlier slot's bias wins
                            rem[j] = float(bias[b, ih, r, si])
                keys = win + sorted(rem)
                logits = [scale * _dot(q[b, h, r], k[b, kh, j]) + rem.get(j, 0.0) for j in keys]
                out[b, h, r] = torch.tensor(_softmax_rows(logits, [v[b, kh, j] for j in keys])[0])
    return out


def _rand(*shape, g):
    return torch.randn(*shape, generator=g)


# ------------------------------------------------------- gather attention
def test_no_selection_full_window_is_causal_sdpa():
    g = torch.Generator().manual_seed(0)
    q, k, v = (_rand(2, 4, 150, 16, g=g) for _ in range(3))
    bi = torch.full((2, 1, 150, 3), -1)
    pos = torch.arange(150)[None].expand(2, -1)
    o, _ = O.gather_attention(q, k, v, bi, pos, 16, 0.3, local_window=150)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.3)
    assert (o - ref).abs().max() < 1e-12


def test_all_blocks_selected_is_causal_sdpa():
    g = torch.Generator().manual_seed(1)
    T, bs = 133, 16
    q, k, v = (_rand(1, 2, T, 8, g=g) for _ in range(3))
    M = -(-T // bs)
    bi = torch.arange(M).view(1, 1, 1, M).expand(1, 1, T, M).contiguous()
    pos = torch.arange(T)[None]
    for lw in (1, 20, 64):
        o, _ = O.gather_attention(q, k, v, bi, pos, bs, 0.5, local_window=lw)
        ref = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.5)
        assert (o - ref).abs().max() < 1e-12, lw


def test_no_selection_is_banded_sdpa():
    g = torch.Generator().manual_seed(2)
    T, lw = 97, 11
    q, k, v = (_rand(1, 3, T, 8, g=g) for _ in range(3))
    band = torch.ones(T, T, dtype=torch.bool).tril().triu(-(lw - 1))
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=band, scale=0.7)
    o, _ = O.gather_attention(q, k, v, torch.full((1, 1, T, 2), -1), torch.arange(T)[None], 8, 0.7,
                              local_window=lw)
    assert (o - ref).abs().max() < 1e-12


@pytest.mark.parametrize("case", ["plain", "packed", "prefix", "gqa_hi", "bias"])
def test_gather_matches_bruteforce(case):
    g = torch.Generator().manual_seed(100 + ["plain", "packed", "prefix", "gqa_hi", "bias"].index(case))
    B, HQ, Hkv, HI, T, Sk, D, bs, lw, S = 2, 2, 2, 1, 40, 40, 8, 4, 7, 3
    if case == "gqa_hi":
        HQ, Hkv, HI = 4, 2, 2
    if case == "prefix":
        Sk = 64
    q = _rand(B, HQ, T, D, g=g)
    k, v = _rand(B, Hkv, Sk, D, g=g), _rand(B, Hkv, Sk, D, g=g)
    nblk = -(-Sk // bs)
    bi = torch.randint(-1, nblk + 2, (B, HI, T, S), generator=g)
    bi[..., 1] = bi[..., 0]                                   # duplicates
    if case == "packed":
        pos = torch.cat([torch.arange(17), torch.arange(T - 17)])[None].expand(B, -1)
    else:
        pos = (Sk - T + torch.arange(T))[None].expand(B, -1)
    bias = None
    dense = None
    if case == "bias":
        bias = _rand(B, T, S, g=g)
        dense = O.bias_slots_to_dense(bias, bi[:, 0], nblk)
    o, lse = O.gather_attention(q, k, v, bi, pos, bs, 0.37, lw, blk_bias_dense=dense)
    ro, rl = brute_gather(q, k, v, bi, pos, bs, 0.37, lw, bias)
    assert (o - ro).abs().max() < 1e-10
    assert (lse - rl).abs().max() < 1e-10


def test_duplicates_equal_dedup_and_out_of_range_ignored():
    g = torch.Generator().manual_seed(3)
    q, k, v = (_rand(1, 1, 50, 8, g=g) for _ in range(3))
    pos = torch.arange(50)[None]
    bi = torch.tensor([1, 1, 2, -1, 99]).view(1, 1, 1, 5).expand(1, 1, 50, 5).contiguous()
    bd = torch.tensor([1, 2, -1, -1, -1]).view(1, 1, 1, 5).expand(1, 1, 50, 5).contiguous()
    a, _ = O.gather_attention(q, k, v, bi, pos, 8, 0.2, 9)
    b, _ = O.gather_attention(q, k, v, bd, pos, 8, 0.2, 9)
    assert (a - b).abs().max() < 1e-14


def test_gather_backward_gradcheck():
    g = torch.Generator().manual_seed(4)
    B, H, T, D, bs, lw = 1, 2, 24, 4, 4, 5
    q, k, v = (_rand(B, H, T, D, g=g).requires_grad_() for _ in range(3))
    bi = torch.randint(-1, T // bs, (B, 1, T, 3), generator=g)
    pos = torch.arange(T)[None]
    bias = _rand(B, T, 3, g=g).requires_grad_()

    def f(q, k, v, bias):
        return O.gather_attention_e2e(q, k, v, bi, bias, pos, bs, 0.5, lw)

    assert torch.autograd.gradcheck(f, (q, k, v, bias), eps=1e-6, atol=1e-6)


def test_bias_gradient_is_sum_of_dS_over_remote_keys():
    """d_bias[t, slot] = sum over heads and the block's remote keys of
    P*(dP - delta): checked against an explicit P/dP computation."""
    g = torch.Generator().manual_seed(6)
    B, H, T, D, bs, lw = 1, 2, 20, 4, 4, 5
    q, k, v = (_rand(B, H, T, D, g=g) for _ in range(3))
    bi = torch.randint(0, T // bs, (B, 1, T, 2), generator=g)
    pos = torch.arange(T)[None]
    bias = _rand(B, T, 2, g=g).requires_grad_()
    do = _rand(B, H, T, D, g=g)
    o = O.gather_attention_e2e(q, k, v, bi, bias, pos, bs, 0.5, lw)
    (o * do).sum().backward()
    # explicit: P from the brute-force logits
    ro, rl = brute_gather(q, k, v, bi, pos, bs, 0.5, lw, bias.detach())
    keep, remote = O.gather_keep_masks(bi, pos, T, bs, lw)
    dense = O.bias_slots_to_dense(bias.detach(), bi[:, 0], -(-T // bs))
    s = (q @ k.transpose(-1, -2)) * 0.5 + torch.where(remote, dense[:, None, :, torch.arange(T) // bs], 0.)
    P = torch.exp(s - rl[..., None]) * keep
    dP = do @ v.transpose(-1, -2)
    delta = (ro * do).sum(-1, keepdim=True)
    dS = P * (dP - delta)
    for t in range(T):
        for si in range(2):
            blk = int(bi[0, 0, t, si])
            if si == 1 and blk == int(bi[0, 0, t, 0]):
                exp = 0.0                      # duplicate slot carries no gradient
            else:
                js = [j for j in range(blk * bs, (blk + 1) * bs) if remote[0, 0, t, j]]
                exp = float(dS[0, :, t, js].sum()) if js else 0.0
            assert abs(float(bias.grad[0, t, si]) - exp) < 1e-10


# ------------------------------------------------------- decode
def test_decode_matches_bruteforce_with_bias_valid_dups():
    g = torch.Generator().manual_seed(7)
    B, H, Hkv, Lq, S, D, bs, lw, K = 2, 4, 2, 2, 90, 8, 8, 13, 4
    q = _rand(B, H, Lq, D, g=g)
    k, v = _rand(B, Hkv, S, D, g=g), _rand(B, Hkv, S, D, g=g)
    topi = torch.randint(0, -(-S // bs), (B, Lq, K), generator=g)
    topi[:, :, 1] = topi[:, :, 0]
    bias = _rand(B, Lq, K, g=g)
    valid = torch.rand(B, Lq, K, generator=g) > 0.3
    q_pos = torch.tensor([[89, 60], [30, 5]])
    o = O.decode_attend(q, k, v, topi, bias, valid, q_pos, bs, lw, 0.4)
    ref = brute_decode(q, k, v, topi[:, None], bias[:, None], valid[:, None], q_pos, bs, lw, 0.4)
    assert (o - ref).abs().max() < 1e-12


def test_decode_agrees_with_prefill_restatement_last_row():
    """Two independent restatements (decode: _decode_attend; prefill: the Triton
    kernel's remote/window split) agree on a causal last row without bias."""
    g = torch.Generator().manual_seed(8)
    B, H, T, D, bs, lw = 1, 2, 77, 8, 8, 16
    q, k, v = (_rand(B, H, T, D, g=g) for _ in range(3))
    bi = torch.randint(0, T // bs, (B, 1, T, 3), generator=g)
    full, _ = O.gather_attention(q, k, v, bi, torch.arange(T)[None], bs, 0.3, lw)
    topi = bi[:, 0, -1:, :]
    dec = O.decode_attend(q[:, :, -1:], k, v, topi, torch.zeros(topi.shape), torch.ones_like(topi, dtype=torch.bool),
                          torch.tensor([[T - 1]]), bs, lw, 0.3)
    assert (full[:, :, -1:] - dec).abs().max() < 1e-12


def test_decode_gather_form_equals_dense_form():
    g = torch.Generator().manual_seed(9)
    B, H, L, D, bs, lw, K = 2, 3, 700, 8, 16, 64, 5
    q = _rand(B, H, D, g=g)
    kc, vc = _rand(B, L, H, D, g=g), _rand(B, L, H, D, g=g)
    idx = torch.randint(-1, L // bs, (B, H, K), generator=g)
    bias = _rand(B, H, K, g=g)
    q_pos = torch.tensor([699, 333])
    a = O.decode_attend_gather(q, kc, vc, idx, q_pos, bs, lw, 0.25, bias=bias)
    b = O.decode_attend(q[:, :, None], kc.transpose(1, 2), vc.transpose(1, 2), idx[:, :, None],
                        bias[:, :, None], idx[:, :, None] >= 0, q_pos[:, None], bs, lw, 0.25)[:, :, 0]
    assert (a - b).abs().max() < 1e-12


def test_decode_without_remote_is_window_softmax():
    g = torch.Generator().manual_seed(10)
    q, k, v = _rand(1, 1, 1, 8, g=g), _rand(1, 1, 50, 8, g=g), _rand(1, 1, 50, 8, g=g)
    o = O.decode_attend(q, k, v, torch.zeros(1, 1, 2, dtype=torch.long), torch.zeros(1, 1, 2),
                        torch.zeros(1, 1, 2, dtype=torch.bool), torch.tensor([[40]]), 8, 10, 0.5)
    w = torch.softmax((k[0, 0, 31:41] @ q[0, 0, 0]) * 0.5, 0)
    assert (o[0, 0, 0] - w @ v[0, 0, 31:41]).abs().max() < 1e-12


# ------------------------------------------------------- indexer
def test_meanpool_scores_closed_form_and_invariants():
    g = torch.Generator().manual_seed(12)
    B, HI, Lq, S, d, bs, lb = 1, 2, 2, 45, 4, 8, 2
    q = _rand(B, HI, Lq, d, g=g)
    k = _rand(B, HI, S, d, g=g)
    q_pos = torch.tensor([[44, 30]])
    z = O.meanpool_block_scores(q, k, q_pos, bs, lb)
    nblk = -(-S // bs)
    for h in range(HI):
        for r in range(Lq):
            for blk in range(nblk):
                rows = [k[0, h, j].tolist() for j in range(blk * bs, min((blk + 1) * bs, S))]
                mean = [sum(c) / len(rows) for c in zip(*rows)]
                remote = blk <= int(q_pos[0, r]) // bs - lb
                want = _dot(q[0, h, r], mean) / math.sqrt(d) if remote else O.SCORE_NEG
                assert abs(float(z[0, h, r, blk]) - want) < 1e-12
    # permuting keys inside a block and scaling q
    perm = torch.arange(S)
    perm[:8] = torch.randperm(8, generator=g)
    assert (O.meanpool_block_scores(q, k[:, :, perm], q_pos, bs, lb) - z).abs().max() < 1e-12
    z2 = O.meanpool_block_scores(2.5 * q, k, q_pos, bs, lb)
    valid = z > O.SCORE_NEG * 0.5
    assert (z2[valid] - 2.5 * z[valid]).abs().max() < 1e-12
    # zero head_cls is mean pooling
    assert torch.equal(O.meanpool_block_scores(q, k, q_pos, bs, lb, head_cls=torch.zeros(d)), z)


def test_head_cls_weights_are_softmax_over_real_keys():
    g = torch.Generator().manual_seed(13)
    d, bs, S = 4, 8, 21
    q = _rand(1, 1, 1, d, g=g)
    k = _rand(1, 1, S, d, g=g)
    hc = _rand(d, g=g)
    z = O.meanpool_block_scores(q, k, torch.tensor([[100]]), bs, 1, head_cls=hc)
    for blk in range(-(-S // bs)):
        js = list(range(blk * bs, min((blk + 1) * bs, S)))
        a = [_dot(k[0, 0, j], hc) / math.sqrt(d) for j in js]
        m = max(a)
        w = [math.exp(x - m) for x in a]
        kb = [sum(w[i] * float(k[0, 0, j, e]) for i, j in enumerate(js)) / sum(w) for e in range(d)]
        assert abs(float(z[0, 0, 0, blk]) - _dot(q[0, 0, 0], kb) / math.sqrt(d)) < 1e-12


def test_block_max_bruteforce():
    g = torch.Generator().manual_seed(14)
    B, C, Sk, D, bs, lw = 2, 6, 50, 4, 8, 10
    q, k = _rand(B, C, D, g=g), _rand(B, Sk, D, g=g)
    pos = torch.randint(0, Sk, (B, C), generator=g)
    seg = torch.randint(0, 10, (B, C), generator=g)
    nblk = 8
    s = O.block_max_scores(q, k, pos, seg, bs, nblk, lw)
    for b in range(B):
        for c in range(C):
            ls = max(int(pos[b, c]) - lw + 1, 0)
            for blk in range(nblk):
                vals = [_dot(q[b, c], k[b, j]) for j in range(blk * bs, min((blk + 1) * bs, Sk))
                        if int(seg[b, c]) <= j < ls]
                want = max(vals) if vals else float("-inf")
                got = float(s[b, c, blk])
                assert (got == want) if want == float("-inf") else abs(got - want) < 1e-12


def test_topk_bruteforce_ties_invalid():
    g = torch.Generator().manual_seed(15)
    s = torch.randint(-3, 4, (20, 30), generator=g).double()
    s[0] = float("-inf")
    s[1, 5:] = O.SCORE_NEG
    s[2, ::3] = float("nan")
    for k in (1, 4, 10, 35):
        got = O.topk_blocks(s, k)
        for r in range(s.shape[0]):
            items = [(-float(x), j) for j, x in enumerate(s[r].tolist())
                     if x == x and x > O.SCORE_NEG * 0.5]
            want = [j for _, j in sorted(items)][:k]
            want += [-1] * (k - len(want))
            assert got[r].tolist() == want


def test_near_tie_rows():
    s = torch.tensor([[5.0, 4.0, 3.0, 3.00001, 1.0], [5.0, 4.0, 3.0, 2.0, 1.0]])
    assert O.near_tie_rows(s, 3).tolist() == [True, False]
    assert O.near_tie_rows(s, 2).tolist() == [False, False]


# ------------------------------------------------------- router (next row)
def _entmax_bisect(x):
    """1.5-entmax by bisection on tau: p_i = max(x_i/2 - tau, 0)^2, sum p = 1."""
    x = [xi / 2 for xi in x]
    lo, hi = max(x) - 1.0, max(x)
    for _ in range(200):
        mid = (lo + hi) / 2
        if sum(max(xi - mid, 0) ** 2 for xi in x) >= 1:
            lo = mid
        else:
            hi = mid
    return [max(xi - lo, 0) ** 2 for xi in x]


def test_entmax15_matches_bisection():
    g = torch.Generator().manual_seed(16)
    for n in (2, 5, 16):
        x = _rand(4, n, g=g) * 3
        p = O.entmax15(x)
        assert (p.sum(-1) - 1).abs().max() < 1e-12
        for r in range(4):
            want = _entmax_bisect(x[r].tolist())
            assert max(abs(a - b) for a, b in zip(p[r].tolist(), want)) < 1e-9
    assert (O.entmax15(torch.zeros(1, 4)) - 0.25).abs().max() < 1e-12


def _route_row(scores, cand_mask, idx_scale, floor, sigma, K, topm, window_all=False):
    """Pure-Python restatement of one row of ``_infer_route_select``
    (HF/modeling_deepseekv2.py:338-362): candidates (remote, intersected with
    the page mask unless that leaves none), x = score * idx_scale (sentinel for
    the rest and for NaN / inf), the top-M by (-x, id), 1.5-entmax of those M
    by bisection, the first K, log(max(prior, floor)) centred over the valid
    slots and divided by sigma.  ``window_all`` is a planted mistake (entmax
    over every block instead of the top-M window) used to show the cases below
    tell the two apart."""
    n = len(scores)
    remote = [s > O.SCORE_NEG * 0.5 for s in scores]          # NaN compares False
    cand = remote if cand_mask is None else [r and c for r, c in zip(remote, cand_mask)]
    if not any(cand):
        cand = remote
    x = []
    for i in range(n):
        v = scores[i] * idx_scale if cand[i] else O.ENTMAX_NEG
        x.append(v if math.isfinite(v) else O.ENTMAX_NEG)
    M = max(1, min(topm, n)) if topm > 0 else n
    order = sorted(range(n), key=lambda i: (-x[i], i))
    if window_all:
        full = _entmax_bisect(x)
        prior = [full[i] for i in order[:M]]
    else:
        prior = _entmax_bisect([x[i] for i in order[:M]])
    Kc = max(1, min(K, M))
    ids, prior = order[:Kc], prior[:Kc]
    valid = [cand[i] for i in ids]
    logp = [math.log(max(p, floor)) for p in prior]
    mu = sum(lp for lp, v in zip(logp, valid) if v) / max(1, sum(valid))
    bias = [(lp - mu) / sigma if v else 0.0 for lp, v in zip(logp, valid)]
    return ids, bias, valid


def _route_cases():
    g = torch.Generator().manual_seed(18)
    n = 40
    base = _rand(6, n, g=g)
    base[:, 30:] = O.SCORE_NEG                                 # blocks 30.. are not remote
    cases = []
    # narrow spread (broad entmax support, wider than the top-M window), sigma != 1
    cases.append(("narrow spread, M < candidates, sigma 0.7", base.clone(), None,
                  dict(idx_scale=0.3, floor=1e-4, sigma=0.7, K=6, topm=8)))
    # wide spread and a large floor: the floor binds on most slots
    cases.append(("binding floor", base.clone(), None, dict(idx_scale=4.0, floor=0.05, sigma=1.3, K=8, topm=16)))
    # page mask: row 0 no candidate left (remote fallback), row 1 fewer candidates than K
    cm = torch.rand(6, n, generator=g) < 0.5
    cm[0] = False
    cm[1] = False
    cm[1, :3] = True
    cases.append(("page mask, fallback, fewer candidates than K", base.clone(), cm,
                  dict(idx_scale=1.0, floor=1e-4, sigma=1.0, K=6, topm=16)))
    # topm = 0 (window = every block) and K > M
    small = base[:, :20].clone()
    cases.append(("topm 0, K > M", small, None, dict(idx_scale=0.5, floor=1e-5, sigma=2.0, K=50, topm=0)))
    # NaN / +inf / -inf scores, exact ties, a row with no remote block
    odd = torch.randint(-3, 4, (6, n), generator=g).double()
    odd[0, 5] = float("nan")
    odd[0, 6] = float("inf")
    odd[0, 7] = float("-inf")
    odd[1] = O.SCORE_NEG
    cases.append(("NaN, inf, ties, no remote row", odd, None, dict(idx_scale=0.7, floor=1e-4, sigma=1.0, K=5,
                                                                  topm=12)))
    return cases


@pytest.mark.parametrize("case", range(5))
def test_route_select_matches_pure_python(case):
    what, sc, cm, p = _route_cases()[case]
    xi, bias, valid = O.infer_route_select(sc, cm, p["idx_scale"], p["floor"], p["sigma"], p["K"], p["topm"])
    differs = False
    for r in range(sc.shape[0]):
        row = sc[r].tolist()
        mrow = None if cm is None else cm[r].tolist()
        ids, b, v = _route_row(row, mrow, **p)
        assert xi[r].tolist() == ids, (what, r)
        assert valid[r].tolist() == v, (what, r)
        assert max(abs(a - c) / max(1.0, abs(c)) for a, c in zip(bias[r].tolist(), b)) < 1e-6, (what, r)
        _, bm, _ = _route_row(row, mrow, **p, window_all=True)
        differs |= max(abs(a - c) for a, c in zip(bm, b)) > 1e-3
    if case == 0:
        # the planted mistake (entmax over every block) is visible in this case
        assert differs


def test_route_select_bias_is_mean_centred():
    g = torch.Generator().manual_seed(17)
    sc = _rand(2, 3, 20, g=g) * 4
    sc[..., 15:] = O.SCORE_NEG
    xi, bias, valid = O.infer_route_select(sc, None, 1.0, 1e-4, 1.0, K=6, topm=16)
    assert xi.shape == (2, 3, 6)
    m = (bias * valid).sum(-1) / valid.sum(-1)
    assert m.abs().max() < 1e-5
    assert (xi[valid] < 15).all()


# ------------------------------------------------------- paged decode (serving layout)
def _paged_brute(q, kc, vc, topk, bias, bt, sl, dql, lb, scale):
    """Key-by-key loop over attend_triton.py:307-518's two passes."""
    page = kc.shape[1]
    H, Hkv = q.shape[1], kc.shape[2]
    out = torch.zeros(q.shape, dtype=torch.float64)
    for n in range(q.shape[0]):
        r, i = n // dql, n % dql
        pos = int(sl[r]) - dql + i
        lws = max(0, pos - lb * page + 1)
        for h in range(H):
            kh = h // (H // Hkv)
            logits, vals = [], []
            seen = set()
            for s_ in range(topk.shape[-1]):
                blk = int(topk[kh, n, s_])
                if blk < 0 or blk in seen:
                    continue
                seen.add(blk)
                for j in range(blk * page, blk * page + page):
                    if j < pos + 1 and j < lws:
                        pg, off = int(bt[r, j // page]), j % page
                        logits.append(float(q[n, h] @ kc[pg, off, kh]) * scale + float(bias[kh, n, s_]))
                        vals.append(vc[pg, off, kh])
            if lb > 0:
                for j in range(lws, pos + 1):
                    pg, off = int(bt[r, j // page]), j % page
                    logits.append(float(q[n, h] @ kc[pg, off, kh]) * scale)
                    vals.append(vc[pg, off, kh])
            if logits:
                w = torch.softmax(torch.tensor(logits, dtype=torch.float64), 0)
                out[n, h] = (w[:, None] * torch.stack(vals)).sum(0)
    return out


def test_paged_decode_matches_key_loop_and_page_permutation():
    g = torch.Generator().manual_seed(31)
    R, dql, H, Hkv, D, page, nb, K, lb = 2, 2, 4, 2, 8, 4, 6, 3, 2
    npages = R * nb + 3
    q = _rand(R * dql, H, D, g=g)
    kc, vc = _rand(npages, page, Hkv, D, g=g), _rand(npages, page, Hkv, D, g=g)
    perm = torch.randperm(npages, generator=g)[:R * nb]
    bt = perm.view(R, nb)
    sl = torch.tensor([23, 17])
    topk = torch.randint(-1, nb, (Hkv, R * dql, K), generator=g)     # some ids past seq_len 17
    topk[0, 0, 1] = topk[0, 0, 0]                                  # repeated id
    topk[:, 3] = -1                                                # a row that selects nothing
    bias = _rand(Hkv, R * dql, K, g=g)
    want = _paged_brute(q, kc, vc, topk, bias, bt, sl, dql, lb, 0.5)
    got = O.paged_decode_attend(q, kc, vc, topk, bias, bt, sl, dql, lb, 0.5)
    assert (got - want).abs().max() < 1e-10
    # the same cache stored under other page ids gives the same result
    remap = torch.randperm(npages, generator=g)
    kc2, vc2 = torch.empty_like(kc), torch.empty_like(vc)
    kc2[remap], vc2[remap] = kc, vc
    got2 = O.paged_decode_attend(q, kc2, vc2, topk, bias, remap[bt], sl, dql, lb, 0.5)
    assert (got2 - got).abs().max() < 1e-12
    # no bias == zero bias
    z = torch.zeros_like(bias)
    assert (O.paged_decode_attend(q, kc, vc, topk, None, bt, sl, dql, lb, 0.5) -
            O.paged_decode_attend(q, kc, vc, topk, z, bt, sl, dql, lb, 0.5)).abs().max() < 1e-12
    # no window (local_blocks = 0): remote keys only, up to the query
    want0 = _paged_brute(q, kc, vc, topk, bias, bt, sl, dql, 0, 0.5)
    assert (want0[3] == 0).all()                                   # empty row -> zeros
    assert (O.paged_decode_attend(q, kc, vc, topk, bias, bt, sl, dql, 0, 0.5) - want0).abs().max() < 1e-10


# ------------------------------------------------------- head_cls summary cache (paged)
def test_kbar_cache_scores_equal_contiguous_scores():
    """Scores off the per-page summary cache == the contiguous head_cls scorer
    (itself pinned above) on each request's gathered keys; refresh_tail after an
    append equals a full rebuild; no head_cls == plain mean."""
    g = torch.Generator().manual_seed(41)
    R, page, nb, d, dql, lb = 3, 8, 9, 16, 2, 2
    npages = R * nb + 4
    keys = _rand(npages, page, d, g=g)
    bt = torch.randperm(npages, generator=g)[:R * nb].view(R, nb)
    sl = torch.tensor([70, 33, 65])
    hc = _rand(d, g=g)
    kbar = O.kbar_pages(keys, hc, bt, sl, torch.zeros(npages, d))
    q = _rand(R * dql, d, g=g)
    got = O.kbar_scores(q, kbar, bt, sl, nb, page, lb, dql=dql)
    for r in range(R):
        k = keys[bt[r]].reshape(nb * page, d)[: int(sl[r])][None, None]
        pos = (sl[r] - dql + torch.arange(dql))[None]
        want = O.meanpool_block_scores(q[r * dql:(r + 1) * dql][None, None], k, pos, page, lb, head_cls=hc)[0, 0]
        w = want.shape[-1]
        assert (got[r * dql:(r + 1) * dql, :w] - want).abs().max() < 1e-12
        assert (got[r * dql:(r + 1) * dql, w:] == O.SCORE_NEG).all()
    # append 5 tokens to request 1 (its last page changes) and refresh the tail
    keys2 = keys.clone()
    sl2 = sl.clone()
    sl2[1] += 5
    keys2[bt[1, 4], 1:6] = _rand(5, d, g=g)
    full = O.kbar_pages(keys2, hc, bt, sl2, torch.zeros(npages, d))
    tail = O.kbar_pages(keys2, hc, bt, sl2, kbar, tail_blocks=2)
    used = bt.flatten()
    assert (full[used] - tail[used]).abs().max() < 1e-12
    # no head_cls -> plain mean of the real keys
    m = O.kbar_pages(keys, None, bt, sl, torch.zeros(npages, d))
    assert (m[bt[1, 4]] - keys[bt[1, 4], :1].mean(0)).abs().max() < 1e-12


# ------------------------------------------------------- paged prefill (serving K10)
def test_paged_prefill_equals_gather_attention_per_kv_head():
    """paged_prefill_attend (K10's two passes, query by query) against the dense
    gather_attention restatement on each request's cache gathered page by page,
    one kv head at a time with that head's ids and slot biases (packed unique
    ids, as the serving router emits): prefix lengths, GQA 2:1, LB = 2."""
    g = torch.Generator().manual_seed(31)
    page, Hkv, G, D, LB = 16, 2, 2, 8, 2
    H = Hkv * G
    q_lens, seq_lens = [5, 9, 3], [40, 9, 70]
    prefix = [s - q for s, q in zip(seq_lens, q_lens)]
    cu = [0, 5, 14, 17]
    R, nb = 3, 5
    npages = R * nb + 2
    kc = torch.randn(npages, page, Hkv, D, generator=g)
    vc = torch.randn(npages, page, Hkv, D, generator=g)
    bt = torch.randperm(npages, generator=g)[:R * nb].view(R, nb)
    total = cu[-1]
    q = torch.randn(total, H, D, generator=g)
    S = 3
    topk = torch.full((Hkv, total, S), -1, dtype=torch.long)
    for n in range(total):
        for kh in range(Hkv):
            ids = torch.randperm(nb, generator=g)[:int(torch.randint(0, S + 1, (1,), generator=g))].sort().values
            topk[kh, n, :len(ids)] = ids
    bias = torch.randn(Hkv, total, S, generator=g)
    got = O.paged_prefill_attend(q, kc, vc, topk, bias, bt, cu, seq_lens, prefix, LB, 0.3)
    for r in range(R):
        rows = slice(cu[r], cu[r + 1])
        L = seq_lens[r]
        kr = kc[bt[r]].reshape(nb * page, Hkv, D)[:L]
        vr = vc[bt[r]].reshape(nb * page, Hkv, D)[:L]
        pos = (prefix[r] + torch.arange(q_lens[r]))[None]
        for kh in range(Hkv):
            hs = slice(kh * G, (kh + 1) * G)
            bi = topk[kh, rows][None, None]                                  # [1,1,T,S]
            dense = O.bias_slots_to_dense(bias[kh, rows][None], bi[:, 0], -(-L // page))
            o, _ = O.gather_attention(q[rows, hs].transpose(0, 1)[None], kr[:, kh:kh + 1].transpose(0, 1)[None],
                                      vr[:, kh:kh + 1].transpose(0, 1)[None], bi, pos, page, 0.3, LB * page,
                                      blk_bias_dense=dense)
            assert (got[rows, hs] - o[0].transpose(0, 1)).abs().max() < 1e-10


def test_paged_prefill_no_window_is_causal_selected_keys():
    """LB = 0: no window pass; a query attends only its selected blocks' keys up
    to and including its own position (enumerated by hand)."""
    g = torch.Generator().manual_seed(32)
    page, D = 16, 4
    kc = torch.randn(4, page, 1, D, generator=g)
    vc = torch.randn(4, page, 1, D, generator=g)
    bt = torch.tensor([[2, 0, 3, 1]])
    q = torch.randn(2, 1, D, generator=g)
    topk = torch.tensor([[[1, 3], [0, -1]]])                 # row 0: blocks 1, 3; row 1: block 0
    got = O.paged_prefill_attend(q, kc, vc, topk, None, bt, [0, 2], [40], [30], 0, 1.0)
    # row 0 at position 30: block 1 keys 16..30 (block 3 starts at 48 > 30)
    keys = list(range(16, 31))
    kv = torch.stack([kc[bt[0, j // page], j % page, 0] for j in keys])
    vv = torch.stack([vc[bt[0, j // page], j % page, 0] for j in keys])
    want = torch.softmax(kv @ q[0, 0], 0) @ vv
    assert (got[0, 0] - want).abs().max() < 1e-12
    # row 1 at position 31: block 0 keys 0..15
    kv = torch.stack([kc[bt[0, 0], j, 0] for j in range(16)])
    vv = torch.stack([vc[bt[0, 0], j, 0] for j in range(16)])
    assert (got[1, 0] - torch.softmax(kv @ q[1, 0], 0) @ vv).abs().max() < 1e-12


def test_indexer_forward_ids_equal_block_max_topk():
    """DeepseekV2Indexer.forward's dense chunked form equals the block-max
    restatement (itself pinned by brute force) followed by the tie-ordered
    top-k, for any chunking, with and without the image-block mask."""
    g = torch.Generator().manual_seed(31)
    B, HI, T, Sk, d, bs, lw, K = 2, 2, 40, 150, 8, 16, 20, 4
    q = _rand(B, HI, T, d, g=g)
    k = _rand(B, 1, Sk, d, g=g)
    pos = torch.stack([torch.randperm(Sk, generator=g)[:T] for _ in range(B)])
    nblk = -(-Sk // bs)
    img = torch.rand(B, nblk, generator=g) < 0.5
    for chunk, ib in ((0, None), (7, None), (13, img)):
        ids, bsc = O.indexer_forward_ids(q, k, pos, bs, lw, K, chunk=chunk, img_blk=ib)
        ref = O.block_max_scores(q.reshape(B * HI, T, d), k.expand(B, HI, Sk, d).reshape(B * HI, Sk, d),
                                 pos.repeat_interleave(HI, 0), torch.zeros(B * HI, T, dtype=torch.long), bs, nblk,
                                 lw).view(B, HI, T, nblk)
        if ib is not None:
            ref = ref.masked_fill(~ib[:, None, None, :], float("-inf"))
        assert torch.equal(bsc, ref)
        assert torch.equal(ids, O.topk_blocks(ref, K, invalid_at=float("-inf")))
    assert (ids == -1).any() and (ids >= 0).any()


def test_indexer_infer_scores_equal_clamped_block_max():
    """The stage0 "indexer" scores: block-max over keys j <= pos - LW (the
    block-max restatement with seg 0), clamped to +-1e4, SCORE_NEG for blocks
    without a key; the clamp is exercised with scaled-up inputs."""
    g = torch.Generator().manual_seed(32)
    B, Lq, S, d, bs, lw = 2, 30, 120, 8, 16, 24
    for scale in (1.0, 200.0):
        q = _rand(B, Lq, d, g=g) * scale
        k = _rand(B, S, d, g=g) * scale
        pos = torch.randint(0, S, (B, Lq), generator=g)
        nblk = -(-S // bs) + 1
        got = O.indexer_infer_block_scores(q, k, pos, nblk, bs, lw, q_chunk=11)
        bm = O.block_max_scores(q, k, pos, torch.zeros_like(pos), bs, nblk, lw)
        want = torch.where(torch.isinf(bm), torch.full_like(bm, O.SCORE_NEG), bm.clamp(-O.ACT_CLAMP, O.ACT_CLAMP))
        assert torch.equal(got, want)
    assert (got == O.ACT_CLAMP).any() and (got == O.SCORE_NEG).any()


def test_topk_blocks_invalid_at_minus_inf():
    """With invalid_at = -inf only -inf and NaN entries are invalid; -1e30 is
    a valid score (so -inf must not be mapped to the most negative float)."""
    s = torch.tensor([[-1e30, float("-inf"), float("nan"), -2e30, float("-inf")]], dtype=torch.float64)
    assert O.topk_blocks(s, 4, invalid_at=float("-inf")).tolist() == [[0, 3, -1, -1]]
    assert not O.near_tie_rows(s, 2, invalid_at=float("-inf")).any()


def _dash_train_case(g, B=2, S=5, nblk=9, scale=1.0):
    sc = _rand(B, S, nblk, g=g) * scale
    sc[0, 0, :] = O.SCORE_NEG                          # a row without a remote block
    sc[0, 1, 3:] = O.SCORE_NEG                         # a row with three remote blocks
    sc[1, :, -1] = O.SCORE_NEG
    return sc


def test_dash_route_train_rows_by_python_loop():
    """Candidates (block mask / image mask / fallback) and the prior row by row
    against a pure-Python restatement with the bisection entmax."""
    g = torch.Generator().manual_seed(41)
    sc = _dash_train_case(g)
    B, S, n = sc.shape
    bcand = torch.rand(B, S, n, generator=g) < 0.4
    bcand[1, 2] = False                                # masked to nothing -> fallback
    img = torch.rand(B, n, generator=g) < 0.5
    for blk, im, only in ((None, None, True), (bcand, None, True), (None, img, True), (None, img, False)):
        prior, cand = O.dash_route_train(sc, im, blk, 0.7, image_only=only)
        for b in range(B):
            for s in range(S):
                remote = [float(v) > -5e8 for v in sc[b, s]]
                m = [True] * n
                if blk is not None:
                    m = [bool(v) for v in blk[b, s]]
                elif only and im is not None:
                    m = [bool(v) for v in im[b]]
                c = [r and mm for r, mm in zip(remote, m)]
                if not any(c):
                    c = remote
                assert cand[b, s].tolist() == c
                x = [float(sc[b, s, j]) * 0.7 if c[j] else -1e4 for j in range(n)]
                want = _entmax_bisect(x)
                assert max(abs(a - w) for a, w in zip(prior[b, s].tolist(), want)) < 1e-9


def test_dash_select_and_bias_by_python_loop():
    g = torch.Generator().manual_seed(42)
    sc = _dash_train_case(g, scale=3.0)
    prior, cand = O.dash_route_train(sc, None, None, 1.0)
    for K, floor, sigma in ((4, 1e-4, 1.0), (6, 0.05, 0.5), (9, 1e-2, 2.0)):
        topi, bias, valid = O.dash_select_and_bias(prior, cand, K, floor, sigma)
        for b in range(sc.shape[0]):
            for s in range(sc.shape[1]):
                sel = [float(p) if bool(c) else -1.0 for p, c in zip(prior[b, s], cand[b, s])]
                order = sorted(range(len(sel)), key=lambda j: (-sel[j], j))[:K]
                assert topi[b, s].tolist() == order
                v = [sel[j] >= 0 for j in order]
                lp = [math.log(max(sel[j], floor)) for j in order]
                mu = sum(l for l, vv in zip(lp, v) if vv) / max(sum(v), 1)
                want = [(l - mu) / sigma if vv else 0.0 for l, vv in zip(lp, v)]
                assert valid[b, s].tolist() == v
                assert max(abs(a - w) for a, w in zip(bias[b, s].tolist(), want)) < 1e-9
    # entmax zeros tie when its support is narrower than K: the lower ids fill the slots
    p = torch.tensor([[[0.0, 0.7, 0.0, 0.3, 0.0, 0.0]]], dtype=torch.float64)
    topi, _, valid = O.dash_select_and_bias(p, torch.ones_like(p, dtype=torch.bool), 4, 1e-4, 1.0)
    assert topi.tolist() == [[[1, 3, 0, 2]]] and valid.all()


def test_dash_train_router_gradcheck():
    """The reference's entmax backward and the select / bias chain against
    finite differences (fp64), with block / image masks and a short row."""
    g = torch.Generator().manual_seed(43)
    sc = _dash_train_case(g, B=2, S=3, nblk=7, scale=0.8)
    img = torch.tensor([[1, 0, 1, 1, 0, 1, 1], [0, 1, 1, 1, 1, 0, 1]], dtype=torch.bool)
    w = torch.randn(2, 3, 4, generator=g, dtype=torch.float64)

    def f(x):
        prior, cand = O.dash_route_train(x, img, None, 1.3)
        _, bias, _ = O.dash_select_and_bias(prior, cand, 4, 1e-3, 0.7)
        return (bias * w).sum() + (prior * prior).sum()

    x = sc.clone().requires_grad_()
    assert torch.autograd.gradcheck(f, (x,), eps=1e-7, atol=1e-6)
