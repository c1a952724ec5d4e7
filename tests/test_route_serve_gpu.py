"""Serving DASH router (srswa.unlimited_dash_ops.route_triton, the drop-in for
the SGLang backend's route_triton.py) vs the CPU oracle (oracle/route_oracle.py).

Bars:
* the router kernel on given fp32 scores: packed block ids bit-exact (-1
  fill, slots >= M untouched), biases within 1e-5 * max(1, |bias|) (the fp32
  log of the two sides may differ by an ulp);
* end to end (summary scores -> router): scores within 1e-5 relative of the
  fp64 oracle; the ids equal the oracle router run on the GPU's own scores
  bit-exactly, and those of the oracle run on its own scores outside near-ties;
* window bounds and plans exact; plan-driven summaries within 1e-5 relative.
"""

import math

import numpy as np
import pytest
import torch

from oracle import route_oracle as RO
from oracle import srswa_oracle as O
from parity_report import report
from srswa import ops
from srswa import unlimited_dash_ops as U

pytestmark = pytest.mark.gpu


def _scores(seed, rows, W, kind):
    rng = np.random.default_rng(seed)
    if kind == "ties":
        s = rng.integers(-3, 4, (rows, W)).astype(np.float32)
    elif kind == "flat":                                   # every z within (-1, 0]: the wide tau set
        s = (1.0 + 1e-3 * rng.standard_normal((rows, W))).astype(np.float32)
    elif kind == "equal":                                  # all candidates tied: the wide budget set
        s = np.ones((rows, W), np.float32)
    else:
        s = (rng.standard_normal((rows, W)) * 3).astype(np.float32)
    # each row's remote blocks end at a random width; the rest are not remote
    ends = rng.integers(0, W + 1, rows)
    ends[0] = W
    for r in range(rows):
        s[r, ends[r]:] = RO.SCORE_NEG
    if kind == "ties":
        s[1, 3] = np.nan
    return s


CASES = {
    # name: (rows, W, kind, K, M, idx_scale, floor, sigma, image mask)
    "decode_w2048": (64, 2048, "normal", 8, 16, 128 / math.sqrt(128), 1e-4, 1.0, False),
    "image_mask": (48, 700, "normal", 6, 8, 2.0, 1e-4, 0.7, True),
    "ties_nan": (32, 300, "ties", 8, 8, 1.0, 1e-4, 1.0, True),
    "budget_over_64": (16, 1000, "normal", 100, 128, 0.5, 1e-5, 1.3, False),
    "wide_tau_set": (8, 2048, "flat", 8, 16, 1.0, 1e-4, 1.0, False),
    "all_tied": (4, 1000, "equal", 8, 8, 1.0, 1e-4, 1.0, False),
    "narrow_w5": (6, 5, "normal", 2, 4, 1.0, 1e-4, 1.0, True),
    "w65": (10, 65, "normal", 64, 64, 3.0, 1e-4, 1.0, False),
    # rows whose waves fill more than the GPU's SIMDs (a prefill chunk) take one
    # wave per row; the cases above, fewer rows, two (tau and budget side by side)
    "many_rows_w2048": (1500, 2048, "normal", 8, 16, 128 / math.sqrt(128), 1e-4, 1.0, True),
    "many_rows_w300": (1100, 300, "ties", 8, 8, 1.0, 1e-4, 1.0, False),
    # rows above 2048 columns take the streaming kernel (the others hold the row in registers)
    "stream_w4100": (8, 4100, "normal", 8, 16, 128 / math.sqrt(128), 1e-4, 1.0, True),
    "stream_flat_w3000": (4, 3000, "flat", 12, 16, 1.0, 1e-4, 1.0, False),
}


@pytest.mark.parametrize("name", list(CASES))
def test_route_kernel_matches_oracle(dev, name):
    rows, W, kind, K, M, idx_scale, floor, sigma, use_img = CASES[name]
    s = _scores(list(CASES).index(name), rows, W, kind)
    img = None
    if use_img:
        rng = np.random.default_rng(99)
        img = rng.random((rows, W)) < 0.3
        img[0] = False                                     # no allowed block: fallback to every remote
        img[1, :] = False
        img[1, W - 1] = True                               # only a (maybe) non-remote block allowed
    ext = 3
    oi = torch.full((rows, M + ext), 99, dtype=torch.int32, device=dev)
    ob = torch.full((rows, M + ext), 7.0, dtype=torch.float32, device=dev)
    ops.route_serve(torch.from_numpy(s).to(dev), None if img is None else torch.from_numpy(img).to(dev), oi, ob,
                    K=K, M=M, idx_scale=idx_scale, prior_floor=floor, inv_sigma=1.0 / sigma)
    ri = np.full((rows, M + ext), 99, np.int32)
    rb = np.full((rows, M + ext), 7.0, np.float32)
    RO.route_entmax(s, img, ri, rb, idx_scale=idx_scale, prior_floor=floor, inv_sigma=np.float32(1.0 / sigma),
                    K=K, M=M)
    gi, gb = oi.cpu().numpy(), ob.cpu().numpy()
    bad = [r for r in range(rows) if not np.array_equal(gi[r], ri[r])]
    assert not bad, (name, bad[:5], gi[bad[0]][:12], ri[bad[0]][:12])
    err = np.abs(gb.astype(np.float64) - rb) / np.maximum(1.0, np.abs(rb))
    report(f"[err] serving router {name}: ids exact ({rows} rows), bias max rel {err.max():.3e} (bar 1e-5)")
    assert err.max() <= 1e-5, (name, float(err.max()))


def _paged(seed, R, page, nb, d, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    npages = R * nb + 5
    keys = torch.randn(npages, page, d, generator=g).to(dtype)
    bt = torch.randperm(npages, generator=g)[:R * nb].view(R, nb).to(torch.int32)
    sl = torch.randint(page * 2, nb * page + 1, (R,), generator=g).to(torch.int32)
    hc = torch.randn(d, generator=g) * 0.5
    return g, npages, keys, bt, sl, hc


def _check_ids_chain(what, got_i, got_b, sc_gpu, sc_ref, img, K, M, p):
    """ids of the oracle router on the GPU's scores: exact; on the oracle's
    scores: equal outside rows whose budget boundary is a near tie."""
    rows = got_i.shape[0]
    ri = np.zeros((rows, M), np.int32)
    rb = np.zeros((rows, M), np.float32)
    RO.route_entmax(sc_gpu, img, ri, rb, idx_scale=p["idx_scale"], prior_floor=p["floor"],
                    inv_sigma=np.float32(1.0 / p["sigma"]), K=K, M=M)
    assert np.array_equal(got_i[:, :M], ri), what
    err = np.abs(got_b[:, :M].astype(np.float64) - rb) / np.maximum(1.0, np.abs(rb))
    assert err.max() <= 1e-5, (what, float(err.max()))
    oi = np.zeros((rows, M), np.int32)
    obb = np.zeros((rows, M), np.float32)
    RO.route_entmax(sc_ref, img, oi, obb, idx_scale=p["idx_scale"], prior_floor=p["floor"],
                    inv_sigma=np.float32(1.0 / p["sigma"]), K=K, M=M)
    same = (oi == ri).all(1)
    cand = sc_ref > -5e8
    if img is not None:
        ci = cand & img
        cand = np.where(ci.any(1, keepdims=True), ci, cand)
    x = np.where(cand, sc_ref * p["idx_scale"], -np.inf)
    top = -np.sort(-x, 1)
    with np.errstate(invalid="ignore"):          # -inf - -inf in rows with few candidates: not a tie
        gap = top[:, K - 1] - top[:, K] if x.shape[1] > K else np.full(rows, np.inf)
    gap = np.where(np.isnan(gap), np.inf, gap)
    near = np.abs(gap) < 1e-4 * np.maximum(1.0, np.abs(top[:, K - 1]))
    report(f"[ids] {what}: rows {rows}, equal to the oracle on its own scores {int(same.sum())}, "
           f"near-tie {int(near.sum())}, differ outside near-ties {int(((~same) & (~near)).sum())}")
    assert not ((~same) & (~near)).any(), what


@pytest.mark.parametrize("d,dql,use_img", [(128, 1, False), (128, 2, True), (64, 1, True)])
def test_route_decode_end_to_end(dev, d, dql, use_img):
    R, page, nb, lb = 6, 64, 40, 4
    g, npages, keys, bt, sl, hc = _paged(11 + d + dql, R, page, nb, d)
    kbar = torch.zeros(npages, d, dtype=torch.float32, device=dev)
    ops.kbar_pages(keys.to(dev), hc.to(dev), bt.to(dev), sl.to(dev), kbar)
    nd = R * dql
    idx_q = torch.randn(nd, d, generator=g).to(torch.bfloat16)
    W = nb + 2
    img = None
    if use_img:
        img = torch.rand(nd, W, generator=g) < 0.25
        img[0] = False
    p = dict(idx_scale=8.0 / math.sqrt(d), floor=1e-4, sigma=1.0)
    M, K = 16, 8
    out_idx = torch.full((nd, 16), -5, dtype=torch.int32, device=dev)
    out_bias = torch.zeros(nd, 16, dtype=torch.float32, device=dev)
    score_buf = torch.empty(nd + 2, W + 3, dtype=torch.float32, device=dev)
    m = U.route_decode_triton(idx_q=idx_q.to(dev), k_bar=kbar, block_table=bt.to(dev), seq_lens=sl.to(dev),
                              image_allow=None if img is None else img.to(dev), out_idx=out_idx, out_bias=out_bias,
                              max_block=W, block_size=page, local_blocks=lb, decode_query_len=dql,
                              idx_scale=p["idx_scale"], prior_floor=p["floor"], sigma=p["sigma"], topm=16,
                              score_buf=score_buf, budget=K, out_slots=16)
    assert m == M
    Wk = min(W, nb)
    sc = score_buf[:nd, :Wk].cpu()
    ref_k = O.kbar_pages(keys.double(), hc.double(), bt, sl, torch.zeros(npages, d, dtype=torch.float64))
    ref = O.kbar_scores(idx_q.double(), ref_k, bt, sl, Wk, page, lb, dql=dql)
    remote = ref > -5e8
    assert torch.equal(sc > -5e8, remote)
    rel = ((sc.double() - ref).abs() / ref.abs().clamp(min=1.0)).masked_fill(~remote, 0).max().item()
    report(f"[err] route_decode scores d={d} dql={dql}: max rel {rel:.3e} (bar 1e-5)")
    assert rel <= 1e-5
    _check_ids_chain(f"route_decode d={d} dql={dql} img={use_img}", out_idx.cpu().numpy(), out_bias.cpu().numpy(),
                     sc.numpy(), ref.float().numpy(), None if img is None else img[:, :Wk].numpy(), K, M, p)


def test_route_prefill_end_to_end_chunks(dev):
    d, page, nb, lb = 128, 32, 30, 4
    R = 4
    g, npages, keys, bt, sl, hc = _paged(5, R, page, nb, d)
    kbar = torch.zeros(npages, d, dtype=torch.float32, device=dev)
    ops.kbar_pages(keys.to(dev), hc.to(dev), bt.to(dev), sl.to(dev), kbar)
    qlen = torch.tensor([7, 0, 40, 13])
    ctx = (sl - qlen).clamp(min=0)
    cu = torch.cat([torch.zeros(1, dtype=torch.int64), qlen.cumsum(0)])
    total_q = int(cu[-1])
    idx_q = torch.randn(total_q, d, generator=g).to(torch.bfloat16)
    row2req = U.prefill_row2req(cu_seqlens_q=cu.to(dev), device=dev)
    rq, pos = RO.prefill_rows(cu.tolist(), ctx.tolist())
    assert row2req.cpu().numpy().tolist() == rq.tolist()
    W = nb
    img = torch.rand(total_q, W, generator=g) < 0.3
    p = dict(idx_scale=1.5, floor=1e-4, sigma=0.8)
    M, K = 8, 6
    out_idx = torch.zeros(total_q, M, dtype=torch.int32, device=dev)
    out_bias = torch.zeros(total_q, M, dtype=torch.float32, device=dev)
    m, sc_last, off = U.route_prefill_triton(
        idx_q=idx_q.to(dev), k_bar=kbar, block_table=bt.to(dev), seq_lens=sl.to(dev), cu_seqlens_q=cu.to(dev),
        context_lens=ctx.to(dev), row2req=row2req, image_allow=img.to(dev), out_idx=out_idx, out_bias=out_bias,
        max_block=W, block_size=page, local_blocks=lb, idx_scale=p["idx_scale"], prior_floor=p["floor"],
        sigma=p["sigma"], topm=M, budget=K, q_chunk=16)
    assert m == M and off == 48 and sc_last.shape[0] == total_q - 48
    ref_k = O.kbar_pages(keys.double(), hc.double(), bt, sl, torch.zeros(npages, d, dtype=torch.float64))
    ref = O.kbar_scores(idx_q.double(), ref_k, bt, sl, W, page, lb, row_req=torch.from_numpy(rq),
                        row_pos=torch.from_numpy(pos))
    last = sc_last.cpu()[:, :W]
    rel = ((last.double() - ref[off:]).abs() / ref[off:].abs().clamp(min=1.0)).masked_fill(
        ref[off:] <= -5e8, 0).max().item()
    assert rel <= 1e-5 and torch.equal(last > -5e8, ref[off:] > -5e8)
    # every row's scores in one launch (a row's arithmetic does not depend on its chunk) for the id chain
    full = ops.kbar_scores(idx_q.to(dev), kbar, bt.to(dev), sl.to(dev), width=W, page_size=page, local_blocks=lb,
                           row_req=row2req, cu_q=cu.to(dev), ctx=ctx.to(dev), row_off=0).cpu()
    assert torch.equal(full[off:], last)
    _check_ids_chain("route_prefill (4 requests, 60 rows, q_chunk 16)", out_idx.cpu().numpy(),
                     out_bias.cpu().numpy(), full.numpy(), ref.float().numpy(), img.numpy(), K, M, p)


def test_win_bounds_matches_oracle(dev):
    g = torch.Generator().manual_seed(3)
    R, dql, W, bs, lb = 9, 2, 60, 32, 4
    sl = torch.randint(0, W * bs, (R,), generator=g).to(torch.int32)
    sl[0] = 0
    sl[1] = 100
    allow = torch.rand(R * dql, W + 4, generator=g) < 0.05
    allow[4] = False
    lo = torch.zeros(R * dql, dtype=torch.int32, device=dev)
    hi = torch.zeros_like(lo)
    fit = torch.zeros(R * dql, dtype=torch.int8, device=dev)
    U.win_bounds_decode(allow=allow.to(dev), seq_lens=sl.to(dev), lo=lo, hi=hi, fit=fit, max_block=W,
                        block_size=bs, local_blocks=lb, decode_query_len=dql, tile=16)
    rl, rh, rf = RO.win_bounds(allow.numpy(), sl.numpy(), max_block=W, block_size=bs, local_blocks=lb, dql=dql,
                               tile=16)
    assert lo.cpu().numpy().tolist() == rl.tolist()
    assert hi.cpu().numpy().tolist() == rh.tolist()
    assert fit.cpu().numpy().tolist() == rf.tolist()


def test_refresh_by_tail_and_prefill_plans(dev):
    d, page, nb = 128, 64, 12
    R = 5
    g, npages, keys, bt, sl, hc = _paged(21, R, page, nb, d)
    kb0 = torch.randn(npages, d, generator=g)
    # tail plan (2 pages per request)
    kbar = kb0.clone().to(dev)
    plan = U.kbar_tail_plan(block_table=bt.to(dev), seq_lens=sl.to(dev), block_size=page, tail_pages=2, device=dev)
    pg, tk = RO.tail_plan(bt.numpy(), sl.numpy(), page, 2)
    assert plan[0].cpu().numpy().tolist() == pg.tolist() and plan[1].cpu().numpy().tolist() == tk.tolist()
    U.kbar_refresh_tail_triton(kv_cache=keys.to(dev), k_bar=kbar, block_table=bt.to(dev), seq_lens=sl.to(dev),
                               head_cls=hc.to(dev), block_size=page, plan=plan)
    want = kb0.double().clone()
    for p_, t_ in zip(pg.tolist(), tk.tolist()):
        want[p_] = O.kbar_summaries(keys[p_][None].double(), (torch.arange(page) < t_)[None], hc.double())[0]
    got = kbar.cpu().double()
    assert ((got - want).abs() / want.abs().clamp(min=1.0)).max().item() <= 1e-5
    # prefill plan: pages past the live ones carry tok 0 and stay untouched
    kbar = kb0.clone().to(dev)
    ctx = (sl - 100).clamp(min=0)
    plan = U.kbar_all_plan(block_table=bt.to(dev), seq_lens=sl.to(dev), context_lens=ctx.to(dev), block_size=page,
                           max_block=nb, max_query_len=100, device=dev)
    pg, tk = RO.all_plan(bt.numpy(), sl.numpy(), ctx.numpy(), page, nb, 100)
    assert plan[0].cpu().numpy().tolist() == pg.tolist() and plan[1].cpu().numpy().tolist() == tk.tolist()
    assert (tk == 0).any()
    U.kbar_refresh_tail_triton(kv_cache=keys.to(dev), k_bar=kbar, block_table=bt.to(dev), seq_lens=sl.to(dev),
                               head_cls=None, block_size=page, plan=plan)
    want = kb0.double().clone()
    for p_, t_ in zip(pg.tolist(), tk.tolist()):
        if t_ > 0:
            want[p_] = O.kbar_summaries(keys[p_][None].double(), (torch.arange(page) < t_)[None], None)[0]
    got = kbar.cpu().double()
    assert ((got - want).abs() / want.abs().clamp(min=1.0)).max().item() <= 1e-5
