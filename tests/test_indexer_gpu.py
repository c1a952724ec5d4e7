"""Block indexer (head_cls / mean-pool scoring + top-k): HIP kernels vs the
CPU oracle, through the C ABI.

Bars (stated by the task): selected block ids bit-exact, except rows whose
k-th and (k+1)-th oracle scores differ by less than 1e-4 * max(1, |s_k|)
("near ties": fp32 summation order may legitimately swap them) -- those are
counted and reported, and must stay a small minority.  Scores: fp32, relative
error <= 1e-5 of the row's largest |score| (plus an absolute 1e-5 floor)."""

import math

import pytest
import torch

from oracle import srswa_oracle as O
from parity_report import compare_selection
import srswa
from srswa import workloads as W

pytestmark = pytest.mark.gpu


def _cmp_scores(got, ref):
    ref = ref.double()
    got = got.double()
    valid = ref > O.SCORE_NEG * 0.5
    assert torch.equal(got > O.SCORE_NEG * 0.5, valid), "remote-block masks differ"
    assert (got[~valid] == O.SCORE_NEG).all()
    scale = ref.abs().masked_fill(~valid, 0).amax(-1, keepdim=True).clamp(min=1.0)
    err = ((got - ref).abs() / scale).masked_fill(~valid, 0).max().item()
    assert err <= 1e-5, err


def _cmp_topk(got, ref_scores, k, what):
    c = compare_selection(got, ref_scores, k, what)
    return c["near_tie"], c["rows"]


@pytest.mark.parametrize("L,B", [(8192, 4), (32768, 2)])
def test_cfg2_family_meanpool_topk(dev, L, B):
    c = W.indexer_config(B=B, H=10, D=128, L=L)
    q, k, pos = c["q"], c["k"], c["q_pos"]
    BS, LB, K = 64, 512 // 64, 8
    ref = O.meanpool_block_scores(q[:, :, None, :], k.float().permute(0, 2, 1, 3),
                                  pos[:, None], BS, LB)
    idx, sc = srswa.index_meanpool_topk(q.to(dev), k.to(dev), pos.to(dev), block_size=BS,
                                        local_blocks=LB, topk=K, return_scores=True)
    _cmp_scores(sc.cpu()[:, :, None], ref)
    _cmp_topk(idx.cpu()[:, :, None], ref, K, f"config-2 family L={L} B={B} (mean pool, top-8)")
    # the shifted ("hot") blocks dominate the selection
    hot = c["hot"]
    for b in range(B):
        for h in range(10):
            sel, hb = set(idx[b, h].tolist()), set(hot[b, h].tolist())
            assert (sel <= hb) if len(hb) >= K else (hb <= sel)


def test_head_cls_prefill_rows_kvlen_shared_key_head(dev):
    """learned head_cls, several query rows at different positions, partial last
    block (kv_len), one key head shared by HI=2 index heads, fp32 keys."""
    g = torch.Generator().manual_seed(11)
    B, HI, Lq, D, L, BS, LB, K = 3, 2, 5, 128, 3000, 32, 4, 6
    q = torch.randn(B, HI, Lq, D, generator=g)
    k = torch.randn(B, L, D, generator=g)
    hc = torch.randn(D, generator=g) * 2.0
    q_pos = torch.tensor([[2999, 2500, 1000, 200, 40], [1500, 1499, 1498, 1497, 1496],
                          [2000, 2100, 2200, 2300, 2400]])
    kv_len = torch.tensor([3000, 1497, 2345])
    idx, sc, kbar = srswa.index_meanpool_topk(q.to(dev), k.to(dev), q_pos.to(dev), block_size=BS,
                                              local_blocks=LB, topk=K, head_cls=hc.to(dev),
                                              kv_len=kv_len.to(dev), return_scores=True,
                                              return_kbar=True)
    for b in range(B):
        Lb = int(kv_len[b])
        kk = k[b:b + 1, :Lb][:, None].expand(1, HI, Lb, D)
        ref = O.meanpool_block_scores(q[b:b + 1], kk, q_pos[b:b + 1], BS, LB, head_cls=hc)
        nb = ref.shape[-1]
        _cmp_scores(sc.cpu()[b:b + 1, ..., :nb], ref)
        assert (sc.cpu()[b, ..., nb:] == O.SCORE_NEG).all()
        _cmp_topk(idx.cpu()[b:b + 1], torch.cat([ref, torch.full((1, HI, Lq, sc.shape[-1] - nb), O.SCORE_NEG)], -1), K,
                  f"head_cls prefill rows, sequence {b}")


def test_topk_rows_ties_invalid_nan(dev):
    g = torch.Generator().manual_seed(5)
    s = torch.randint(-4, 5, (64, 300), generator=g).float()     # many exact ties
    s[0] = float("-inf")
    s[1, :3] = torch.tensor([1.0, float("nan"), 2.0])
    s[1, 3:] = O.SCORE_NEG
    s[2, ::2] = float("nan")
    for k in (1, 8, 37, 64):
        got = srswa.topk_rows(s.to(dev), k).cpu().long()
        assert torch.equal(got, O.topk_blocks(s, k)), k
        asc = srswa.topk_rows(s.to(dev), k, ascending=True).cpu().long()
        ref = O.topk_blocks(s, k)
        ref_asc = torch.where(ref >= 0, ref, torch.full_like(ref, 1 << 30)).sort(-1).values
        ref_asc = ref_asc.masked_fill(ref_asc == (1 << 30), -1)
        assert torch.equal(asc, ref_asc), k
