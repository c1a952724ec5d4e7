"""head_cls summary cache over a paged index-key cache (srswa_kbar_pages /
srswa_kbar_scores; KBarCache, headcls_scores_prefill / _decode of the
serving stage 0) vs the CPU oracle: page summaries and scores within 1e-5
relative (fp32 on bf16 keys), remote / non-remote pattern exact; tail refresh
after appended tokens; plain mean (no head_cls); D = 64 and 128."""

import pytest
import torch

from oracle import srswa_oracle as O

pytestmark = pytest.mark.gpu


def _setup(seed, R, page, nb, d, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    npages = R * nb + 7
    keys = torch.randn(npages, page, d, generator=g).to(dtype)
    bt = torch.randperm(npages, generator=g)[:R * nb].view(R, nb).to(torch.int32)
    sl = torch.randint(page, nb * page + 1, (R,), generator=g).to(torch.int32)
    hc = torch.randn(d, generator=g)
    return g, npages, keys, bt, sl, hc


def _close(got, ref, what):
    err = ((got.double() - ref.double()).abs() / ref.double().abs().clamp(min=1.0)).max().item()
    assert err <= 1e-5, (what, err)


@pytest.mark.parametrize("d,use_hc", [(128, True), (128, False), (64, True)])
def test_pages_scores_and_tail_refresh(dev, d, use_hc):
    from srswa import unlimited_dash_ops as U

    R, page, nb, dql, lb = 4, 32, 20, 2, 4
    g, npages, keys, bt, sl, hc = _setup(3 + d, R, page, nb, d)
    hc = hc if use_hc else None
    cache = U.KBarCache(npages, d, dev)
    # prefill: summaries of every used page + scores of the prefill rows
    cu = torch.tensor([0, 3, 3, 8, 10])
    ctx = (sl - torch.tensor([3, 0, 5, 2])).clamp(min=0)
    iq = torch.randn(10, d, generator=g)
    sc = U.headcls_scores_prefill(idx_q=iq.to(dev), kv_cache=keys.to(dev), block_table=bt.to(dev),
                                  cu_seqlens_q=cu.to(dev), seq_lens=sl.to(dev), context_lens=ctx.to(dev),
                                  head_cls=None if hc is None else hc.to(dev), max_block=nb + 3, block_size=page,
                                  local_blocks=lb, cache=cache)
    ref_kbar = O.kbar_pages(keys.double(), None if hc is None else hc.double(), bt, sl,
                            torch.zeros(npages, d, dtype=torch.float64))
    used = bt.flatten().long()
    _close(cache.k_bar.cpu()[used], ref_kbar[used], "kbar")
    req = torch.tensor([0, 0, 0, 2, 2, 2, 2, 2, 3, 3])
    pos = ctx[req] + (torch.arange(10) - cu[req])
    ref = O.kbar_scores(iq.double(), ref_kbar, bt, sl, nb + 3, page, lb, row_req=req, row_pos=pos)
    got = sc[0].cpu()
    assert torch.equal(got > O.SCORE_NEG * 0.5, ref > O.SCORE_NEG * 0.5)
    _close(got, ref, "prefill scores")
    # decode: append tokens, refresh the tail pages, score off the cache
    sl2 = (sl + torch.tensor([1, 5, 0, 9])).clamp(max=nb * page)
    keys2 = keys.clone()
    for r in range(R):
        for j in range(int(sl[r]), int(sl2[r])):
            keys2[bt[r, j // page], j % page] = torch.randn(d, generator=g).to(keys.dtype)
    cache.refresh_tail(kv_cache=keys2.to(dev), block_table=bt.to(dev), seq_lens=sl2.to(dev),
                       head_cls=None if hc is None else hc.to(dev), block_size=page, tail_pages=2)
    ref_kbar2 = O.kbar_pages(keys2.double(), None if hc is None else hc.double(), bt, sl2, ref_kbar, tail_blocks=2)
    _close(cache.k_bar.cpu()[used], ref_kbar2[used], "kbar after refresh")
    dq = torch.randn(R * dql, d, generator=g)
    sd = U.headcls_scores_decode(idx_q=dq.to(dev), cache=cache, block_table=bt.to(dev), seq_lens=sl2.to(dev),
                                 max_block=nb, block_size=page, local_blocks=lb, decode_query_len=dql)
    ref = O.kbar_scores(dq.double(), ref_kbar2, bt, sl2, nb, page, lb, dql=dql)
    got = sd[0].cpu()
    assert torch.equal(got > O.SCORE_NEG * 0.5, ref > O.SCORE_NEG * 0.5)
    _close(got, ref, "decode scores")
    # a score row wider than the block table: the extra columns are SCORE_NEG
    sw = U.headcls_scores_decode(idx_q=dq.to(dev), cache=cache, block_table=bt.to(dev), seq_lens=sl2.to(dev),
                                 max_block=nb + 3, block_size=page, local_blocks=lb, decode_query_len=dql)
    assert torch.equal(sw[0, :, :nb], sd[0]) and bool((sw[0, :, nb:] == O.SCORE_NEG).all())
