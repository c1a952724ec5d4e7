"""srswa.patch on a stand-in of the reference's modeling_deepseekv2 namespace.

CPU part: rebinding, idempotence, restore, and that host tensors still reach
the original (eager) functions.  GPU part: the rebound functions on device
tensors agree with the oracle restatements of the reference functions."""

import math
import types

import pytest
import torch

from oracle import srswa_oracle as O
from srswa import patch


def _fake_module():
    calls = []

    def _decode_attend(*args):
        calls.append("decode")
        return "eager-decode"

    def _block_scores_infer(*args):
        calls.append("scores")
        return "eager-scores"

    def _infer_route_select(*args):
        calls.append("route")
        return "eager-route"

    return types.SimpleNamespace(_decode_attend=_decode_attend, _block_scores_infer=_block_scores_infer,
                                 _infer_route_select=_infer_route_select), calls


def test_apply_restore_and_host_fallback():
    mod, calls = _fake_module()
    orig = mod._decode_attend
    names = ["_decode_attend", "_block_scores_infer", "_infer_route_select"]
    assert patch.apply(mod) == names
    assert patch.apply(mod) == names     # idempotent
    q = torch.zeros(1, 1, 1, 8)
    assert mod._decode_attend(q, q, q, None, None, None, None, 8, 8, 1.0) == "eager-decode"
    router = types.SimpleNamespace(stage0="head_cls")
    assert mod._block_scores_infer(router, q, q, None, 4) == "eager-scores"
    assert mod._infer_route_select(torch.zeros(1, 1, 4), None, {}) == "eager-route"
    assert calls == ["decode", "scores", "route"]
    patch.restore(mod)
    assert mod._decode_attend is orig


@pytest.mark.gpu
def test_patched_functions_on_device(dev):
    mod, calls = _fake_module()
    patch.apply(mod)
    g = torch.Generator().manual_seed(4)
    B, H, Lq, S, D, bs, lw, K = 2, 4, 1, 900, 128, 32, 128, 4
    q = torch.randn(B, H, Lq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    topi = torch.randint(0, S // bs, (B, Lq, K), generator=g)
    bias = torch.randn(B, Lq, K, generator=g)
    valid = torch.ones(B, Lq, K, dtype=torch.bool)
    q_pos = torch.tensor([[899], [500]])
    got = mod._decode_attend(q.to(dev), k.to(dev), v.to(dev), topi.to(dev), bias.to(dev), valid.to(dev),
                             q_pos.to(dev), bs, lw, 1 / math.sqrt(D)).cpu()
    ref = O.decode_attend(q.double(), k.double(), v.double(), topi, bias.double(), valid, q_pos, bs, lw,
                          1 / math.sqrt(D))
    assert (got.double() - ref).abs().max().item() <= 2e-2
    # head_cls router scores (fp32 router q/k, learned head_cls)
    d = 128
    router = types.SimpleNamespace(stage0="head_cls", block_size=bs, local_blocks=lw // bs,
                                   head_cls=torch.randn(d, generator=g).to(dev))
    iq = torch.randn(B, Lq, d, generator=g)
    ik = torch.randn(B, S, d, generator=g)
    nblk = -(-S // bs)
    sc = mod._block_scores_infer(router, iq.to(dev), ik.to(dev), q_pos.to(dev), nblk).cpu()
    ref = O.meanpool_block_scores(iq[:, None], ik[:, None], q_pos, bs, lw // bs,
                                  head_cls=router.head_cls.cpu())[:, 0]
    valid_b = ref > O.SCORE_NEG * 0.5
    assert torch.equal(sc > O.SCORE_NEG * 0.5, valid_b)
    assert (sc[valid_b] - ref[valid_b]).abs().max().item() <= 1e-4
    # router on those scores (shipped parameters)
    p = dict(idx_scale=128.0 / math.sqrt(d), floor=1e-4, sigma=1.0, K=12, topm=16)
    xi, rb, rv = mod._infer_route_select(sc.to(dev), None, p)
    ox, ob, ov = O.infer_route_select(sc, None, p["idx_scale"], p["floor"], p["sigma"], p["K"], p["topm"])
    assert torch.equal(xi.cpu(), ox) and torch.equal(rv.cpu(), ov)
    assert ((rb.cpu() - ob).abs() <= 1e-5 * ob.abs().clamp(min=1.0)).all()
    assert calls == []


def test_select_and_kl_loss_rebinding_host_fallback():
    """Host tensors reach the indexer's own select_and_kl_loss; restore puts
    it back."""
    calls = []

    class DeepseekV2Indexer:
        block_size = 64

        def select_and_kl_loss(self, hidden_states, query_states, key_states, position_embeddings, position_ids,
                               scaling, image_token_mask=None, image_token_page_ids=None, query_token_page_ids=None):
            calls.append((image_token_mask, image_token_page_ids, query_token_page_ids))
            return "eager-select"

    orig = DeepseekV2Indexer.select_and_kl_loss
    base = types.ModuleType("_sparse_base_impl")
    base.DeepseekV2Indexer = DeepseekV2Indexer
    mod = types.SimpleNamespace(_base=base)
    assert "DeepseekV2Indexer.select_and_kl_loss" in patch.apply(mod)
    assert DeepseekV2Indexer.select_and_kl_loss is not orig
    x = torch.zeros(1, 4, 8)
    q = torch.zeros(1, 2, 4, 64)
    got = DeepseekV2Indexer().select_and_kl_loss(x, q, q, None, torch.arange(4)[None], 0.1, image_token_mask="m",
                                                  image_token_page_ids="p", query_token_page_ids="qp")
    assert got == "eager-select" and calls == [("m", "p", "qp")]
    patch.restore(mod)
    assert DeepseekV2Indexer.select_and_kl_loss is orig
