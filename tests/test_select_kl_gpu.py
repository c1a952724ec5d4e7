"""``DeepseekV2Indexer.select_and_kl_loss`` (HF/_sparse_base_impl.py:3240-3516)
rebound by srswa.patch onto the HIP kernels, on a stand-in indexer whose index
projection returns two parameter tensors, vs the CPU oracle of every stage:

* block ids: per chunk, the top-k of the oracle's block-max scores
  (``srswa_oracle.block_max_scores``) after the candidate mask and the
  short-row fallback -- equal outside near-ties (tests/parity_report.py);
* loss: ``kl_oracle.gather_kl_dense`` + ``kl_loss`` on the kernel's ids, in
  float64 with the reference's 16-bit rounding of the logits, within 2e-3
  absolute + 1e-3 relative (the per-row bar of tests/test_kl_gpu.py);
* gradients of both index tensors within the 16-bit tolerance of
  tests/tolerance.py, from the same oracle through autograd.

Cases: the shipped single index head (the reference's gather branch); two
index heads (the reference's ``_KLChunkFn`` branch, the same KL computed
densely); a packed row of two block-aligned samples with an image-bucket
candidate mask that leaves some rows short of top-k candidates."""

import types

import pytest
import torch

from oracle import kl_oracle as K
from oracle import srswa_oracle as O
from parity_report import compare_selection
from tolerance import assert_close_lowp

pytestmark = pytest.mark.gpu


class StandInIndexer:
    """The attributes and helpers ``select_and_kl_loss`` reads; its index
    projection returns the parameters ``iq`` [B, HI, S, d] and ``ik``
    [B, 1, S, d] (through a multiply, so they are not the leaves)."""

    def __init__(self, iq, ik, *, local_blocks, topk_blocks, kl_chunk_size, image_bucket_constraint=False):
        self.iq, self.ik = iq, ik
        self.num_heads = iq.shape[1]
        self.head_dim = iq.shape[-1]
        self.block_size = 64
        self.local_blocks = local_blocks
        self.local_window = local_blocks * 64
        self.topk_blocks = topk_blocks
        self.kl_chunk_size = kl_chunk_size
        self.image_bucket_constraint = image_bucket_constraint
        self.layer_idx = 0
        self.kl_log_interval = 1
        self.eager_calls = 0

    def _project_index_qk(self, hidden_states, position_ids, past_key_values):
        return self.iq * 1.0, self.ik * 1.0

    def _remote_topk(self, num_key_blocks):
        return min(max(self.topk_blocks - self.local_blocks, 0), num_key_blocks)

    def _build_image_block_allow_mask(self, image_token_mask, nblk):
        B, S = image_token_mask.shape
        m = torch.zeros(B, nblk * 64, dtype=torch.bool, device=image_token_mask.device)
        m[:, :S] = image_token_mask.bool()
        return m.view(B, nblk, 64).any(-1)

    def _build_kl_candidate_mask(self, pos_chunk, nblk, image_token_mask, batch, cq, image_token_page_ids=None,
                                 query_token_page_ids=None):
        """Every image block (flat image mask), else every block; a row
        without one is open to every block."""
        if image_token_mask is None:
            return torch.ones(batch, 1, cq, nblk, dtype=torch.bool, device=pos_chunk.device)
        blk = self._build_image_block_allow_mask(image_token_mask, nblk)
        blk = torch.where(blk.any(-1, keepdim=True), blk, torch.ones_like(blk))
        return blk[:, None, None, :].expand(batch, 1, cq, nblk)

    def select_and_kl_loss(self, *args, **kwargs):
        self.eager_calls += 1
        return "eager"


def _bind():
    from srswa import patch
    base = types.ModuleType("_sparse_base_impl")
    base.DeepseekV2Indexer = StandInIndexer
    mod = types.SimpleNamespace(_base=base)
    assert "DeepseekV2Indexer.select_and_kl_loss" in patch.apply(mod)
    return patch, mod


def _expected(iq, ik, q_main, k_main, position_ids, got_bi, *, lw, topk, chunk, scaling, dtype, cand_fn):
    """(loss, per-chunk oracle scores after the candidate mask and fallback)
    on the kernel's selection; iq / ik float64 leaves."""
    B, HI, S, D = iq.shape
    nblk = -(-S // 64)
    packed = bool((position_ids[:, 1:] == 0).any())
    tot_kl = torch.zeros((), dtype=torch.float64)
    tot_cnt = torch.zeros((), dtype=torch.float64)
    scores = []
    for c0 in range(0, S, chunk):
        c1 = min(c0 + chunk, S)
        cq = c1 - c0
        if packed:
            pos = torch.arange(c0, c1).view(1, -1).expand(B, -1)
            seg = pos - position_ids[:, c0:c1]
        else:
            pos = position_ids[:, c0:c1]
            seg = torch.zeros_like(pos)
        posh = pos.unsqueeze(1).expand(B, HI, cq).reshape(B * HI, cq)
        segh = seg.unsqueeze(1).expand(B, HI, cq).reshape(B * HI, cq)
        keys = ik.detach().expand(B, HI, S, D).reshape(B * HI, S, D)
        bs_ = O.block_max_scores(iq.detach()[:, :, c0:c1].reshape(B * HI, cq, D), keys, posh, segh, 64, nblk,
                                 lw).view(B, HI, cq, nblk)
        cand = cand_fn(pos, nblk, cq)
        sc = bs_.masked_fill(~cand.expand_as(bs_), float("-inf"))
        short = (sc > float("-inf")).sum(-1, keepdim=True) < topk
        sc = torch.where(short, bs_, sc)
        scores.append(sc)
        kl, valid = K.gather_kl_dense(iq[:, :, c0:c1], ik[:, 0], q_main[:, :, c0:c1], k_main,
                                      got_bi[:, :, c0:c1], pos, block_size=64, local_window=lw, scaling=scaling,
                                      seg=seg if packed else None, round_dtype=dtype)
        v = valid.to(kl.dtype)
        tot_kl = tot_kl + (kl * v).sum()
        tot_cnt = tot_cnt + v.sum()
    return tot_kl / (tot_cnt + 1e-6), scores


CASES = {
    # B, HI, G (q heads per index head), HKV, S, D, local_blocks, topk_blocks, chunk, packed, image
    "shipped_one_index_head": (2, 1, 10, 10, 900, 128, 2, 10, 256, False, False),
    "two_index_heads_gqa": (1, 2, 3, 2, 700, 128, 2, 8, 300, False, False),
    "packed_image_buckets_d64": (1, 1, 4, 4, 704, 64, 2, 5, 0, True, True),
}


@pytest.mark.parametrize("name", list(CASES))
def test_select_and_kl_loss_matches_oracle(dev, name):
    B, HI, G, HKV, S, D, lb, tk, chunk, packed, image = CASES[name]
    print(f"select_and_kl_loss {name}", flush=True)
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(list(CASES).index(name) + 90)
    HQ = HI * G
    scaling = D ** -0.5
    iq0 = (torch.randn(B, HI, S, D, generator=g) * D ** -0.5).to(dtype)
    ik0 = torch.randn(B, 1, S, D, generator=g).to(dtype)
    q_main = torch.randn(B, HQ, S, D, generator=g).to(dtype)
    k_main = torch.randn(B, HKV, S, D, generator=g).to(dtype)
    if packed:
        position_ids = torch.cat([torch.arange(320), torch.arange(S - 320)]).view(1, S).expand(B, S).clone()
    else:
        position_ids = torch.arange(S).view(1, S).expand(B, S).clone()
    img = None
    if image:
        img = torch.zeros(B, S, dtype=torch.bool)
        img[:, 70:200] = True                 # blocks 1..3: rows with fewer than top-k take the fallback
        img[:, 400:520] = True                # blocks 6..8
    patch, mod = _bind()
    try:
        iq = torch.nn.Parameter(iq0.to(dev))
        ik = torch.nn.Parameter(ik0.to(dev))
        idx = StandInIndexer(iq, ik, local_blocks=lb, topk_blocks=tk, kl_chunk_size=chunk,
                             image_bucket_constraint=image)
        hidden = torch.zeros(B, S, 8, dtype=dtype, device=dev)
        bi, loss = idx.select_and_kl_loss(hidden, q_main.to(dev), k_main.to(dev), None, position_ids.to(dev),
                                          scaling, image_token_mask=None if img is None else img.to(dev))
        assert idx.eager_calls == 0
        nblk = -(-S // 64)
        topk = min(max(tk - lb, 0), nblk)
        assert bi.dtype == torch.long and bi.shape == (B, HI, S, topk)
        loss.backward()
        got_bi = bi.cpu()

        iqr = iq0.double().requires_grad_()
        ikr = ik0.double().requires_grad_()
        ref_idx = StandInIndexer(iq0, ik0, local_blocks=lb, topk_blocks=tk, kl_chunk_size=chunk,
                                 image_bucket_constraint=image)

        def cand_fn(pos, nb, cq):
            return ref_idx._build_kl_candidate_mask(pos, nb, img, B, cq)

        ch = chunk if chunk > 0 else S
        ref_loss, ref_scores = _expected(iqr, ikr, q_main.double(), k_main.double(), position_ids, got_bi,
                                         lw=lb * 64, topk=topk, chunk=ch, scaling=scaling, dtype=dtype,
                                         cand_fn=cand_fn)
        for i, sc in enumerate(ref_scores):
            c0 = i * ch
            compare_selection(got_bi[:, :, c0:c0 + sc.shape[2]], sc, topk, f"{name} chunk {i}")
        err = abs(loss.item() - ref_loss.item())
        assert err <= 2e-3 + 1e-3 * abs(ref_loss.item()), (loss.item(), ref_loss.item())
        ref_loss.backward()
        assert_close_lowp(iq.grad.cpu(), iqr.grad, dtype, what=f"{name} d iq")
        assert_close_lowp(ik.grad.cpu(), ikr.grad, dtype, what=f"{name} d ik")
        if image:
            # image blocks 1..3 and 6..8; the second sample's rows reach all of
            # 6..8 from position 640 on, earlier rows take the fallback
            live = (got_bi >= 0).any(-1)
            other = ((got_bi >= 0) & ~torch.isin(got_bi, torch.tensor([1, 2, 3, 6, 7, 8]))).any(-1)
            assert other.any() and (live & ~other).any()
    finally:
        patch.restore(mod)
    assert StandInIndexer.select_and_kl_loss.__name__ == "select_and_kl_loss"
    assert "_srswa_orig_select_and_kl_loss" not in vars(StandInIndexer)
