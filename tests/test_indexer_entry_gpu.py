"""The indexer's selection entry points rebound by srswa.patch, against the
oracle restatements of the reference functions:

* ``DeepseekV2Indexer.forward`` (HF/_sparse_base_impl.py:3065-3105) on a
  stand-in indexer -> ``srswa_oracle.indexer_forward_ids``: ids bit-exact
  outside near-ties (bf16 and fp32 projections, one and two index heads, the
  image-bucket block mask, a decode row against a longer key cache);
* ``_block_scores_infer`` with stage0 "indexer" (HF/modeling_deepseekv2.py:
  419-430) on the router's fp32 q / k -> ``srswa_oracle.indexer_infer_block_scores``:
  the SCORE_NEG pattern exact, scores within 1e-5 of sum |q_i k_i| (the fp32
  matrix-core block max), the +-1e4 clamp;
* the fp32 block-max kernel itself at block sizes 16..128."""

import types

import pytest
import torch

from oracle import srswa_oracle as O
from parity_report import compare_selection, report

pytestmark = pytest.mark.gpu


class StandInIndexer:
    """The attributes and helpers ``DeepseekV2Indexer.forward`` reads; the
    index projection returns fixed q [B, HI, T, d] / k [B, 1, Sk, d]."""

    def __init__(self, iq, ik, *, block_size, local_blocks, topk_blocks, image_bucket_constraint=False):
        self.iq, self.ik = iq, ik
        self.num_heads = iq.shape[1]
        self.block_size = block_size
        self.local_blocks = local_blocks
        self.local_window = local_blocks * block_size
        self.topk_blocks = topk_blocks
        self.kl_chunk_size = 256
        self.image_bucket_constraint = image_bucket_constraint
        self.eager_calls = 0

    def _project_index_qk(self, hidden_states, position_ids, past_key_values):
        return self.iq, self.ik

    def _remote_topk(self, num_key_blocks):
        return min(max(self.topk_blocks - self.local_blocks, 0), num_key_blocks)

    def _build_image_block_allow_mask(self, image_token_mask, nblk):
        B, S = image_token_mask.shape
        m = torch.zeros(B, nblk * self.block_size, dtype=torch.bool, device=image_token_mask.device)
        m[:, :S] = image_token_mask.bool()
        return m.view(B, nblk, self.block_size).any(-1)

    def forward(self, *args, **kwargs):
        self.eager_calls += 1
        return "eager"


FWD_CASES = {
    # B, HI, T, Sk, D, bs, local_blocks, topk_blocks, dtype, image, decode
    "bf16_one_head_bs64": (2, 1, 300, 1500, 128, 64, 2, 10, torch.bfloat16, False, False),
    "bf16_two_heads_image": (1, 2, 260, 1300, 128, 64, 2, 8, torch.bfloat16, True, False),
    "fp32_bs32_d64": (2, 1, 200, 900, 64, 32, 4, 12, torch.float32, False, False),
    "bf16_decode_row": (3, 1, 1, 2000, 128, 64, 2, 10, torch.bfloat16, False, True),
}


@pytest.mark.parametrize("name", list(FWD_CASES))
def test_indexer_forward_matches_oracle(dev, name):
    from srswa import patch
    B, HI, T, Sk, D, bs, lb, tk, dtype, image, decode = FWD_CASES[name]
    print(f"indexer forward {name}", flush=True)
    g = torch.Generator().manual_seed(list(FWD_CASES).index(name) + 200)
    iq = torch.randn(B, HI, T, D, generator=g).to(dtype)
    ik = torch.randn(B, 1, Sk, D, generator=g).to(dtype)
    if decode:
        pos = torch.full((B, 1), Sk - 1, dtype=torch.long)
    elif image:                               # rows spread over the sequence: early ones see few image blocks
        pos = (torch.arange(T) * (Sk // T)).expand(B, T).contiguous()
    else:
        pos = (torch.arange(T) + (Sk - T)).expand(B, T).contiguous()
    img = None
    if image:
        img = torch.zeros(B, Sk, dtype=torch.bool)
        img[:, 100:700] = True
    base = types.ModuleType("_sparse_base_impl")
    base.DeepseekV2Indexer = StandInIndexer
    mod = types.SimpleNamespace(_base=base)
    assert "DeepseekV2Indexer.forward" in patch.apply(mod)
    try:
        idx = StandInIndexer(iq.to(dev), ik.to(dev), block_size=bs, local_blocks=lb, topk_blocks=tk,
                             image_bucket_constraint=image)
        hidden = torch.zeros(B, T, 8, dtype=dtype, device=dev)
        got = idx.forward(hidden, None, None, pos.to(dev), None if img is None else img.to(dev))
        assert idx.eager_calls == 0
        nblk = -(-Sk // bs)
        K = min(tk - lb, nblk)
        assert got.dtype == torch.long and got.shape == (B, HI, T, K)
        ib = None if img is None else idx._build_image_block_allow_mask(img, nblk)
        ref_ids, ref_sc = O.indexer_forward_ids(iq.double(), ik.double(), pos, bs, lb * bs, K, img_blk=ib)
        counts = compare_selection(got.cpu(), ref_sc, K, f"indexer forward {name}", invalid_at=float("-inf"))
        assert counts["exact"] >= counts["rows"] - counts["near_tie"]
        if image:
            assert (got.cpu() == -1).any()                   # rows with fewer remote image blocks than K
            assert torch.isin(got.cpu()[got.cpu() >= 0], torch.arange(100 // bs, 700 // bs + 1)).all()
    finally:
        patch.restore(mod)
    assert StandInIndexer.forward.__name__ == "forward"


def _infer_case(seed, B, Lq, S, d, scale, tail=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, d, generator=g) * scale
    k = torch.randn(B, S, d, generator=g) * scale
    pos = (torch.arange(Lq) + (S - Lq)).expand(B, Lq).contiguous() if tail else \
        torch.randint(0, S, (B, Lq), generator=g)
    return q, k, pos


@pytest.mark.parametrize("bs,d,scale", [(64, 128, 1.0), (32, 64, 1.0), (64, 128, 60.0)])
def test_stage0_indexer_scores_fp32(dev, bs, d, scale):
    from srswa import patch
    print(f"stage0 indexer bs={bs} d={d} scale={scale}", flush=True)
    calls = []

    def _block_scores_infer(*args):
        calls.append(1)
        return "eager"

    mod = types.SimpleNamespace(_block_scores_infer=_block_scores_infer)
    patch.apply(mod)
    try:
        B, Lq, S, lw = 2, 300, 2500, 8 * bs
        q, k, pos = _infer_case(bs + d, B, Lq, S, d, scale)
        nblk = -(-S // bs)
        router = types.SimpleNamespace(stage0="indexer", block_size=bs, local_window=lw, q_chunk=128)
        got = mod._block_scores_infer(router, q.to(dev), k.to(dev), pos.to(dev), nblk).cpu()
        assert calls == [] and got.dtype == torch.float32 and got.shape == (B, Lq, nblk)
        ref = O.indexer_infer_block_scores(q.double(), k.double(), pos, nblk, bs, lw, q_chunk=128)
        neg = ref == O.SCORE_NEG
        assert torch.equal(got == O.SCORE_NEG, neg)
        bound = O.block_max_scores(q.double().abs(), k.double().abs(), pos, torch.zeros_like(pos), bs, nblk, lw)
        err = (got.double() - ref).abs()[~neg]
        rel = (err / bound[~neg].clamp(min=1e-30)).max().item()
        report(f"[err] stage0 indexer fp32 bs={bs} d={d} scale={scale}: max-abs {err.max().item():.3e}, "
               f"max |err| / sum|q k| {rel:.3e} (bar 1e-5)")
        assert rel <= 1e-5
        if scale > 1:
            assert (got == O.ACT_CLAMP).any()
        # host tensors still reach the original
        assert mod._block_scores_infer(router, q, k, pos, nblk) == "eager"
    finally:
        patch.restore(mod)


@pytest.mark.parametrize("bs", [16, 32, 64, 128])
def test_block_max_score_fp32(dev, bs):
    """The fp32 operand path of srswa_block_max_score (v_mfma_f32_32x32x2_f32),
    with sequence segments, against the fp64 oracle."""
    from srswa import ops
    g = torch.Generator().manual_seed(700 + bs)
    B, C, Sk, D, lw = 2, 270, 1100, 128, 100
    q = torch.randn(B, C, D, generator=g)
    k = torch.randn(B, Sk, D, generator=g)
    pos = torch.randint(0, Sk + 40, (B, C), generator=g)
    seg = torch.randint(0, 300, (B, C), generator=g)
    nblk = -(-Sk // bs) + 1
    got = ops.block_max_score(q.to(dev), k.to(dev), pos.to(dev), seg.to(dev), block_size=bs, num_key_blocks=nblk,
                              local_window=lw).cpu()
    ref = O.block_max_scores(q.double(), k.double(), pos, seg, bs, nblk, lw)
    bound = O.block_max_scores(q.double().abs(), k.double().abs(), pos, seg, bs, nblk, lw)
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(got), fin)
    rel = ((got.double()[fin] - ref[fin]).abs() / bound[fin]).max().item()
    report(f"[err] block max fp32 bs={bs}: max |err| / sum|q k| {rel:.3e} (bar 1e-5)")
    assert rel <= 1e-5
