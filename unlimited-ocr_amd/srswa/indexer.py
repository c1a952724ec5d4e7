"""The indexer's block selection on the MI355X kernels.

* ``indexer_forward`` -- ``DeepseekV2Indexer.forward``
  (HF/_sparse_base_impl.py:3065-3105): remote top-k block ids per query from
  the block-max scores, with the image-bucket block mask.
* ``block_scores_indexer`` -- the stage0 == "indexer" branch of the
  inference router's ``_block_scores_infer`` (HF/modeling_deepseekv2.py:419-430).
* ``select_and_kl_loss`` -- the training step's selection and distillation KL
  (HF/_sparse_base_impl.py:3240-3516), below.

``select_and_kl_loss``, per pass of query rows (at least ``kl_chunk_size``;
the reference's chunks bound its dense [B, H, C, Sk] tensors, which do not
exist here):

1. block scores -- ``srswa_block_max_score``: max over each 64-key block of
   the index logits over causal, non-local, same-sample keys (:3319-3348; the
   reference's Triton path, whose dense fallback :3350-3366 masks the same keys);
2. candidates -- the indexer's own ``_build_kl_candidate_mask`` (page /
   image buckets, :3368-3371), masked to -inf, and the per-row fallback to the
   unconstrained scores when fewer than ``topk`` candidates stay finite
   (:3388-3396; applied without the reference's host-side ``any`` test, which
   leaves the values unchanged);
3. top-k -- ``srswa_topk_rows``: descending, ties to the lower block id,
   -inf entries never chosen (-1 in their slots), as ``topk`` +
   ``masked_fill(score == -inf, -1)`` (:3398-3404);
4. the KL -- ``srswa.kl.gather_kl`` over the selected blocks: the gather form
   of the n_idx_heads == 1 branch (:3413-3478), which the kernel also runs for
   several index heads, where the reference's ``_KLChunkFn`` (:3479-3496)
   computes the same KL densely;
5. ``sum(kl * valid) / (sum(valid) + 1e-6)`` over all chunks (:3497-3498, 3516).

Gradients reach the index projection through q_idx / idx_k; the teacher
(main q / k) is detached, as in the reference.  The diagnostic prints of the
reference (:3373-3386, :3500-3514) are kept; their counts stay on the device
until a print needs them.
"""

from __future__ import annotations

import torch

from . import kl as _kl
from . import ops
from ._lib import UnsupportedShape

_DTYPES = (torch.bfloat16, torch.float16)
SCORE_NEG = -1.0e9
ACT_CLAMP = 1.0e4


def _fold_heads(idx_q, idx_k):
    """(q [B*HI, T, d], keys [B*HI, Sk, d]) of idx_q [B, HI, T, d] and the
    shared idx_k [B, 1, Sk, d]."""
    B, HI, T, D = idx_q.shape
    Sk = idx_k.shape[2]
    keys = idx_k[:, 0] if HI == 1 else idx_k.expand(B, HI, Sk, D).reshape(B * HI, Sk, D)
    return idx_q.reshape(B * HI, T, D), keys


@torch.no_grad()
def indexer_forward(self, hidden_states, position_embeddings, past_key_values, position_ids, image_token_mask=None):
    """int64 [B, HI, q_len, topk] remote block ids of ``DeepseekV2Indexer.forward``
    (``self`` the indexer): the block max of q . k over each block's keys below
    the query's token window (j < max(pos - local_window + 1, 0)), image-bucket
    blocks only when the indexer is so configured (a row may then select
    nothing), then the top-k, -1 where the score is -inf.  The reference's
    per-chunk loop is one launch here (the rows are independent).  Raises
    UnsupportedShape for what the kernels do not take."""
    del position_embeddings                 # the reference projects without them as well (:3070)
    if not hidden_states.is_cuda:
        raise UnsupportedShape("indexer forward: host tensors")
    bs = int(self.block_size)
    idx_q, idx_k = self._project_index_qk(hidden_states, position_ids, past_key_values)
    if idx_q.dtype != idx_k.dtype or idx_q.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise UnsupportedShape("indexer forward: index q / k dtype")
    B, HI, T, D = idx_q.shape
    k_len = int(idx_k.shape[2])
    nblk = -(-k_len // bs)
    topk = self._remote_topk(nblk)
    if topk == 0:
        return torch.empty(B, HI, T, 0, dtype=torch.long, device=idx_q.device)
    q, keys = _fold_heads(idx_q, idx_k)
    pos = position_ids.to(idx_q.device)
    posh = pos.unsqueeze(1).expand(B, HI, T).reshape(B * HI, T)
    sc = ops.block_max_score(q, keys, posh, None, block_size=bs, num_key_blocks=nblk,
                             local_window=self.local_window).view(B, HI, T, nblk)
    if self.image_bucket_constraint and image_token_mask is not None:
        img_blk = self._build_image_block_allow_mask(image_token_mask, nblk)
        sc = sc.masked_fill(~img_blk[:, None, None, :], float("-inf"))
    return ops.topk_rows(sc, topk, invalid_at=float("-inf")).long()


@torch.no_grad()
def block_scores_indexer(router, idx_q, idx_k, q_pos, nblk):
    """[B, Lq, nblk] fp32 scores of the stage0 == "indexer" router: per block
    the max of q . k (clamped to +-1e4) over its keys j <= pos - local_window,
    SCORE_NEG for a block without one.  idx_q [B, Lq, d], idx_k [B, S, d]
    (the router's fp32 q / k; bf16 / fp16 also taken), q_pos [B, Lq]."""
    if not idx_q.is_cuda:
        raise UnsupportedShape("block scores: host tensors")
    S = int(idx_k.shape[1])
    if int(nblk) * int(router.block_size) < S:
        raise UnsupportedShape("block scores: nblk blocks do not cover the keys")
    sc = ops.block_max_score(idx_q, idx_k, q_pos, None, block_size=int(router.block_size), num_key_blocks=int(nblk),
                             local_window=int(router.local_window))
    return torch.where(sc == float("-inf"), torch.full_like(sc, SCORE_NEG), sc.clamp(-ACT_CLAMP, ACT_CLAMP))


def _is_packed(position_ids) -> bool:
    """A packed row restarts its positions at 0 past column 0
    (HF/packing_patch.py:48-56)."""
    if position_ids is None or position_ids.dim() != 2 or position_ids.shape[1] < 2:
        return False
    return bool((position_ids[:, 1:] == 0).any())


def check_supported(indexer, query_states, key_states, hidden_states) -> None:
    """Raise UnsupportedShape for the cases the kernels do not take (the caller
    then runs the model's own method)."""
    if not (hidden_states.is_cuda and query_states.is_cuda and key_states.is_cuda):
        raise UnsupportedShape("select_and_kl_loss: host tensors")
    if int(indexer.block_size) != 64:
        raise UnsupportedShape("select_and_kl_loss: block_size must be 64")
    if query_states.dtype not in _DTYPES or key_states.dtype != query_states.dtype:
        raise UnsupportedShape("select_and_kl_loss: main q / k must be bf16 or fp16")
    D = int(query_states.shape[-1])
    if D not in (64, 128) or int(key_states.shape[-1]) != D:
        raise UnsupportedShape("select_and_kl_loss: head dim must be 64 or 128")
    HQ, HKV, HI = int(query_states.shape[1]), int(key_states.shape[1]), int(indexer.num_heads)
    if HI <= 0 or HQ % HI or HQ % HKV:
        raise UnsupportedShape("select_and_kl_loss: head counts")
    nblk = -(-int(key_states.shape[2]) // 64)
    if indexer._remote_topk(nblk) > 64:
        raise UnsupportedShape("select_and_kl_loss: at most 64 remote blocks per row")


def select_and_kl_loss(self, hidden_states, query_states, key_states, position_embeddings, position_ids, scaling,
                       image_token_mask=None, image_token_page_ids=None, query_token_page_ids=None, *, pk=None):
    """(block_indices int64 [B, HI, Sq, topk], kl_loss fp32 scalar) of the
    reference method; ``self`` is the ``DeepseekV2Indexer``.  ``pk``: the model
    package's packing module, for its one-shot block-alignment warning.
    Raises UnsupportedShape (before any work) for what the kernels do not take."""
    del position_embeddings                 # the reference projects without them as well (:3256)
    check_supported(self, query_states, key_states, hidden_states)
    batch, q_len, _ = hidden_states.shape
    idx_q, idx_k = self._project_index_qk(hidden_states.detach(), position_ids, None)
    q_main = query_states.detach()
    k_main = key_states.detach()
    if idx_q.dtype != q_main.dtype or idx_k.dtype != q_main.dtype or idx_q.shape[-1] != q_main.shape[-1]:
        raise UnsupportedShape("select_and_kl_loss: index and main heads differ in dtype or head dim")
    n_idx_heads = int(self.num_heads)
    D = int(idx_q.shape[-1])
    bs = int(self.block_size)
    k_len = int(idx_k.shape[2])
    nblk = -(-k_len // bs)
    topk = self._remote_topk(nblk)
    dev = idx_q.device

    chunk = self.kl_chunk_size if self.kl_chunk_size and self.kl_chunk_size > 0 else q_len
    block_indices = torch.empty(batch, n_idx_heads, q_len, topk, dtype=torch.long, device=dev)
    total_kl = torch.zeros((), dtype=torch.float32, device=dev)
    total_cnt = torch.zeros((), dtype=torch.float32, device=dev)
    fallback_rows = torch.zeros((), dtype=torch.int64, device=dev)
    page_scope = (self.image_bucket_constraint and image_token_page_ids is not None
                  and query_token_page_ids is not None)
    packed = _is_packed(position_ids)
    if packed and pk is not None and hasattr(pk, "check_block_alignment"):
        pk.check_block_alignment(position_ids, bs)
    # idx_k is [B, 1, Sk, d]: one key set shared by the index heads
    keys = idx_k[:, 0] if n_idx_heads == 1 else \
        idx_k.expand(batch, n_idx_heads, k_len, D).reshape(batch * n_idx_heads, k_len, D)

    # passes of at least kl_chunk_size rows, as many as a 1 GiB fp32 score
    # buffer holds: the rows are independent, so the pass size only sets the
    # number of launches (small passes leave most of the GPU idle)
    step = min(q_len, max(chunk, (1 << 30) // max(1, 4 * batch * n_idx_heads * nblk)))
    for c0 in range(0, q_len, step):
        c1 = min(c0 + step, q_len)
        cq = c1 - c0
        if packed:
            pos_chunk = torch.arange(c0, c1, device=position_ids.device).view(1, -1).expand(batch, -1)
            seg_chunk = pos_chunk - position_ids[:, c0:c1]
        else:
            pos_chunk = position_ids[:, c0:c1]
            seg_chunk = None
        q_chunk = idx_q[:, :, c0:c1]

        with torch.no_grad():
            posh = pos_chunk.unsqueeze(1).expand(batch, n_idx_heads, cq).reshape(batch * n_idx_heads, cq)
            segh = None if seg_chunk is None else \
                seg_chunk.unsqueeze(1).expand(batch, n_idx_heads, cq).reshape(batch * n_idx_heads, cq)
            block_scores = ops.block_max_score(q_chunk.reshape(batch * n_idx_heads, cq, D), keys, posh, segh,
                                               block_size=bs, num_key_blocks=nblk,
                                               local_window=self.local_window).view(batch, n_idx_heads, cq, nblk)
            candidate = self._build_kl_candidate_mask(pos_chunk, nblk, image_token_mask, batch, cq,
                                                      image_token_page_ids=image_token_page_ids,
                                                      query_token_page_ids=query_token_page_ids)
            if c0 == 0 and self.image_bucket_constraint and not getattr(self, "_img_blk_kl_logged", False):
                self._img_blk_kl_logged = True
                if image_token_mask is not None:
                    img_blk = self._build_image_block_allow_mask(image_token_mask, nblk)
                    avg_img_blk = img_blk.float().sum(dim=-1).mean().item()
                    print(f"[ImageConstraint layer={self.layer_idx}] select_and_kl_loss() "
                          f"num_key_blocks={nblk} avg_image_blocks={avg_img_blk:.1f} "
                          f"image_block_ratio={avg_img_blk / nblk * 100:.1f}% "
                          f"(KL/selection candidates: image blocks; token-level local excluded)", flush=True)
            if topk == 0:
                continue
            scores_c = block_scores.masked_fill(~candidate.expand_as(block_scores), float("-inf"))
            short = (scores_c > float("-inf")).sum(dim=-1, keepdim=True) < topk
            scores_c = torch.where(short, block_scores, scores_c)
            bi = ops.topk_rows(scores_c, topk, invalid_at=float("-inf"))
            block_indices[:, :, c0:c1] = bi
            if image_token_mask is not None:
                fallback_rows += (bi < 0).all(dim=-1).sum()

        kl_rows, valid = _kl.gather_kl(q_chunk, idx_k, q_main[:, :, c0:c1], k_main, bi, pos_chunk, block_size=bs,
                                       local_window=self.local_window, scaling=scaling, seg=seg_chunk)
        v = valid.to(torch.float32)
        total_kl = total_kl + (kl_rows * v).sum()
        total_cnt = total_cnt + v.sum()

    self._kl_log_step = getattr(self, "_kl_log_step", 0) + 1
    if self.layer_idx == 2 and self._kl_log_step % self.kl_log_interval == 0:
        keep_avg = (total_kl.detach() / (total_cnt.detach() + 1e-6)).item() if total_cnt.item() > 0 else 0.0
        fb = f" fallback_queries={int(fallback_rows.item())}" if self.image_bucket_constraint else ""
        print(f"[KLMask layer={self.layer_idx} step={self._kl_log_step}] stage=sparse "
              f"image_bucket_constraint={self.image_bucket_constraint} page_image_scope={page_scope} "
              f"keep_avg_keys={keep_avg:.1f} valid_queries={int(total_cnt.item())}/{batch * n_idx_heads * q_len}"
              f"{fb}", flush=True)
    return block_indices, total_kl / (total_cnt + 1e-6)
