"""Drop-in for ``sglang.srt.layers.attention.unlimited_dash_ops.attend_triton``:
``dash_sparse_attn`` (the paged bias-aware prefill K10,
WHL!layers/attention/unlimited_dash_ops/attend_triton.py:521-597) on the
matrix-core prefill kernel, and ``dash_sparse_attn_decode`` (:600-715, the
paged bias-aware decode with split-K and merge) on the MI355X decode kernel.

Same names, arguments and in-place output convention as the reference; every
tensor must live on the GPU (no host path).
"""

from __future__ import annotations

import torch

from .. import ops

SPARSE_BLOCK_SIZE = 128     # fallback page size, WHL!layers/attention/unlimited_dash_ops/common.py:10


def dash_sparse_attn(q, k_cache, v_cache, topk_idx, blk_bias, block_table, cu_seqlens_q, seq_lens, prefix_lens,
                     max_query_len, num_kv_heads, sm_scale, output, local_blocks=0,
                     sparse_block_size=SPARSE_BLOCK_SIZE):
    """Bias-aware block-sparse prefill over the paged cache, written into ``output``.

    q [total_q, num_heads, D]; k_cache, v_cache [num_pages, page_size,
    num_kv_heads, D]; topk_idx / blk_bias [num_kv_heads, total_q, K] (ids packed
    at the front, -1 after); block_table [num_reqs, max_blocks]; cu_seqlens_q
    [num_reqs + 1]; seq_lens / prefix_lens [num_reqs] (request r's query t sits
    at key prefix_lens[r] + t).  Window: the last local_blocks * page_size keys
    of each query; remote: the selected blocks' keys before it, plus the bias."""
    if k_cache.shape[2] != int(num_kv_heads):
        raise ValueError(f"k_cache has {k_cache.shape[2]} kv heads, num_kv_heads={num_kv_heads}")
    if k_cache.shape[1] != int(sparse_block_size):
        raise ValueError(f"page size {k_cache.shape[1]} != sparse_block_size {sparse_block_size}")
    if blk_bias is not None:
        assert blk_bias.shape == topk_idx.shape, (blk_bias.shape, topk_idx.shape)
        assert blk_bias.dtype == torch.float32, blk_bias.dtype
    ops.gather_fwd_paged(q, k_cache, v_cache, topk_idx, blk_bias, block_table, cu_seqlens_q, seq_lens, prefix_lens,
                         max_query_len, local_blocks=local_blocks, scale=sm_scale, out=output)
    return None


def dash_sparse_attn_decode(q, k_cache, v_cache, topk_idx, blk_bias, block_table, seq_lens, num_kv_heads,
                            sm_scale, output, decode_query_len, local_blocks=0,
                            sparse_block_size=SPARSE_BLOCK_SIZE, chunk_width=None, cg_rows=None):
    """Bias-aware block-sparse decode over the paged cache, written into ``output``.

    q [total_q, num_heads, D]; k_cache, v_cache [num_pages, page_size,
    num_kv_heads, D]; topk_idx / blk_bias [num_kv_heads, total_q, K];
    block_table [num_reqs, max_blocks]; seq_lens [num_reqs].  One page is one
    sparse block (``sparse_block_size`` must equal the page size).
    ``chunk_width`` / ``cg_rows`` (the reference's split-K sizing hints) are
    accepted and unused: the split and its scratch are sized by the kernel."""
    del chunk_width, cg_rows
    if k_cache.shape[2] != int(num_kv_heads):
        raise ValueError(f"k_cache has {k_cache.shape[2]} kv heads, num_kv_heads={num_kv_heads}")
    if k_cache.shape[1] != int(sparse_block_size):
        raise ValueError(f"page size {k_cache.shape[1]} != sparse_block_size {sparse_block_size}")
    ops.gather_decode_paged(q, k_cache, v_cache, topk_idx, blk_bias, block_table, seq_lens,
                            decode_query_len=decode_query_len, local_blocks=local_blocks, scale=sm_scale,
                            out=output)
    return None
