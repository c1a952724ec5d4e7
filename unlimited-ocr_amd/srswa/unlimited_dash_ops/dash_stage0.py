"""Drop-in for ``sglang.srt.layers.attention.unlimited_dash_ops.dash_stage0``:
``KBarCache``, ``headcls_scores_prefill``, ``headcls_scores_decode``
(WHL!layers/attention/unlimited_dash_ops/dash_stage0.py:62-199: one fp32 head_cls
summary per KV page, decode scores off the cache), on the MI355X summary kernels.
"""

from __future__ import annotations

import torch

from .. import ops


class KBarCache:
    """One fp32 ``head_cls`` summary per KV page (dash_stage0.py:106-148).

    Prefill fills the used pages, decode refreshes each request's tail pages;
    like the reference, prefix-shared pages are not supported."""

    def __init__(self, num_pages: int, dim: int, device, dtype=torch.float32):
        if dtype != torch.float32:
            raise ValueError("the summary cache is fp32")
        self.k_bar = torch.zeros(num_pages, dim, dtype=dtype, device=device)

    def put(self, pages: torch.Tensor, k_bar: torch.Tensor) -> None:
        """Write summaries computed elsewhere for the given pages."""
        self.k_bar[pages] = k_bar.to(self.k_bar.dtype)

    @torch.no_grad()
    def refresh_tail(self, *, kv_cache, block_table, seq_lens, head_cls, block_size: int,
                     tail_pages: int = 2) -> None:
        """Recompute the last ``tail_pages`` summaries of every request (no host sync)."""
        if kv_cache.shape[1] != int(block_size):
            raise ValueError(f"page size {kv_cache.shape[1]} != block_size {block_size}")
        ops.kbar_pages(kv_cache, head_cls, block_table, seq_lens, self.k_bar, tail_blocks=max(1, int(tail_pages)))


@torch.no_grad()
def headcls_scores_prefill(*, idx_q, kv_cache, block_table, cu_seqlens_q, seq_lens, context_lens, head_cls,
                           max_block, block_size, local_blocks, q_chunk=2048, cache=None):
    """Prefill block scores [1, total_q, max_block] fp32 (SCORE_NEG elsewhere);
    the page summaries land in ``cache`` when given.  idx_q [total_q, d] (one
    router head), kv_cache [num_pages, block_size, d]."""
    del q_chunk
    dev = idx_q.device
    num_pages, page, d = kv_cache.shape
    if page != int(block_size):
        raise ValueError(f"page size {page} != block_size {block_size}")
    kbar = cache.k_bar if cache is not None else torch.zeros(num_pages, d, dtype=torch.float32, device=dev)
    ops.kbar_pages(kv_cache, head_cls, block_table, seq_lens, kbar)
    cu = cu_seqlens_q.to(device=dev, dtype=torch.int64)
    total_q = idx_q.shape[0]
    n = torch.arange(total_q, device=dev)
    req = torch.searchsorted(cu[1:], n, right=True)                  # request of each query row
    pos = context_lens.to(device=dev, dtype=torch.int64)[req] + (n - cu[req])
    width = min(int(max_block), block_table.shape[1])
    sc = torch.full((1, total_q, int(max_block)), -1.0e9, dtype=torch.float32, device=dev)
    ops.kbar_scores(idx_q, kbar, block_table, seq_lens, width=width, page_size=page, local_blocks=local_blocks,
                    row_req=req, row_pos=pos, out=sc[0, :, :width])
    return sc


@torch.no_grad()
def headcls_scores_decode(*, idx_q, cache, block_table, seq_lens, max_block, block_size, local_blocks,
                          decode_query_len, req_chunk=64):
    """Decode block scores [1, R * decode_query_len, max_block] fp32 off the
    summary cache (SCORE_NEG elsewhere); no host sync."""
    del req_chunk
    dql = max(1, int(decode_query_len))
    R = int(seq_lens.shape[0])
    width = min(int(max_block), block_table.shape[1])
    out = torch.empty((1, R * dql, int(max_block)), dtype=torch.float32, device=idx_q.device)
    if width < int(max_block):            # the kernel writes every column below width
        out[..., width:] = -1.0e9
    ops.kbar_scores(idx_q, cache.k_bar, block_table, seq_lens, width=width, page_size=int(block_size),
                    local_blocks=local_blocks, dql=dql, out=out[0, :, :width])
    return out
