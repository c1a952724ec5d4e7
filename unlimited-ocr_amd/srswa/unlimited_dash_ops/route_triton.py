"""Drop-in for ``sglang.srt.layers.attention.unlimited_dash_ops.route_triton``
(WHL!layers/attention/unlimited_dash_ops/route_triton.py): the serving DASH
router of the Unlimited-OCR v2 backend -- page summaries, remote block scores
and 1.5-entmax selection capped by a hard top-k budget -- on the MI355X
kernels.

Same names, keyword-only signatures, caller-owned outputs and return values as
the reference (the backend imports them at
WHL!layers/attention/unlimited_ocr_v2_backend.py:45-54):

* ``route_decode_triton`` / ``route_prefill_triton``: scores off the summary
  cache (``srswa_kbar_scores``) then the router (``srswa_route_serve``), which
  packs each row's active blocks ascending into ``out_idx`` / ``out_bias``
  (-1 / 0.0 in the rest of the first M slots).
* ``kbar_refresh_tail_triton``: the plan's page summaries (``srswa_kbar_plan``).
* ``win_bounds_decode``: the per-row remote page span (``srswa_win_bounds``).
* ``kbar_tail_plan`` / ``kbar_all_plan`` / ``prefill_row2req``: the plan
  helpers (torch index arithmetic on the device, like the reference's).

The reference narrows its score and entmax scans to the page-mask window
(``entmax_base`` / ``entmax_fit`` / ``entmax_width`` / ``score_buf_win`` /
``bounds``).  The window always holds every candidate block (all allowed
remote blocks lie in [lo, hi], and without an allowed block it spans every
live remote block), so the selection is the full-width one; these arguments
are accepted and the kernels scan the full width.  The reference's tiled form
(block-table width >= 8192) sums tau's bisection in fp32 instead of fp64; the
block ids are the same, and the bias can differ in its last bits there.
Every tensor must live on the GPU.
"""

from __future__ import annotations

import torch

from .. import ops

# The tau bisection reaches fp32 resolution after 24 steps; the budget
# bisection keeps 40 (route_triton.py:11-14).
ENTMAX_ITERS = 24
ENTMAX_ITERS_CAP = 40
# Width of the backend's decode page-window scan (route_triton.py:16).
SCAN_TILE = 128

SCORE_NEG = -1.0e9
ENTMAX_NEG = -1.0e4
ACT_CLAMP = 1.0e4


def _want_tiled(bw_full: int) -> bool:
    """The reference switches to its tiled router at 8192 score columns."""
    return bw_full >= 8192


def _slots(out_idx, topm, out_slots):
    m = min(int(out_slots or topm), int(out_idx.shape[-1]))
    assert m > 0 and m & (m - 1) == 0, f"out_slots must be a power of two, got {m}"
    return m


def _budget(budget, m):
    return max(1, min(int(budget or m), m))


@torch.no_grad()
def win_bounds_decode(*, allow, seq_lens, lo, hi, fit, max_block: int, block_size: int, local_blocks: int,
                      decode_query_len: int, tile: int):
    """Fill ``lo`` / ``hi`` / ``fit`` (int32 / int32 / int8 [nd]) in place from
    the page mask ``allow`` [>= nd, WQ] (bool / int8; the first nd rows)."""
    if int(lo.numel()) <= 0:
        return
    ops.win_bounds(allow, seq_lens, lo, hi, fit, max_block=max_block, block_size=block_size,
                   local_blocks=local_blocks, dql=decode_query_len, tile=tile)


@torch.no_grad()
def kbar_tail_plan(*, block_table, seq_lens, block_size: int, tail_pages: int, device, out=None):
    """(pages int64, tok int32), flattened [R * tail_pages]: each request's last
    ``tail_pages`` logical blocks (counting back from its last live one, never
    below block 0) and the live keys each holds.  ``out``: preallocated pair
    (used when large enough)."""
    bs = int(block_size)
    sl = seq_lens.to(device=device, dtype=torch.int64)
    last = torch.clamp((sl + bs - 1) // bs - 1, min=0)
    blk = torch.clamp(last[:, None] - torch.arange(int(tail_pages), device=device)[None, :], min=0)
    width = int(block_table.shape[1])
    pages = torch.gather(block_table[:, :width].to(torch.int64), 1, torch.clamp(blk, max=width - 1)).reshape(-1)
    tok = torch.clamp(sl[:, None] - blk * bs, 0, bs).reshape(-1).to(torch.int32)
    n = pages.numel()
    if out is None or out[0].shape[0] < n:
        return pages.contiguous(), tok.contiguous()
    out[0][:n].copy_(pages)
    out[1][:n].copy_(tok)
    return out[0][:n], out[1][:n]


@torch.no_grad()
def kbar_all_plan(*, block_table, seq_lens, context_lens, block_size: int, max_block: int, max_query_len: int,
                  device, out=None):
    """(pages int64, tok int32) of the pages a prefill step changes: per
    request, from the block holding its first new token, ceil(max_query_len /
    block_size) + 1 blocks (blocks past the live ones get tok 0 and are
    skipped by the refresh).  ``out``: preallocated pair."""
    bs = int(block_size)
    W = min(int(max_block), int(block_table.shape[1]))
    width = min(W, -(-int(max_query_len) // bs) + 1)
    sl = seq_lens.to(device=device, dtype=torch.int64)
    ctx = context_lens.to(device=device, dtype=torch.int64)
    blk = (ctx // bs)[:, None] + torch.arange(width, device=device)[None, :]
    pages = torch.gather(block_table[:, :W].to(torch.int64), 1, torch.clamp(blk, max=W - 1)).reshape(-1)
    tok = torch.clamp(sl[:, None] - blk * bs, 0, bs).reshape(-1).to(torch.int32)
    if out is not None:
        p_buf, t_buf = out
        n = pages.numel()
        assert p_buf.shape[0] >= n and t_buf.shape[0] >= n
        p_buf[:n].copy_(pages)
        t_buf[:n].copy_(tok)
        return p_buf[:n], t_buf[:n]
    return pages.contiguous(), tok.contiguous()


@torch.no_grad()
def prefill_row2req(*, cu_seqlens_q, device, out=None, total_q=None):
    """int32 [total_q]: the request of every prefill query row (the counts come
    from ``cu_seqlens_q``, which takes one host read, as in the reference)."""
    cu = cu_seqlens_q.to(device=device, dtype=torch.int64)
    counts = cu[1:] - cu[:-1]
    row2req = torch.repeat_interleave(torch.arange(counts.numel(), device=device), counts).to(torch.int32)
    if out is not None:
        n = row2req.shape[0]
        assert out.shape[0] >= n
        out[:n].copy_(row2req)
        return out[:n]
    return row2req.contiguous()


@torch.no_grad()
def kbar_refresh_tail_triton(*, kv_cache, k_bar, block_table, seq_lens, head_cls, block_size: int,
                             tail_pages: int = 1, plan=None):
    """Recompute the summaries of the plan's pages (default: every request's
    last ``tail_pages`` pages) into ``k_bar`` [num_pages, d] fp32."""
    if plan is None:
        plan = kbar_tail_plan(block_table=block_table, seq_lens=seq_lens, block_size=block_size,
                              tail_pages=tail_pages, device=k_bar.device)
    pages, tok = plan
    ops.kbar_plan(kv_cache, head_cls, pages, tok, k_bar)


@torch.no_grad()
def route_decode_triton(*, idx_q, k_bar, block_table, seq_lens, image_allow, out_idx, out_bias, max_block: int,
                        block_size: int, local_blocks: int, decode_query_len: int, idx_scale: float,
                        prior_floor: float, sigma: float, topm: int, score_buf=None, budget: int | None = None,
                        out_slots: int | None = None, entmax_base=None, entmax_fit=None, entmax_width: int = 0,
                        score_buf_win=None, bounds=None):
    """Decode routing into the caller's ``out_idx`` / ``out_bias`` [nd, >= M];
    returns M, the packed width.  Scores land in ``score_buf[:nd, :W]`` when it
    is large enough (else in fresh memory)."""
    nd = int(idx_q.shape[0])
    W = min(int(max_block), int(block_table.shape[1]))
    M = _slots(out_idx, topm, out_slots)
    bw_full = 1 << (max(W, 1) - 1).bit_length()
    if entmax_base is not None and entmax_fit is not None and 0 < int(entmax_width) < bw_full:
        assert int(entmax_width) & (int(entmax_width) - 1) == 0, \
            f"entmax_width must be a power of two, got {entmax_width}"
    del score_buf_win, bounds                # the full-width scan selects the same blocks
    if score_buf is not None and score_buf.shape[0] >= nd and score_buf.shape[1] >= W:
        sc = score_buf[:nd, :W]
    else:
        sc = torch.empty(nd, W, dtype=torch.float32, device=idx_q.device)
    if nd == 0:
        return M
    ops.kbar_scores(idx_q, k_bar, block_table, seq_lens, width=W, page_size=block_size, local_blocks=local_blocks,
                    dql=max(1, int(decode_query_len)), out=sc)
    ops.route_serve(sc, image_allow, out_idx, out_bias, K=_budget(budget, M), M=M, idx_scale=idx_scale,
                    prior_floor=prior_floor, inv_sigma=1.0 / sigma)
    return M


@torch.no_grad()
def route_prefill_triton(*, idx_q, k_bar, block_table, seq_lens, cu_seqlens_q, context_lens, row2req, image_allow,
                         out_idx, out_bias, max_block: int, block_size: int, local_blocks: int, idx_scale: float,
                         prior_floor: float, sigma: float, topm: int, budget: int | None = None, q_chunk: int = 2048,
                         out_slots: int | None = None, score_buf: torch.Tensor | None = None):
    """Chunked prefill routing into the caller's ``out_idx`` / ``out_bias``
    [total_q, >= M].  Returns (M, the last chunk's scores, that chunk's first
    query row), as the reference does."""
    dev = idx_q.device
    total_q = int(idx_q.shape[0])
    W = min(int(max_block), int(block_table.shape[1]))
    M = _slots(out_idx, topm, out_slots)
    QC = max(1, min(int(q_chunk), total_q))
    if score_buf is not None:
        assert score_buf.dtype == torch.float32
        sc = score_buf
    else:
        sc = torch.empty(QC, W, dtype=torch.float32, device=dev)
    K = _budget(budget, M)
    off = 0
    for off in range(0, total_q, QC):
        n = min(QC, total_q - off)
        sc_v = sc[:n, :W]
        ops.kbar_scores(idx_q[off:off + n], k_bar, block_table, seq_lens, width=W, page_size=block_size,
                        local_blocks=local_blocks, row_req=row2req, cu_q=cu_seqlens_q, ctx=context_lens,
                        row_off=off, out=sc_v)
        img = None if image_allow is None else image_allow[off:off + n]
        ops.route_serve(sc_v, img, out_idx[off:off + n], out_bias[off:off + n], K=K, M=M, idx_scale=idx_scale,
                        prior_floor=prior_floor, inv_sigma=1.0 / sigma)
    return M, sc[:min(QC, total_q - off)], off
