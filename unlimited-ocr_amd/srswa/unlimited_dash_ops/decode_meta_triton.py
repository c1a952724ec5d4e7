"""Drop-in for ``sglang.srt.layers.attention.unlimited_dash_ops.decode_meta_triton``:
the fused one-token decode metadata of page isolation and Page2D RoPE
(WHL!layers/attention/unlimited_dash_ops/decode_meta_triton.py:246-422), on the
MI355X page kernels.

Same names, keyword arguments, output buffers and return values as the
reference.  ``page_state`` / ``coord_state`` are the serving backend's
``PageIsolationState`` / ``PageCoordState`` objects (duck-typed: the per-slot
and per-row int32 state tensors, ``_ensure`` and the coordinate state's
``_rows`` row allocation, which stays the caller's torch code).
"""

from __future__ import annotations

import torch

from .. import page_ops


class _LayoutShim:
    """The two fields ``PageCoordState._rows`` reads, built from decode inputs
    (WHL!…/decode_meta_triton.py:425-434): a decode request never starts at
    position 0, so ``start_pos`` = seq_len - 1."""

    __slots__ = ("block_table", "start_pos")

    def __init__(self, block_table, seq_lens, block_size):
        self.block_table = block_table
        self.start_pos = seq_lens.to(torch.int64) - 1


@torch.no_grad()
def decode_meta_fused(*, input_ids, block_table, seq_lens, slot_mapping, page_state, coord_state, num_slots: int,
                      block_size: int, out_q_page=None, out_tok=None, out_page=None):
    """Page state and Page2D coordinates for one-token decode; returns
    ``(q_page [R] int32, (tok [R] int64, page [R] int64))``."""
    device = input_ids.device
    page_state._ensure(num_slots, device)
    coord_state._ensure(device)
    row = coord_state._rows(_LayoutShim(block_table, seq_lens, block_size))
    q_page, tok, page = page_ops.page_decode_meta(
        input_ids, block_table, seq_lens, slot_mapping, row,
        s_page=page_state._slot_img_page, s_mark=page_state._slot_marker_cum, s_run=page_state._slot_img_run,
        s_pp=page_state._slot_prompt_pages, c_mark=coord_state.st_marker, c_pp=coord_state.st_pp,
        c_cnt=coord_state.cnt, image_token_id=page_state.image_token_id, page_token_id=page_state.page_token_id,
        per_page=page_state.per_page_image_tokens, block_size=block_size, n_slots=num_slots,
        out_q_page=out_q_page, out_tok=out_tok, out_page=out_page)
    # the backend's one-shot diagnostic reads this; the fused path leaves it unset
    page_state._last_img_run_max = None
    return q_page, (tok, page)


@torch.no_grad()
def decode_allow_fused(*, block_table, page_state, q_page, seq_lens, max_block: int, num_blocks: int,
                       block_size: int, out=None):
    """Page-isolation candidate mask ``[R, max_block]`` int8 (1 = candidate)."""
    return page_ops.page_decode_allow(block_table, page_state._slot_img_page, q_page, seq_lens,
                                      max_block=max_block, num_blocks=num_blocks, block_size=block_size, out=out)


@torch.no_grad()
def cos_sin_2d_fused(*, rope, tok_pos, page_pos, dtype, out_cos, out_sin):
    """A Page2D rotary's cos / sin table written into the caller's buffers."""
    inv_tok, inv_page = rope._freqs(tok_pos.device)
    return page_ops.page2d_cos_sin(tok_pos, page_pos, inv_tok, inv_page, dim=int(rope.dim),
                                   page_mod=int(rope.page_mod), dtype=dtype, out_cos=out_cos, out_sin=out_sin)


@torch.no_grad()
def local_union_fused(*, allow, seq_lens, out, max_block: int, block_size: int, local_blocks: int):
    """The local window OR-ed into ``allow``, written as int8 into ``out``."""
    return page_ops.page_local_union(allow, seq_lens, out, max_block=max_block, block_size=block_size,
                                     local_blocks=local_blocks)
