"""Page isolation + Page2D RoPE CPU oracle -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker.  The product path never
imports it.

Each function restates, on the CPU in numpy / plain Python, one reference
function of the metadata step that precedes block scoring and cites the
reference file:line it follows (``HF/x.py:N`` = ``hf-model-code/x.py``;
``WHL!p:N`` = ``sglang/srt/p`` inside the reference's SGLang wheel).

Pinning (``tests/test_page_pins.py``), none of which retypes these formulas:

* ``decode_meta_step``: run token by token over whole synthetic documents and
  compared with the whole-sequence scan formulation (cumsum / cummax) of
  ``PageIsolationState.step`` and ``_uocr_dash_decode_allow``'s prefill branch;
  the coordinates against a brute-force count of earlier tokens per page.
* ``decode_allow`` / ``block_bounds`` / ``candidate_mask_*``: against
  brute-force set membership ("some token of the block has page qp") on
  documents whose pages are contiguous runs, where the min/max form is exact.
* ``page2d_cos_sin``: the angles are single fp32 products (checked against
  ``torch`` fp32 multiplication), cos^2 + sin^2 = 1, the page_mod fold, and
  the 1D llama table when page_pairs carries the tail of the spectrum.
* ``rope_apply``: bit-exact against ``transformers``' llama
  ``apply_rotary_pos_emb`` evaluated by torch on the CPU in bf16 / fp16 / fp32
  (the library routine the HF indexer applies), plus rotation invariants.
"""

from __future__ import annotations

import math

import numpy as np

MM_PAD_SHIFT = 1_000_000          # WHL!…/page_state.py:19
INT16_MAX = 32767                 # WHL!…/page_state.py:16


# ----------------------------------------------------------------- state
class SlotState:
    """Per-slot page-isolation state (``PageIsolationState._ensure``,
    WHL!…/page_state.py:185-198)."""

    def __init__(self, num_slots: int):
        self.img_page = np.full(num_slots, -1, np.int32)
        self.marker_cum = np.zeros(num_slots, np.int32)
        self.img_run = np.zeros(num_slots, np.int32)
        self.prompt_pages = np.zeros(num_slots, np.int32)


class CoordState:
    """Per-row Page2D coordinate state (``PageCoordState._ensure``,
    WHL!…/page2d_rope.py:388-398)."""

    def __init__(self, rows: int, max_pages: int):
        self.st_marker = np.zeros(rows, np.int32)
        self.st_pp = np.zeros(rows, np.int32)
        self.cnt = np.zeros((rows, max_pages), np.int32)
        self.max_pages = max_pages


def _trunc_div(a: int, b: int) -> int:
    """Integer division rounding toward zero (Triton's ``//`` on ints)."""
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b > 0) else -q


def decode_meta_step(ids, block_table, seq_lens, slot_mapping, coord_row, st: SlotState, cs: CoordState,
                     image_token_id: int, page_token_id, per_page: int, block_size: int):
    """One-token decode update of the page state and the Page2D coordinates.

    ``_decode_meta_kernel``, WHL!…/decode_meta_triton.py:18-104 (one program
    per request, requests in order).  Mutates ``st`` / ``cs``; returns
    (q_page int32 [R], tok int64 [R], page int64 [R])."""
    R = len(seq_lens)
    n_slots = len(st.img_page)
    bt_w = block_table.shape[1]
    bs = block_size
    q_page = np.zeros(R, np.int32)
    tok = np.zeros(R, np.int64)
    page = np.zeros(R, np.int64)
    for r in range(R):
        tid = int(ids[r])
        is_img = tid >= MM_PAD_SHIFT or tid == image_token_id
        is_mark = page_token_id is not None and tid == page_token_id
        seq = int(seq_lens[r])
        prev_pos = seq - 2
        valid = prev_pos >= 0
        p = max(prev_pos, 0)
        blk = min(p // bs, bt_w - 1)
        phys = int(block_table[r, blk])
        prev_slot = min(max(phys * bs + p % bs, 0), n_slots - 1) if valid else 0
        prev_m = int(st.marker_cum[prev_slot]) if valid else 0
        prev_i = int(st.img_run[prev_slot]) if valid else 0
        prev_pp = int(st.prompt_pages[prev_slot]) if valid else 0
        marker = prev_m + int(is_mark)
        run = prev_i + int(is_img)
        img_page = (marker - 1 if marker > 0 else _trunc_div(run - 1, per_page)) if is_img else -1
        pp = max(marker if is_img else 0, prev_pp)
        resp = marker - 1 - pp
        resp = resp if resp >= 0 else -1
        q_page[r] = img_page if is_img else resp
        slot = min(max(int(slot_mapping[r]), 0), n_slots - 1)
        st.img_page[slot] = img_page
        st.marker_cum[slot] = marker
        st.img_run[slot] = run
        st.prompt_pages[slot] = pp
        last_blk = min(max(_trunc_div(seq - 1, bs), 0), bt_w - 1)
        tail_phys = int(block_table[r, last_blk])
        rem = seq % bs if seq >= 0 else -((-seq) % bs)
        if rem > 0:
            for off in range(rem, bs):
                st.img_page[min(max(tail_phys * bs + off, 0), n_slots - 1)] = -1
        row = int(coord_row[r])
        c_m = int(cs.st_marker[row]) + int(is_mark)
        c_p = max(c_m if is_img else 0, int(cs.st_pp[row]))
        c_resp = min(max(c_m - c_p, 0), c_p)
        cpage = min(max(c_resp, 0), cs.max_pages - 1)
        tok[r] = int(cs.cnt[row, cpage])
        page[r] = cpage
        cs.cnt[row, cpage] += 1
        cs.st_marker[row] = c_m
        cs.st_pp[row] = c_p
    return q_page, tok, page


def decode_allow(block_table, s_page, q_page, seq_lens, max_block: int, num_blocks: int, block_size: int):
    """Page-isolation candidate mask of decode rows, int8 [R, max_block].

    ``_decode_allow_kernel``, WHL!…/decode_meta_triton.py:107-163, with the
    width of ``decode_allow_fused`` (:330-351)."""
    R = len(q_page)
    bs = block_size
    W = min(max_block, block_table.shape[1])
    out = np.zeros((R, max_block), np.int8)
    for r in range(R):
        qp = int(q_page[r])
        seq = int(seq_lens[r])
        same = np.zeros(max_block, bool)
        for w in range(W):
            if w * bs >= seq:
                continue
            pg = min(max(int(block_table[r, w]), 0), num_blocks - 1)
            ip = s_page[pg * bs:(pg + 1) * bs].astype(np.int64)
            hi = int(np.where(ip >= 0, ip, -1).max())
            lo = int(np.where(ip >= 0, ip, INT16_MAX).min())
            lo = lo if hi >= 0 else -1
            same[w] = lo >= 0 and lo <= qp <= hi and qp >= 0
        open_row = qp < 0 or not same.any()
        out[r] = (same | open_row).astype(np.int8)
    return out


def local_union(allow, seq_lens, out, max_block: int, block_size: int, local_blocks: int):
    """Local window OR-ed into the candidate mask; writes ``out`` in place.

    ``_local_union_kernel``, WHL!…/decode_meta_triton.py:212-243."""
    R = len(seq_lens)
    a_w, o_w = allow.shape[1], out.shape[1]
    for r in range(R):
        q_blk = _trunc_div(int(seq_lens[r]) - 1, block_size)
        hi = min(max(q_blk, 0), max_block - 1)
        lo = min(max(q_blk - (local_blocks - 1), 0), max_block - 1)
        for w in range(min(max_block, o_w)):
            a = w < a_w and allow[r, w] != 0
            out[r, w] = 1 if (a or lo <= w <= hi) else 0
    return out


# ----------------------------------------------------------------- HF masks
def block_bounds(ids, nblk: int, block_size: int):
    """Per-block (min, max) page id, -1 where the block has none: int32 [B, nblk, 2].

    ``PageIsolationState.block_page_bounds`` WHL!…/page_state.py:315-328 and
    the prefill bmin / bmax of ``_uocr_dash_decode_allow``
    HF/modeling_unlimitedocr.py:498-510 (positions past the ids are -1)."""
    B, L = ids.shape
    out = np.full((B, nblk, 2), -1, np.int32)
    for b in range(B):
        for k in range(nblk):
            seg = ids[b, k * block_size:min((k + 1) * block_size, L)].astype(np.int64)
            seg = seg[seg >= 0]
            if seg.size:
                out[b, k] = (seg.min(), seg.max())
    return out


def candidate_mask_page_aware(image_token_page_ids, query_token_page_ids, pos_chunk, nblk: int,
                              block_size: int):
    """Same-page image blocks per query with the open-row fallback, bool [B, cq, nblk].

    ``_build_page_aware_image_block_mask`` HF/_sparse_base_impl.py:2629-2649
    (token-level equality, ids padded with -1 / cut to nblk*block_size) and the
    per-query fallback of ``_build_kl_candidate_mask`` :2733-2736."""
    B, k_len = image_token_page_ids.shape
    S = query_token_page_ids.shape[1]
    span = nblk * block_size
    kp = np.full((B, span), -1, np.int64)
    n = min(k_len, span)
    kp[:, :n] = image_token_page_ids[:, :n]
    kp = kp.reshape(B, nblk, block_size)
    pos = np.clip(pos_chunk, 0, S - 1)
    qp = np.take_along_axis(query_token_page_ids, pos, axis=1)             # [B, cq]
    same = ((qp[:, :, None, None] >= 0) & (qp[:, :, None, None] == kp[:, None])).any(-1)
    has = same.any(-1, keepdims=True)
    return np.where(has, same, True)


def candidate_mask_image(image_token_mask, nblk: int, block_size: int, cq: int):
    """All image blocks (any page) with the open-row fallback, bool [B, cq, nblk].

    ``_build_image_block_allow_mask`` HF/_sparse_base_impl.py:2392-2402, the
    broadcast of ``_build_kl_candidate_mask`` :2726-2729 and its fallback :2733-2736."""
    B, Sk = image_token_mask.shape
    span = nblk * block_size
    m = np.zeros((B, span), bool)
    n = min(Sk, span)
    m[:, :n] = image_token_mask[:, :n]
    img_blk = m.reshape(B, nblk, block_size).any(-1)
    cand = np.broadcast_to(img_blk[:, None, :], (B, cq, nblk))
    has = cand.any(-1, keepdims=True)
    return np.where(has, cand, True)


# ----------------------------------------------------------------- Page2D RoPE
def page2d_freqs(dim: int, base_tok: float, base_page: float, page_pairs: int, tok_freq_mode: str = "resample"):
    """Frequency tables (fp32), ``PageRope2D.__init__`` WHL!…/page2d_rope.py:39-73 =
    ``DeepseekV2IndexerRotary2D.__init__`` HF/_sparse_base_impl.py:2019-2036,
    evaluated in float64 and rounded once (the reference's fp32 pow may differ
    by an ulp; the product path takes the tables as inputs)."""
    half = dim // 2
    n_tok = half - page_pairs
    ar = np.arange(n_tok, dtype=np.float64)
    if tok_freq_mode == "truncate":
        inv_tok = 1.0 / (float(base_tok) ** (ar * 2 / dim))
    else:
        inv_tok = 1.0 / (float(base_tok) ** (ar / n_tok))
    inv_page = 1.0 / (float(base_page) ** (np.arange(page_pairs, dtype=np.float64) / page_pairs))
    return inv_tok.astype(np.float32), inv_page.astype(np.float32)


def page2d_cos_sin(tok, page, inv_tok, inv_page, dim: int, page_mod: int = 0):
    """cos / sin [T, dim] in float64 of the fp32 angles.

    ``PageRope2D.cos_sin`` WHL!…/page2d_rope.py:108-127 and
    ``DeepseekV2IndexerRotary2D.forward`` HF/_sparse_base_impl.py:2046-2061:
    ang = [t * inv_tok, p * inv_page] (fp32 products), emb = cat(ang, ang)."""
    t = np.asarray(tok, np.int64).astype(np.float32)[:, None]
    p = np.asarray(page, np.int64)
    if page_mod > 0:
        p = np.remainder(p, page_mod)
    p = p.astype(np.float32)[:, None]
    ang = np.concatenate([t * inv_tok[None, :], p * inv_page[None, :]], axis=1).astype(np.float32)
    emb = np.concatenate([ang, ang], axis=1).astype(np.float64)
    return np.cos(emb), np.sin(emb)


def round_to(x, dtype: str):
    """Round float32 values to bf16 / fp16 / fp32 (RNE), returned as float32."""
    x = np.asarray(x, np.float32)
    if dtype == "f32":
        return x
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def rope_apply(x, cos, sin, dtype: str):
    """x * cos + rotate_half(x) * sin with each product and the sum rounded to
    ``dtype`` (the eager torch order): ``_rope2d_torch`` WHL!…/page2d_rope.py:130-141,
    its bit-identical kernel :148-189, and llama ``apply_rotary_pos_emb`` as the
    HF indexer applies it (HF/_sparse_base_impl.py:3049).

    x [..., hd] float32 holding dtype values; cos / sin broadcastable to x."""
    x = np.asarray(x, np.float32)
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    a = round_to(x * np.asarray(cos, np.float32), dtype)
    b = round_to(rot * np.asarray(sin, np.float32), dtype)
    return round_to((a + b).astype(np.float32), dtype)


def angle_close(a, b):
    """|a - b| as angles (helper for the identity checks)."""
    d = np.remainder(np.asarray(a) - np.asarray(b) + math.pi, 2 * math.pi) - math.pi
    return np.abs(d)
