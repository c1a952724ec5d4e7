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


# ----------------------------------------------------------------- multi-token steps
def _seg_scan(vals, q_start, T, op, init):
    """Per-request inclusive scan (request r owns [q_start[r], q_start[r+1]),
    the tokens past q_start[R] continue request R - 1) seeded with init[r]."""
    out = np.zeros(T, np.int64)
    R = len(q_start) - 1
    for r in range(R):
        lo = int(q_start[r])
        hi = T if r == R - 1 else int(q_start[r + 1])
        acc = int(init[r])
        for t in range(lo, hi):
            acc = op(acc, int(vals[t]))
            out[t] = acc
    return out


def _req_of(q_start, T):
    R = len(q_start) - 1
    req = np.zeros(T, np.int64)
    for r in range(R):
        hi = T if r == R - 1 else int(q_start[r + 1])
        req[int(q_start[r]):hi] = r
    return req


def _generated(T, q_start, start_pos, gen_start, num_decode_tokens):
    """``generated_mask`` WHL!…/page_state.py:56-62."""
    req = _req_of(q_start, T)
    t = np.arange(T)
    gen = t < int(num_decode_tokens)
    if gen_start is not None:
        abs_pos = np.asarray(start_pos)[req] + (t - np.asarray(q_start)[req])
        gen = gen | (abs_pos >= np.asarray(gen_start)[req])
    return gen


def page_step(ids, q_start, start_pos, block_table, slot_mapping, st: SlotState, image_token_id: int,
              page_token_id, per_page: int, block_size: int, num_decode_tokens: int = 0, gen_start=None):
    """Multi-token ``PageIsolationState.step`` (WHL!…/page_state.py:218-313):
    the carry-in of ``_carry`` (:200-216), the per-request scans, the page
    rules and the per-slot scatter, then the stale-tail reset.  Mutates
    ``st``; returns q_page int32 [T]."""
    ids = np.asarray(ids, np.int64)
    T = len(ids)
    R = len(q_start) - 1
    n = len(st.img_page)
    bs = block_size
    bt_w = block_table.shape[1]
    is_img = (ids >= MM_PAD_SHIFT) | (ids == image_token_id)
    is_mark = np.zeros(T, bool) if page_token_id is None else ids == page_token_id
    pm, pi, ppp = np.zeros(R, np.int64), np.zeros(R, np.int64), np.zeros(R, np.int64)
    for r in range(R):
        p = int(start_pos[r]) - 1
        if p >= 0:
            blk = min(p // bs, bt_w - 1)
            slot = min(max(int(block_table[r, blk]) * bs + p % bs, 0), n - 1)
            pm[r], pi[r], ppp[r] = st.marker_cum[slot], st.img_run[slot], st.prompt_pages[slot]
    marker = _seg_scan(is_mark.astype(np.int64), q_start, T, lambda a, b: a + b, pm)
    run = _seg_scan(is_img.astype(np.int64), q_start, T, lambda a, b: a + b, pi)
    pp = _seg_scan(np.where(is_img, marker, 0), q_start, T, max, ppp)
    img_page = np.where(marker > 0, marker - 1, (run - 1) // per_page)
    img_page = np.where(is_img, img_page, -1)
    gen = _generated(T, q_start, start_pos, gen_start, num_decode_tokens)
    prefill_page = np.where(marker > pp, marker - 1, -1)
    resp = marker - 1 - pp
    resp = np.where(resp >= 0, resp, -1)
    q_page = np.where(is_img, img_page, np.where(gen, resp, prefill_page)).astype(np.int32)
    for t in range(T):
        sl = min(max(int(slot_mapping[t]), 0), n - 1)
        st.img_page[sl] = img_page[t]
        st.marker_cum[sl] = marker[t]
        st.img_run[sl] = run[t]
        st.prompt_pages[sl] = pp[t]
    for r in range(R):
        end = int(start_pos[r]) + int(q_start[r + 1]) - int(q_start[r])
        rem = end % bs
        if rem > 0:
            blk = min(max((end - 1) // bs, 0), bt_w - 1)
            phys = int(block_table[r, blk])
            for off in range(rem, bs):
                st.img_page[min(max(phys * bs + off, 0), n - 1)] = -1
    return q_page


def coord_step(ids, q_start, start_pos, rows, cs: CoordState, image_token_id: int, page_token_id,
               num_decode_tokens: int = 0, gen_start=None):
    """The scans, ranks and carry of ``PageCoordState.step``
    (WHL!…/page2d_rope.py:534-620) for given state rows: marker / pp scans
    seeded by the row's carry, the page rule, tok = the row's count plus the
    rank among the request's earlier tokens of that page (stable sort),
    then the carry written back.  Mutates ``cs``; returns (tok, page, marker, pp)."""
    ids = np.asarray(ids, np.int64)
    T = len(ids)
    R = len(q_start) - 1
    pages = cs.max_pages
    is_img = (ids >= MM_PAD_SHIFT) | (ids == image_token_id)
    is_mark = np.zeros(T, bool) if page_token_id is None else ids == page_token_id
    rows = np.asarray(rows, np.int64)
    marker = _seg_scan(is_mark.astype(np.int64), q_start, T, lambda a, b: a + b, cs.st_marker[rows])
    pp = _seg_scan(np.where(is_img, marker, 0), q_start, T, max, cs.st_pp[rows])
    gen = _generated(T, q_start, start_pos, gen_start, num_decode_tokens)
    in_prefill = (~gen) & (is_img | (marker > pp))
    resp = np.minimum(np.maximum(marker - pp, 0), pp)
    page = np.clip(np.where(in_prefill, marker, resp), 0, pages - 1)
    req = _req_of(q_start, T)
    flat = req * pages + page
    order = np.argsort(flat, kind="stable")
    rank = np.zeros(T, np.int64)
    prev, start = None, 0
    for i, t in enumerate(order):
        if flat[t] != prev:
            prev, start = flat[t], i
        rank[t] = i - start
    cnt_in = cs.cnt[rows]
    tok = cnt_in[req, page] + rank
    for r in range(R):
        lo, hi = int(q_start[r]), int(q_start[r + 1])
        if hi <= lo:
            continue
        row = int(rows[r])
        for t in range(lo, hi):
            cs.cnt[row, page[t]] += 1
        cs.st_marker[row] = marker[hi - 1]
        cs.st_pp[row] = pp[hi - 1]
    return tok.astype(np.int64), page.astype(np.int64), marker.astype(np.int32), pp.astype(np.int32)


def page_aware_ids(source_ids, image_token_id: int, page_token_id: int, key_length: int, per_page: int,
                   page_scope_prefill: bool = True):
    """``DeepseekV2Indexer._build_page_aware_ids`` (HF/_sparse_base_impl.py:2404-2502)
    without its one-shot diagnostic print: (image_token_mask, image_token_page_ids,
    query_token_page_ids) [B, key_length], or (None, None, None)."""
    ids = np.asarray(source_ids, np.int64)[:, :key_length]
    if ids.shape[1] < key_length:
        ids = np.pad(ids, ((0, 0), (0, key_length - ids.shape[1])), constant_values=-1)
    B, S = ids.shape
    img = ids == image_token_id
    mk = ids == page_token_id
    cum = np.cumsum(mk, axis=1)
    ar = np.arange(S)
    last = (img * (ar + 1)).max(axis=1) - 1
    prompt_pages = cum[np.arange(B), np.maximum(last, 0)] * (last >= 0)
    marker_mode = prompt_pages > 0
    run = np.cumsum(img, axis=1) - 1
    ipage = np.where(marker_mode[:, None], cum - 1, run // per_page)
    ipage = np.where(img, ipage, -1)
    raw = cum - 1
    resp = raw - np.where(marker_mode, prompt_pages, 0)[:, None]
    in_prefill = ar[None, :] <= last[:, None]
    q = np.where(in_prefill, raw, resp)
    if not page_scope_prefill:
        q = np.where(in_prefill, -1, q)
    q = np.where(q < 0, -1, q)
    if img.sum() == 0 or (q >= 0).sum() == 0:
        return None, None, None
    return img, ipage.astype(np.int64), q.astype(np.int64)


def page_rope_pos(source_ids, image_token_id: int, page_token_id: int, key_length: int):
    """``_build_page_rope_pos`` + the running counts of ``_page_rope_offsets``
    (HF/_sparse_base_impl.py:2511-2570, no span ablation): (tok_pos, page_pos,
    pf_cnt) or None where the reference bails to the 1D RoPE."""
    ids = np.asarray(source_ids, np.int64)[:, :key_length]
    if ids.shape[1] < key_length:
        ids = np.pad(ids, ((0, 0), (0, key_length - ids.shape[1])), constant_values=-1)
    B, S = ids.shape
    ar = np.arange(S)
    img = ids == image_token_id
    mk = ids == page_token_id
    if not img.any() or not mk.any():
        return None
    cum = np.cumsum(mk, axis=1)
    last = (img * (ar + 1)).max(axis=1) - 1
    n_pages = cum[np.arange(B), np.maximum(last, 0)] * (last >= 0)
    if not (n_pages > 0).all():
        return None
    in_prefill = ar[None, :] <= last[:, None]
    page = np.maximum(np.where(in_prefill, cum, cum - n_pages[:, None]), 0)
    n_pg = int(page.max()) + 1
    onehot = np.eye(n_pg, dtype=np.int64)[page]                   # [B, S, n_pg]
    run = np.cumsum(onehot, axis=1)
    tok = np.take_along_axis(run, page[:, :, None], axis=2)[:, :, 0] - 1
    pf_cnt = (onehot * in_prefill[:, :, None]).sum(axis=1)
    return tok.astype(np.int64), page.astype(np.int64), pf_cnt.astype(np.int64)
