"""Torch-facing page-isolation and Page2D RoPE operators (device tensors only).

Thin launchers over the C ABI (``srswa_page_*`` / ``srswa_page2d_*``): they
check shapes on the host, pass pointers and strides, and enqueue on torch's
current stream.  Index tensors may be int32 or int64 (the kernels read either);
nothing here runs on the CPU.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import UnsupportedShape


def _cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("srswa page ops take device (cuda/hip) tensors; there is no CPU path")


def _ix(t: torch.Tensor):
    """(1-D/2-D index tensor with unit inner stride, int64 flag)."""
    if t.dtype not in (torch.int32, torch.int64):
        t = t.to(torch.int64)
    if t.dim() > 0 and t.stride(-1) != 1:
        t = t.contiguous()
    return t, int(t.dtype == torch.int64)


def _vec(t: torch.Tensor):
    t, f = _ix(t)
    return (t if t.is_contiguous() else t.contiguous()), f


def _state(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.int32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int32 state tensor (it is updated in place)")
    return t


def _run(fn: str, args, *extra, device) -> None:
    _lib.check(getattr(_lib.lib(), fn)(ctypes.byref(args), *extra, _lib.stream_ptr(device)), fn)


# ---------------------------------------------------------------------------
# one-token decode: page state, candidate mask, local union
# ---------------------------------------------------------------------------
def page_decode_meta(input_ids, block_table, seq_lens, slot_mapping, coord_row, *, s_page, s_mark, s_run, s_pp,
                     c_mark, c_pp, c_cnt, image_token_id, page_token_id, per_page, block_size,
                     n_slots=None, out_q_page=None, out_tok=None, out_page=None):
    """Page state + Page2D coordinates of one decode token per request.

    Updates the per-slot state (``s_*``, [n_slots] int32) and the per-row
    coordinate state (``c_mark`` / ``c_pp`` [rows], ``c_cnt`` [rows,
    max_pages] int32) in place; returns (q_page int32 [R], tok int64 [R],
    page int64 [R]) -- views of the ``out_*`` buffers when given."""
    _cuda(input_ids, block_table, seq_lens, slot_mapping, coord_row, s_page, c_cnt)
    R = int(seq_lens.shape[0])
    dev = seq_lens.device
    ids, ids64 = _vec(input_ids[:R])
    bt, bt64 = _ix(block_table)
    sl, sl64 = _vec(seq_lens)
    sm, sm64 = _vec(slot_mapping[:R])
    row = coord_row.to(torch.int64).contiguous()
    for t, n in ((s_page, "s_page"), (s_mark, "s_mark"), (s_run, "s_run"), (s_pp, "s_pp"), (c_mark, "c_mark"),
                 (c_pp, "c_pp")):
        _state(t, n)
    if c_cnt.dtype != torch.int32 or c_cnt.dim() != 2 or c_cnt.stride(1) != 1:
        raise ValueError("c_cnt must be an int32 [rows, max_pages] tensor with unit inner stride")

    def _slot(buf, dtype):
        if buf is None or buf.shape[0] < R:
            return torch.empty(R, dtype=dtype, device=dev)
        return buf[:R]

    q_page, tok, page = _slot(out_q_page, torch.int32), _slot(out_tok, torch.int64), _slot(out_page, torch.int64)
    a = _lib.PageMetaArgs(
        input_ids=ids.data_ptr(), ids_i64=ids64, block_table=bt.data_ptr(), bt_i64=bt64, bt_sr=bt.stride(0),
        seq_lens=sl.data_ptr(), seq_i64=sl64, slot_mapping=sm.data_ptr(), slot_i64=sm64, coord_row=row.data_ptr(),
        s_page=s_page.data_ptr(), s_mark=s_mark.data_ptr(), s_run=s_run.data_ptr(), s_pp=s_pp.data_ptr(),
        c_mark=c_mark.data_ptr(), c_pp=c_pp.data_ptr(), c_cnt=c_cnt.data_ptr(), cnt_sr=c_cnt.stride(0),
        q_page=q_page.data_ptr(), tok=tok.data_ptr(), page=page.data_ptr(),
        image_token_id=int(image_token_id), page_token_id=int(page_token_id or 0),
        R=R, bt_w=int(bt.shape[1]), n_slots=min(int(n_slots or s_page.numel()), s_page.numel()),
        n_rows=min(c_mark.numel(), c_pp.numel(), int(c_cnt.shape[0])), max_pages=int(c_cnt.shape[1]),
        block_size=int(block_size), per_page=max(1, int(per_page)), has_marker=int(page_token_id is not None))
    _run("srswa_page_decode_meta", a, device=dev)
    return q_page, tok, page


def page_decode_allow(block_table, s_page, q_page, seq_lens, *, max_block, num_blocks, block_size, out=None):
    """Page-isolation candidate mask [R, max_block] int8 of the decode rows
    (1 = candidate); a view of ``out`` when given."""
    _cuda(block_table, s_page, q_page, seq_lens, out)
    R = int(q_page.shape[0])
    max_block = int(max_block)
    bt, bt64 = _ix(block_table)
    sl, sl64 = _vec(seq_lens)
    qp = q_page if (q_page.dtype == torch.int32 and q_page.is_contiguous()) else q_page.to(torch.int32).contiguous()
    sp = _state(s_page, "s_page")
    if out is None or out.shape[0] < R or out.shape[1] < max_block:
        out = torch.zeros(R, max_block, dtype=torch.int8, device=q_page.device)
    view = out[:R, :max_block]
    if view.dtype != torch.int8 or view.stride(1) != 1:
        raise ValueError("out must be an int8 [R, >= max_block] tensor with unit inner stride")
    a = _lib.PageAllowArgs(block_table=bt.data_ptr(), bt_i64=bt64, bt_sr=bt.stride(0), s_page=sp.data_ptr(),
                           n_slots=sp.numel(), q_page=qp.data_ptr(), seq_lens=sl.data_ptr(), seq_i64=sl64,
                           out=view.data_ptr(), out_sr=view.stride(0), R=R, bt_w=int(bt.shape[1]),
                           max_block=max_block, num_blocks=int(num_blocks), block_size=int(block_size))
    need = ctypes.c_size_t()
    _lib.check(_lib.lib().srswa_page_decode_allow_workspace(ctypes.byref(a), ctypes.byref(need)),
               "srswa_page_decode_allow_workspace")
    scr = _lib.scratch(q_page.device, need.value)
    _run("srswa_page_decode_allow", a, _lib.ptr(scr), need.value, device=q_page.device)
    return view


def page_local_union(allow, seq_lens, out, *, max_block, block_size, local_blocks):
    """Union of the local window into ``allow``, written as int8 into ``out``
    (first ``max_block`` columns); returns ``out[:R, :max_block]``."""
    _cuda(allow, seq_lens, out)
    R = int(seq_lens.shape[0])
    sl, sl64 = _vec(seq_lens)
    if allow.stride(-1) != 1 or out.stride(-1) != 1 or out.dtype != torch.int8:
        raise ValueError("allow / out must be 2-D with unit inner stride; out int8")
    al = allow if allow.dtype == torch.int8 else allow.to(torch.int8)
    a = _lib.LocalUnionArgs(allow=al.data_ptr(), a_sr=al.stride(0), out=out.data_ptr(), o_sr=out.stride(0),
                            seq_lens=sl.data_ptr(), seq_i64=sl64, R=R, a_w=int(al.shape[1]),
                            o_w=int(out.shape[1]), max_block=int(max_block), block_size=int(block_size),
                            local_blocks=int(local_blocks))
    _run("srswa_page_local_union", a, device=out.device)
    return out[:R, :int(max_block)]


# ---------------------------------------------------------------------------
# Page2D RoPE
# ---------------------------------------------------------------------------
def page2d_cos_sin(tok, page, inv_tok, inv_page, *, dim, page_mod=0, dtype=torch.float32, out_cos=None,
                   out_sin=None):
    """cos / sin [T, dim] of the (tok, page) coordinates in ``dtype`` (fp32
    angles and functions); written into ``out_cos`` / ``out_sin`` when given."""
    _cuda(tok, page, out_cos, out_sin)
    T = int(tok.shape[0])
    tk, tk64 = _vec(tok)
    pg, pg64 = _vec(page)
    it = inv_tok.to(device=tok.device, dtype=torch.float32).contiguous()
    ip = inv_page.to(device=tok.device, dtype=torch.float32).contiguous()
    cos = out_cos[:T] if out_cos is not None else torch.empty(T, dim, dtype=dtype, device=tok.device)
    sin = out_sin[:T] if out_sin is not None else torch.empty(T, dim, dtype=dtype, device=tok.device)
    if (cos.dtype != sin.dtype or cos.stride(-1) != 1 or sin.stride(-1) != 1 or cos.shape[-1] < dim
            or sin.shape[-1] < dim or cos.shape[0] < T or sin.shape[0] < T):
        raise ValueError("cos / sin buffers must hold [T, dim], share a dtype and have unit inner stride")
    if it.numel() + ip.numel() != dim // 2 or it.numel() == 0:
        raise ValueError("inv_tok and inv_page must hold dim / 2 frequencies together")
    a = _lib.CosSinArgs(tok=tk.data_ptr(), tok_i64=tk64, page=pg.data_ptr(), page_i64=pg64, inv_tok=it.data_ptr(),
                        inv_page=ip.data_ptr() if ip.numel() else None, cos=cos.data_ptr(), c_st=cos.stride(0),
                        sin=sin.data_ptr(), s_st=sin.stride(0), page_mod=int(page_mod or 0), T=T, dim=int(dim),
                        n_tok=int(it.numel()), out_dtype=_lib.dtype_code(cos.dtype))
    _run("srswa_page2d_cos_sin", a, device=tok.device)
    return cos, sin


def _bshd(t: torch.Tensor, layout: str):
    """(B, S, H, hd) sizes and (b, s, h) strides of a [T, H*hd] ('flat', head
    dim given separately) or [B, H, S, hd] ('bhsd') tensor."""
    if layout == "bhsd":
        B, H, S, _ = t.shape
        return (B, S, H), (t.stride(0), t.stride(2), t.stride(1))
    raise AssertionError(layout)


def _rope(x, y, cos, sin, head_dim, layout):
    _cuda(x, y, cos, sin)
    dt = x.dtype
    if any(t is not None and t.dtype != dt for t in (y, cos, sin)):
        raise UnsupportedShape("page2d rope: x, y, cos and sin must share one dtype")
    code = _lib.dtype_code(dt)
    hd = int(head_dim)
    if layout == "flat":
        T = x.shape[0]
        if x.dim() != 2 or x.shape[1] % hd or x.stride(1) != 1:
            raise UnsupportedShape("page2d rope: x must be [T, H * head_dim] with unit inner stride")
        B, S = 1, T
        HX = x.shape[1] // hd
        xs = (0, x.stride(0), hd)
        ox = torch.empty_like(x, memory_format=torch.contiguous_format)
        oxs = (0, ox.stride(0), hd)
        if cos.shape != (T, hd) or sin.shape != (T, hd) or cos.stride(1) != 1 or sin.stride(1) != 1:
            raise UnsupportedShape("page2d rope: cos / sin must be [T, head_dim]")
        cs, ss = (0, cos.stride(0)), (0, sin.stride(0))
        if y is not None:
            if y.dim() != 2 or y.shape[0] != T or y.shape[1] % hd or y.stride(1) != 1:
                raise UnsupportedShape("page2d rope: y must be [T, H * head_dim] with unit inner stride")
            HY = y.shape[1] // hd
            ys = (0, y.stride(0), hd)
            oy = torch.empty_like(y, memory_format=torch.contiguous_format)
            oys = (0, oy.stride(0), hd)
    else:
        if x.dim() != 4 or x.shape[-1] != hd or x.stride(-1) != 1:
            raise UnsupportedShape("page2d rope: q must be [B, H, S, head_dim] with unit inner stride")
        (B, S, HX), xs = _bshd(x, layout)
        ox = torch.empty_like(x)
        _, oxs = _bshd(ox, layout)
        ce = cos.expand(B, S, hd)
        se = sin.expand(B, S, hd)
        if ce.stride(-1) != 1 or se.stride(-1) != 1:
            raise UnsupportedShape("page2d rope: cos / sin need a unit inner stride")
        cs, ss = (ce.stride(0), ce.stride(1)), (se.stride(0), se.stride(1))
        if y is not None:
            if y.dim() != 4 or y.shape[0] != B or y.shape[2] != S or y.shape[-1] != hd or y.stride(-1) != 1:
                raise UnsupportedShape("page2d rope: k must be [B, H, S, head_dim] like q")
            (_, _, HY), ys = _bshd(y, layout)
            oy = torch.empty_like(y)
            _, oys = _bshd(oy, layout)
    if y is None:
        HY, ys, oy, oys = 0, (0, 0, 0), None, (0, 0, 0)
    a = _lib.RopeArgs(x=x.data_ptr(), x_sb=xs[0], x_ss=xs[1], x_sh=xs[2],
                      ox=ox.data_ptr(), ox_sb=oxs[0], ox_ss=oxs[1], ox_sh=oxs[2],
                      y=_lib.ptr(y), y_sb=ys[0], y_ss=ys[1], y_sh=ys[2],
                      oy=_lib.ptr(oy), oy_sb=oys[0], oy_ss=oys[1], oy_sh=oys[2],
                      cos=cos.data_ptr(), c_sb=cs[0], c_ss=cs[1], sin=sin.data_ptr(), s_sb=ss[0], s_ss=ss[1],
                      B=B, S=S, HX=HX, HY=HY, head_dim=hd, dtype=code)
    _run("srswa_page2d_rope", a, device=x.device)
    return ox, oy


def page2d_rope(x, cos, sin, head_dim, y=None):
    """x [T, H*hd] (and y [T, H'*hd]) rotated with per-token cos / sin [T, hd]:
    x * cos + rotate_half(x) * sin, each product and the sum rounded to the
    dtype.  Returns ox (or (ox, oy))."""
    ox, oy = _rope(x, y, cos, sin, head_dim, "flat")
    return ox if y is None else (ox, oy)


def rope_bhsd(q, k, cos, sin):
    """The same rotation for the HF layout: q [B, Hq, S, hd], k [B, Hk, S, hd]
    (k may be None), cos / sin [B or 1, S, hd].  Returns (q_embed, k_embed)."""
    return _rope(q, k, cos, sin, q.shape[-1], "bhsd")


# ---------------------------------------------------------------------------
# page-aware candidate masks of query rows (HF prefill / training chunks)
# ---------------------------------------------------------------------------
def page_block_bounds(ids, *, nblk, block_size, out=None):
    """Per-block (min, max) page id of ids [B, L] (-1 = none): int32 [B, nblk, 2]."""
    _cuda(ids, out)
    B, L = ids.shape
    idt, i64 = _ix(ids)
    if out is None:
        out = torch.empty(B, int(nblk), 2, dtype=torch.int32, device=ids.device)
    a = _lib.BlockBoundsArgs(ids=idt.data_ptr(), ids_i64=i64, id_sb=idt.stride(0), bounds=out.data_ptr(),
                             bd_sb=out.stride(0), B=B, L=L, nblk=int(nblk), block_size=int(block_size))
    _run("srswa_page_block_bounds", a, device=ids.device)
    return out


def page_candidate_mask(bounds, ids, qpage, pos=None, *, nblk, block_size, range_test=False, out=None):
    """bool [B, nq, nblk]: block k is a candidate of query row (b, i) when it
    holds a token of the query's page (qpage[b, clamp(pos[b, i])]) -- or, with
    ``range_test``, when that page lies in the block's [lo, hi] bounds; blocks
    past the bounds' width never match; rows with no match (or no page) are
    open to every block.  ``ids`` may be None with ``range_test``."""
    _cuda(bounds, ids, qpage, pos, out)
    B = bounds.shape[0]
    if ids is None:
        if not range_test:
            raise ValueError("the token-level test needs the ids")
        idt, i64, L = None, 0, 0
    else:
        idt, i64 = _ix(ids)
        L = idt.shape[1]
    qp, q64 = _ix(qpage)
    if pos is not None:
        ps, p64 = _ix(pos)
        nq = ps.shape[1]
    else:
        ps, p64, nq = None, 0, qp.shape[1]
    if out is None:
        out = torch.empty(B, nq, int(nblk), dtype=torch.bool, device=bounds.device)
    if out.stride(-1) != 1:
        raise ValueError("out needs a unit inner stride")
    if bounds.dtype != torch.int32 or bounds.stride(-1) != 1 or bounds.stride(-2) != 2:
        raise ValueError("bounds must be int32 [B, nblk, 2] as page_block_bounds returns")
    nbd = min(int(bounds.shape[1]), int(nblk))
    a = _lib.CandidateArgs(bounds=bounds.data_ptr(), bd_sb=bounds.stride(0), ids=_lib.ptr(idt), ids_i64=i64,
                           id_sb=0 if idt is None else idt.stride(0), qpage=qp.data_ptr(), qp_i64=q64,
                           qp_sb=qp.stride(0), pos=_lib.ptr(ps), pos_i64=p64,
                           pos_sb=0 if ps is None else ps.stride(0), out=out.data_ptr(), o_sb=out.stride(0),
                           o_sq=out.stride(1), B=B, nq=nq, qlen=int(qp.shape[1]), L=L, nblk=int(nblk), nbd=nbd,
                           block_size=int(block_size), range_test=int(bool(range_test)))
    _run("srswa_page_candidate_mask", a, device=bounds.device)
    return out


# ---------------------------------------------------------------------------
# multi-token steps: serving page state / coordinates, HF prompt-wide ids
# ---------------------------------------------------------------------------
def _i64vec(t: torch.Tensor) -> torch.Tensor:
    t = t.to(torch.int64)
    return t if t.is_contiguous() else t.contiguous()


def page_step(input_ids, q_start, start_pos, block_table, slot_mapping, *, s_page, s_mark, s_run, s_pp,
              image_token_id, page_token_id, per_page, block_size, num_decode_tokens=0, gen_start=None,
              n_slots=None, out_q_page=None):
    """Multi-token page-state step (``srswa_page_step``): q_page int32 [T]
    for the T tokens of ``input_ids`` laid out by ``q_start`` [R + 1] /
    ``start_pos`` [R]; the per-slot state ``s_*`` is updated in place."""
    _cuda(input_ids, q_start, start_pos, block_table, slot_mapping, s_page, gen_start)
    T = int(input_ids.shape[0])
    R = int(start_pos.shape[0])
    dev = input_ids.device
    ids, ids64 = _vec(input_ids)
    qs, sp = _i64vec(q_start), _i64vec(start_pos)
    gs = None if gen_start is None else _i64vec(gen_start)
    bt, bt64 = _ix(block_table)
    sm, sm64 = _vec(slot_mapping[:T])
    for t, n in ((s_page, "s_page"), (s_mark, "s_mark"), (s_run, "s_run"), (s_pp, "s_pp")):
        _state(t, n)
    q_page = out_q_page[:T] if out_q_page is not None and out_q_page.shape[0] >= T else \
        torch.empty(T, dtype=torch.int32, device=dev)
    a = _lib.PageStepArgs(
        input_ids=ids.data_ptr(), ids_i64=ids64, q_start=qs.data_ptr(), start_pos=sp.data_ptr(),
        gen_start=_lib.ptr(gs), block_table=bt.data_ptr(), bt_i64=bt64, bt_sr=bt.stride(0),
        slot_mapping=sm.data_ptr(), slot_i64=sm64, s_page=s_page.data_ptr(), s_mark=s_mark.data_ptr(),
        s_run=s_run.data_ptr(), s_pp=s_pp.data_ptr(), q_page=q_page.data_ptr(),
        image_token_id=int(image_token_id), page_token_id=int(page_token_id or 0),
        num_decode_tokens=int(num_decode_tokens), R=R, T=T, bt_w=int(bt.shape[1]),
        n_slots=min(int(n_slots or s_page.numel()), s_page.numel()), block_size=int(block_size),
        per_page=max(1, int(per_page)), has_marker=int(page_token_id is not None))
    _run("srswa_page_step", a, device=dev)
    return q_page


def coord_step(input_ids, q_start, start_pos, rows, *, st_marker, st_pp, cnt, image_token_id, page_token_id,
               num_decode_tokens=0, gen_start=None, with_carry=False):
    """The scans, ranks and carry of a Page2D coordinate step
    (``srswa_coord_step``) for state rows ``rows`` [R]: (tok int64 [T],
    page int64 [T]) and, with ``with_carry``, marker / pp int32 [T]; the row
    state is updated in place."""
    _cuda(input_ids, q_start, start_pos, rows, st_marker, cnt, gen_start)
    T = int(input_ids.shape[0])
    R = int(start_pos.shape[0])
    dev = input_ids.device
    ids, ids64 = _vec(input_ids)
    qs, sp, rw = _i64vec(q_start), _i64vec(start_pos), _i64vec(rows)
    gs = None if gen_start is None else _i64vec(gen_start)
    _state(st_marker, "st_marker")
    _state(st_pp, "st_pp")
    if cnt.dtype != torch.int32 or cnt.dim() != 2 or cnt.stride(1) != 1:
        raise ValueError("cnt must be an int32 [rows, pages] tensor with unit inner stride")
    tok = torch.empty(T, dtype=torch.int64, device=dev)
    page = torch.empty(T, dtype=torch.int64, device=dev)
    mk = torch.empty(T, dtype=torch.int32, device=dev) if with_carry else None
    pp = torch.empty(T, dtype=torch.int32, device=dev) if with_carry else None
    a = _lib.CoordStepArgs(
        input_ids=ids.data_ptr(), ids_i64=ids64, q_start=qs.data_ptr(), start_pos=sp.data_ptr(),
        gen_start=_lib.ptr(gs), row=rw.data_ptr(), st_marker=st_marker.data_ptr(), st_pp=st_pp.data_ptr(),
        cnt=cnt.data_ptr(), cnt_sr=cnt.stride(0), tok=tok.data_ptr(), page=page.data_ptr(),
        marker_out=_lib.ptr(mk), pp_out=_lib.ptr(pp), image_token_id=int(image_token_id),
        page_token_id=int(page_token_id or 0), num_decode_tokens=int(num_decode_tokens), R=R, T=T,
        n_rows=min(st_marker.numel(), st_pp.numel(), int(cnt.shape[0])), pages=int(cnt.shape[1]),
        has_marker=int(page_token_id is not None))
    _run("srswa_coord_step", a, device=dev)
    return (tok, page, mk, pp) if with_carry else (tok, page)


def _ids2d(ids, key_length, device):
    t = ids.to(device)
    if t.dtype not in (torch.int32, torch.int64):
        t = t.to(torch.int64)
    if t.stride(-1) != 1:
        t = t.contiguous()
    return t, int(t.dtype == torch.int64), min(int(t.shape[-1]), int(key_length))


def page_aware_ids(source_ids, *, image_token_id, page_token_id, key_length, per_page, page_scope_prefill=True,
                   device=None):
    """Prompt-wide page ids (``srswa_page_ids``): (image_token_mask bool,
    image_token_page_ids int64, query_token_page_ids int64) [B, key_length]
    and the per-row counts [B, 2] int32 (query tokens with a page, image tokens)."""
    dev = device or source_ids.device
    ids, ids64, n_ids = _ids2d(source_ids, key_length, dev)
    _cuda(ids)
    B, L = int(ids.shape[0]), int(key_length)
    img = torch.empty(B, L, dtype=torch.bool, device=dev)
    ipage = torch.empty(B, L, dtype=torch.int64, device=dev)
    qpage = torch.empty(B, L, dtype=torch.int64, device=dev)
    counts = torch.empty(B, 2, dtype=torch.int32, device=dev)
    a = _lib.PageIdsArgs(ids=ids.data_ptr(), ids_i64=ids64, id_sb=ids.stride(0), img_mask=img.data_ptr(),
                         img_page=ipage.data_ptr(), q_page=qpage.data_ptr(), o_sb=L, row_counts=counts.data_ptr(),
                         image_token_id=int(image_token_id), page_token_id=int(page_token_id), B=B, L=L,
                         n_ids=n_ids, per_page=max(1, int(per_page)), page_scope_prefill=int(bool(page_scope_prefill)))
    _run("srswa_page_ids", a, device=dev)
    return img, ipage, qpage, counts


def page_rope_pos(source_ids, *, image_token_id, page_token_id, key_length, device=None):
    """Prompt-wide Page2D positions: pass 1 (``srswa_page_rope_pos``) gives
    page / in_prefill [B, L] and the per-row info [B, 4] (n_pages, max page,
    any image, any marker); the caller reads it back (the reference's own
    data-dependent checks) and, unless it bails, calls ``page_rope_tok``."""
    dev = device or source_ids.device
    ids, ids64, n_ids = _ids2d(source_ids, key_length, dev)
    _cuda(ids)
    B, L = int(ids.shape[0]), int(key_length)
    page = torch.empty(B, L, dtype=torch.int32, device=dev)
    pre = torch.empty(B, L, dtype=torch.uint8, device=dev)
    info = torch.empty(B, 4, dtype=torch.int32, device=dev)
    a = _lib.PagePosArgs(ids=ids.data_ptr(), ids_i64=ids64, id_sb=ids.stride(0), page=page.data_ptr(),
                         prefill=pre.data_ptr(), o_sb=L, row_info=info.data_ptr(),
                         image_token_id=int(image_token_id), page_token_id=int(page_token_id), B=B, L=L,
                         n_ids=n_ids, n_pg=0)
    _run("srswa_page_rope_pos", a, device=dev)
    return page, pre, info


def page_rope_tok(page, prefill, n_pg):
    """Pass 2: (tok int64 [B, L] running count inside each page bucket,
    pf_cnt int64 [B, n_pg] prefill tokens per page)."""
    _cuda(page, prefill)
    B, L = int(page.shape[0]), int(page.shape[1])
    dev = page.device
    tok = torch.empty(B, L, dtype=torch.int64, device=dev)
    pf = torch.empty(B, int(n_pg), dtype=torch.int32, device=dev)
    a = _lib.PagePosArgs(page=page.data_ptr(), prefill=prefill.data_ptr(), o_sb=L, tok=tok.data_ptr(),
                         pf_cnt=pf.data_ptr(), pf_sb=int(n_pg), B=B, L=L, n_pg=int(n_pg))
    _run("srswa_page_rope_tok", a, device=dev)
    return tok, pf.to(torch.int64)
