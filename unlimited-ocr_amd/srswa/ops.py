"""Torch-facing SR-SWA operators (device tensors in, device tensors out).

Each function validates shapes on the host, builds the C-ABI argument struct
from tensor pointers/strides (no ``.contiguous()`` copies of q/k/v), and
launches on torch's current stream.  Unsupported shapes raise
``UnsupportedShape``; nothing here runs on the CPU.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import UnsupportedShape


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("srswa ops take device (cuda/hip) tensors; there is no CPU path")


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 else t.to(torch.int32)


class _Launch:
    """A prepared launch: the C-ABI struct, the tensors it points into (kept
    alive), the scratch buffer and the entry point.  ``__call__``
    enqueues the kernel on the stream captured at preparation time without
    rebuilding anything (a few microseconds of host time)."""

    def __init__(self, fn, args, keep, extra, stream, what):
        self.fn, self.args, self.keep, self.extra = fn, args, keep, extra
        self.stream, self.what = stream, what
        self._ref = ctypes.byref(args)
        self._extra = tuple(_lib.ptr(x) if isinstance(x, torch.Tensor) else x for x in extra)

    def __call__(self):
        _lib.check(self.fn(self._ref, *self._extra, self.stream), self.what)


def prepare_gather_decode(q, k_cache, v_cache, block_indices, q_pos, *, block_size, local_window,
                          scale, bias=None, valid=None, kv_len=None, out=None, out_dtype=None,
                          return_lse=False):
    """Validate, allocate outputs and build the launch of ``gather_decode``.

    Returns (launch, out, lse); ``launch()`` runs the kernel (again) into
    ``out``/``lse``.  Shapes as in ``gather_decode``."""
    _require_cuda(q, k_cache, v_cache, block_indices, q_pos, bias, valid, kv_len, out)
    squeeze = q.dim() == 3
    if squeeze:
        q = q.unsqueeze(1)
        block_indices = block_indices.unsqueeze(2)
        if bias is not None:
            bias = bias.unsqueeze(2)
        if valid is not None:
            valid = valid.unsqueeze(2)
        if q_pos.dim() == 1:
            q_pos = q_pos.unsqueeze(1)
    B, Lq, HQ, D = q.shape
    Bk, L, HKV, Dk = k_cache.shape
    if Bk != B or Dk != D or tuple(v_cache.shape) != tuple(k_cache.shape):
        raise ValueError(f"cache shape {tuple(k_cache.shape)} / {tuple(v_cache.shape)} vs q {tuple(q.shape)}")
    HI, S = block_indices.shape[1], block_indices.shape[-1]
    if tuple(block_indices.shape) != (B, HI, Lq, S):
        raise ValueError(f"block_indices shape {tuple(block_indices.shape)} != {(B, HI, Lq, S)}")
    if q.dtype != k_cache.dtype or q.dtype != v_cache.dtype:
        raise ValueError("q, k_cache, v_cache must share a dtype")
    for t in (q, k_cache, v_cache):
        if t.stride(-1) != 1:
            raise UnsupportedShape("head dim must be contiguous")
    idx = _i32(block_indices).contiguous()
    if bias is not None:
        bias = bias.to(torch.float32).expand(idx.shape).contiguous()
    if valid is not None:
        valid = valid.to(torch.bool).expand(idx.shape).contiguous().view(torch.uint8)
    pos = _i32(q_pos).contiguous()
    if tuple(pos.shape) != (B, Lq):
        raise ValueError(f"q_pos shape {tuple(pos.shape)} != {(B, Lq)}")
    kvl = None if kv_len is None else _i32(kv_len).contiguous()
    odt = out_dtype or q.dtype
    if out is None:
        out = torch.empty(B, Lq, HQ, D, dtype=odt, device=q.device)
    elif squeeze:
        out = out.unsqueeze(1)
    lse = torch.empty(B, Lq, HQ, dtype=torch.float32, device=q.device) if return_lse else None

    a = _lib.DecodeArgs()
    a.q = q.data_ptr(); a.q_sb, a.q_sq, a.q_sh = q.stride(0), q.stride(1), q.stride(2)
    a.k = k_cache.data_ptr(); a.k_sb, a.k_st, a.k_sh = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.v = v_cache.data_ptr(); a.v_sb, a.v_st, a.v_sh = v_cache.stride(0), v_cache.stride(1), v_cache.stride(2)
    a.idx = idx.data_ptr()
    a.idx_sb, a.idx_sh, a.idx_sq, a.idx_ss = idx.stride(0), idx.stride(1), idx.stride(2), idx.stride(3)
    a.bias = _lib.ptr(bias)
    a.valid = _lib.ptr(valid)
    a.q_pos = pos.data_ptr(); a.pos_sb, a.pos_sq = pos.stride(0), pos.stride(1)
    a.kv_len = _lib.ptr(kvl)
    a.out = out.data_ptr(); a.o_sb, a.o_sq, a.o_sh = out.stride(0), out.stride(1), out.stride(2)
    if lse is not None:
        a.lse = lse.data_ptr(); a.lse_sb, a.lse_sq, a.lse_sh = lse.stride(0), lse.stride(1), lse.stride(2)
    a.B, a.Lq, a.HQ, a.HKV, a.HI, a.D, a.S, a.L = B, Lq, HQ, HKV, HI, D, S, L
    a.block_size, a.local_window = int(block_size), max(1, int(local_window))
    a.scale = float(scale)
    a.in_dtype = _lib.dtype_code(q.dtype)
    a.out_dtype = _lib.dtype_code(odt)
    L_ = _lib.lib()
    nscr = L_.srswa_gather_decode_workspace(ctypes.byref(a))
    scr = _lib.scratch(q.device, nscr)
    launch = _Launch(L_.srswa_gather_decode, a,
                     (q, k_cache, v_cache, idx, bias, valid, pos, kvl, out, lse),
                     (scr, nscr), _lib.stream_ptr(q.device), "srswa_gather_decode")
    if squeeze:
        out = out.squeeze(1)
        if lse is not None:
            lse = lse.squeeze(1)
    return launch, out, lse


def gather_decode(q, k_cache, v_cache, block_indices, q_pos, *, block_size, local_window,
                  scale, bias=None, valid=None, kv_len=None, out=None, out_dtype=None,
                  return_lse=False):
    """Block-sparse decode attention over a KV cache.

    q            [B, Lq, HQ, D] (or [B, HQ, D] for one row per sequence)
    k_cache      [B, L, HKV, D] any strides with unit head-dim stride
    v_cache      [B, L, HKV, D]
    block_indices[B, HI, Lq, S] (or [B, HI, S]) block ids, -1 = empty slot
    q_pos        [B, Lq] (or [B]) absolute query positions
    bias, valid  like block_indices (fp32 / bool), optional
    kv_len       [B] cache fill (keys >= kv_len are never read), optional
    Returns o [B, Lq, HQ, D] (or [B, HQ, D]) in ``out_dtype`` (default q.dtype)
    and, if asked, lse [B, Lq, HQ] (natural log).
    """
    launch, out, lse = prepare_gather_decode(
        q, k_cache, v_cache, block_indices, q_pos, block_size=block_size,
        local_window=local_window, scale=scale, bias=bias, valid=valid, kv_len=kv_len,
        out=out, out_dtype=out_dtype, return_lse=return_lse)
    launch()
    return (out, lse) if return_lse else out


def decode_attend(q, k_all, v_all, topi, bias, valid, q_pos, block_size, local_window, scale):
    """Drop-in for ``_decode_attend`` (HF/modeling_deepseekv2.py:454-481).

    q [B,H,Lq,D]; k_all, v_all [B,Hkv,S,D]; topi/bias/valid [B,Lq,K] (one
    index head for all heads, as the reference) or [B,HI,Lq,K]; q_pos [B,Lq].
    Returns fp32 [B,H,Lq,D] like the reference (which computes in fp32)."""
    if topi.dim() == 3:
        topi, bias, valid = topi[:, None], bias[:, None], valid[:, None]
    qv = q.transpose(1, 2)                   # [B,Lq,H,D] view
    kv = k_all.transpose(1, 2)               # [B,S,Hkv,D] view
    vv = v_all.transpose(1, 2)
    o = gather_decode(qv, kv, vv, topi, q_pos, block_size=block_size,
                      local_window=local_window, scale=scale, bias=bias, valid=valid,
                      out_dtype=torch.float32)
    return o.transpose(1, 2)


# ---------------------------------------------------------------------------
# indexer
# ---------------------------------------------------------------------------
SCORE_NEG = -1.0e9


def prepare_index_meanpool_topk(q, k, q_pos, *, block_size, local_blocks, topk, head_cls=None,
                                kv_len=None, nblk=None, return_scores=False, return_kbar=False,
                                ascending=False):
    """Build the launch of the head_cls / mean-pool indexer (see ``index_meanpool_topk``).

    Returns (launch, idx, scores_or_None, kbar_or_None)."""
    _require_cuda(q, k, q_pos, head_cls, kv_len)
    squeeze = q.dim() == 3
    if squeeze:                                   # [B, HI, D] -> one query row
        q = q.unsqueeze(2)
        if q_pos.dim() == 1:
            q_pos = q_pos.unsqueeze(1)
    B, HI, Lq, D = q.shape
    if k.dim() == 3:                              # [B, L, D]: one key head shared by all HI
        k = k.unsqueeze(2)
    Bk, L, HK, Dk = k.shape
    if Bk != B or Dk != D or HK not in (1, HI):
        raise ValueError(f"k shape {tuple(k.shape)} incompatible with q {tuple(q.shape)}")
    if k.stride(-1) != 1:
        raise UnsupportedShape("key head dim must be contiguous")
    nblk = int(nblk) if nblk is not None else -(-L // int(block_size))
    qf = q.to(torch.float32)
    pos = _i32(q_pos).contiguous()
    if tuple(pos.shape) != (B, Lq):
        raise ValueError(f"q_pos shape {tuple(pos.shape)} != {(B, Lq)}")
    kvl = None if kv_len is None else _i32(kv_len).contiguous()
    hc = None if head_cls is None else head_cls.to(torch.float32).contiguous()
    scores = torch.empty(B, HI, Lq, nblk, dtype=torch.float32, device=q.device) if return_scores else None
    kbar = torch.empty(B, HI, nblk, D, dtype=torch.float32, device=q.device) if return_kbar else None
    idx = torch.empty(B, HI, Lq, int(topk), dtype=torch.int32, device=q.device) if topk > 0 else None

    a = _lib.IndexArgs()
    a.q = qf.data_ptr(); a.q_sb, a.q_sh, a.q_sq = qf.stride(0), qf.stride(1), qf.stride(2)
    a.k = k.data_ptr(); a.k_sb, a.k_st = k.stride(0), k.stride(1)
    a.k_sh = 0 if HK == 1 else k.stride(2)
    if kbar is not None:
        a.kbar_out = kbar.data_ptr(); a.kb_sb, a.kb_sh, a.kb_sn = kbar.stride(0), kbar.stride(1), kbar.stride(2)
    a.head_cls = _lib.ptr(hc)
    a.q_pos = pos.data_ptr(); a.pos_sb, a.pos_sq = pos.stride(0), pos.stride(1)
    a.kv_len = _lib.ptr(kvl)
    if scores is not None:
        a.scores = scores.data_ptr(); a.sc_sb, a.sc_sh, a.sc_sq = scores.stride(0), scores.stride(1), scores.stride(2)
    if idx is not None:
        a.topk_idx = idx.data_ptr(); a.ti_sb, a.ti_sh, a.ti_sq = idx.stride(0), idx.stride(1), idx.stride(2)
    a.B, a.HI, a.Lq, a.D, a.L, a.nblk = B, HI, Lq, D, L, nblk
    a.block_size, a.local_blocks, a.K, a.ascending = int(block_size), int(local_blocks), int(topk), int(bool(ascending))
    a.k_dtype = _lib.dtype_code(k.dtype)
    L_ = _lib.lib()
    nscr = L_.srswa_index_workspace(ctypes.byref(a))
    scr = _lib.scratch(q.device, nscr)
    launch = _Launch(L_.srswa_index_meanpool_topk, a, (qf, k, pos, kvl, hc, scores, kbar, idx),
                     (scr, nscr), _lib.stream_ptr(q.device), "srswa_index_meanpool_topk")
    if squeeze:
        idx = None if idx is None else idx.squeeze(2)
        scores = None if scores is None else scores.squeeze(2)
    return launch, idx, scores, kbar


def index_meanpool_topk(q, k, q_pos, *, block_size, local_blocks, topk, head_cls=None,
                        kv_len=None, nblk=None, return_scores=False, return_kbar=False,
                        ascending=False):
    """head_cls / mean-pool block indexer with top-k selection.

    q       [B, HI, Lq, D] (or [B, HI, D]) index queries (any float dtype; scored in fp32)
    k       [B, L, HI, D] or [B, L, D] (one key head shared) index keys, bf16/fp16/fp32
    q_pos   [B, Lq] (or [B]) absolute positions
    head_cls[D] learned summary query (None -> mean pooling, the zero-init value)
    Returns idx [B, HI, Lq, topk] int32 (descending score, ties -> lower id, -1 pad;
    ``ascending=True`` re-packs ascending), plus scores [B, HI, Lq, nblk] and
    k_bar [B, HI, nblk, D] when asked.  Restates ``_block_scores_infer`` head_cls +
    top-k (HF/modeling_deepseekv2.py:380-417, HF/_sparse_base_impl.py:3100-3105).
    """
    launch, idx, scores, kbar = prepare_index_meanpool_topk(
        q, k, q_pos, block_size=block_size, local_blocks=local_blocks, topk=topk,
        head_cls=head_cls, kv_len=kv_len, nblk=nblk, return_scores=return_scores,
        return_kbar=return_kbar, ascending=ascending)
    launch()
    out = [idx]
    if return_scores:
        out.append(scores)
    if return_kbar:
        out.append(kbar)
    return out[0] if len(out) == 1 else tuple(out)


def topk_rows(scores, k, *, invalid_at=SCORE_NEG * 0.5, ascending=False, return_values=False):
    """Top-k along the last dim of an fp32 device tensor: descending, ties ->
    lower index, entries <= invalid_at (and NaN) never selected, missing -1."""
    _require_cuda(scores)
    s = scores.to(torch.float32).contiguous()
    n = s.shape[-1]
    rows = s.numel() // max(n, 1)
    idx = torch.empty(*s.shape[:-1], int(k), dtype=torch.int32, device=s.device)
    val = torch.empty(idx.shape, dtype=torch.float32, device=s.device) if return_values else None
    st = _lib.lib().srswa_topk_rows(s.data_ptr(), rows, n, n, int(k), int(bool(ascending)),
                                    float(invalid_at), idx.data_ptr(), _lib.ptr(val), int(k),
                                    _lib.stream_ptr(s.device))
    _lib.check(st, "srswa_topk_rows")
    return (idx, val) if return_values else idx


def _kv_fp8(q, k_cache, v_cache) -> int:
    """The fp8 format code of the paged caches (0 when they share q's dtype).
    fp8 caches (float8_e4m3fn / e4m3fnuz / e5m2 / e5m2fnuz) are converted
    exactly to q's dtype as the kernels load them, as the reference's
    ``k.to(q.dtype)`` (WHL!layers/attention/unlimited_dash_ops/attend_triton.py:193)."""
    if k_cache.dtype != v_cache.dtype:
        raise ValueError("k_cache and v_cache must share a dtype")
    code = _lib.fp8_code(k_cache.dtype)
    if code:
        if q.dtype not in (torch.bfloat16, torch.float16):
            raise UnsupportedShape("fp8 caches take bf16 / fp16 queries")
        return code
    if q.dtype != k_cache.dtype:
        raise ValueError("q, k_cache, v_cache must share a dtype")
    return 0


def prepare_gather_decode_paged(q, k_cache, v_cache, topk_idx, blk_bias, block_table, seq_lens, *,
                                decode_query_len, local_blocks, scale, out=None):
    """Validate, allocate and build the launch of the paged decode
    (``srswa_gather_decode_paged``).  Returns (launch, out).

    q [total_q, HQ, D] with total_q = R * decode_query_len; k_cache, v_cache
    [num_pages, page_size, HKV, D] (page_size = block size); topk_idx
    [HKV, total_q, K] logical block ids (-1 = empty); blk_bias like topk_idx
    (fp32) or None; block_table [R, max_blocks] page ids; seq_lens [R]."""
    _require_cuda(q, k_cache, v_cache, topk_idx, blk_bias, block_table, seq_lens, out)
    total_q, HQ, D = q.shape
    npages, page, HKV, Dk = k_cache.shape
    dql = int(decode_query_len)
    R = seq_lens.shape[0]
    if total_q != R * dql:
        raise ValueError(f"total_q {total_q} != {R} requests x {dql} queries")
    if Dk != D or tuple(v_cache.shape) != tuple(k_cache.shape):
        raise ValueError(f"cache shape {tuple(k_cache.shape)} / {tuple(v_cache.shape)} vs q {tuple(q.shape)}")
    if topk_idx.dim() != 3 or topk_idx.shape[0] != HKV or topk_idx.shape[1] != total_q:
        raise ValueError(f"topk_idx shape {tuple(topk_idx.shape)} != ({HKV}, {total_q}, K)")
    kv8 = _kv_fp8(q, k_cache, v_cache)
    for t in (q, k_cache, v_cache):
        if t.stride(-1) != 1:
            raise UnsupportedShape("head dim must be contiguous")
    # ids and bias are read through strides (a head-expanded view is taken as
    # is); the kernel addresses both with the ids' strides
    ti = _i32(topk_idx)
    bias = None
    if blk_bias is not None:
        if tuple(blk_bias.shape) != tuple(topk_idx.shape):
            raise ValueError(f"blk_bias shape {tuple(blk_bias.shape)} != topk_idx {tuple(topk_idx.shape)}")
        bias = blk_bias.to(torch.float32)
        if bias.stride() != ti.stride():
            ti, bias = ti.contiguous(), bias.contiguous()
    bt = _i32(block_table)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    sl = _i32(seq_lens).contiguous()
    if out is None:
        out = torch.empty(total_q, HQ, D, dtype=q.dtype, device=q.device)
    a = _lib.PagedDecodeArgs()
    a.q = q.data_ptr(); a.q_sn, a.q_sh = q.stride(0), q.stride(1)
    a.k_cache = k_cache.data_ptr(); a.k_sp, a.k_st, a.k_sh = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.v_cache = v_cache.data_ptr(); a.v_sp, a.v_st, a.v_sh = v_cache.stride(0), v_cache.stride(1), v_cache.stride(2)
    a.topk = ti.data_ptr(); a.t_sh, a.t_sn, a.t_sk = ti.stride(0), ti.stride(1), ti.stride(2)
    a.bias = _lib.ptr(bias)
    a.block_table = bt.data_ptr(); a.bt_sr = bt.stride(0)
    a.seq_lens = sl.data_ptr()
    a.out = out.data_ptr(); a.o_sn, a.o_sh = out.stride(0), out.stride(1)
    a.R, a.dql, a.HQ, a.HKV, a.D, a.topk_n = R, dql, HQ, HKV, D, ti.shape[-1]
    a.max_blocks, a.page_size, a.local_blocks = bt.shape[1], page, int(local_blocks)
    a.scale = float(scale)
    a.in_dtype = _lib.dtype_code(q.dtype)
    a.out_dtype = _lib.dtype_code(out.dtype)
    a.kv_fp8 = kv8
    L_ = _lib.lib()
    nscr = L_.srswa_gather_decode_paged_workspace(ctypes.byref(a))
    scr = _lib.scratch(q.device, nscr)
    launch = _Launch(L_.srswa_gather_decode_paged, a, (q, k_cache, v_cache, ti, bias, bt, sl, out),
                     (scr, nscr), _lib.stream_ptr(q.device), "srswa_gather_decode_paged")
    return launch, out


def gather_decode_paged(q, k_cache, v_cache, topk_idx, blk_bias, block_table, seq_lens, *,
                        decode_query_len, local_blocks, scale, out=None):
    """Block-sparse decode over a paged KV cache (see ``prepare_gather_decode_paged``)."""
    launch, out = prepare_gather_decode_paged(q, k_cache, v_cache, topk_idx, blk_bias, block_table, seq_lens,
                                              decode_query_len=decode_query_len, local_blocks=local_blocks,
                                              scale=scale, out=out)
    launch()
    return out


def gather_fwd_paged(q, k_cache, v_cache, topk_idx, blk_bias, block_table, cu_seqlens_q, seq_lens, prefix_lens,
                     max_query_len, *, local_blocks, scale, out=None):
    """Block-sparse prefill over the paged cache (see ``srswa_gather_fwd_paged``).

    q [total_q, HQ, D]; k_cache, v_cache [num_pages, page_size, HKV, D];
    topk_idx [HKV, total_q, K] block ids (-1 = empty) and blk_bias like it
    (fp32) or None, both read through their strides (slot stride 1);
    block_table [R, max_blocks]; cu_seqlens_q [R + 1]; seq_lens, prefix_lens
    [R]; ``max_query_len`` the longest request (sizes the grid)."""
    _require_cuda(q, k_cache, v_cache, topk_idx, blk_bias, block_table, cu_seqlens_q, seq_lens, prefix_lens, out)
    total_q, HQ, D = q.shape
    npages, page, HKV, Dk = k_cache.shape
    if Dk != D or tuple(v_cache.shape) != tuple(k_cache.shape):
        raise ValueError(f"cache shape {tuple(k_cache.shape)} / {tuple(v_cache.shape)} vs q {tuple(q.shape)}")
    if topk_idx.dim() != 3 or topk_idx.shape[0] != HKV or topk_idx.shape[1] != total_q:
        raise ValueError(f"topk_idx shape {tuple(topk_idx.shape)} != ({HKV}, {total_q}, K)")
    kv8 = _kv_fp8(q, k_cache, v_cache)
    for t in (q, k_cache, v_cache):
        if t.stride(-1) != 1:
            raise UnsupportedShape("head dim must be contiguous")
    ti = _i32(topk_idx)
    if ti.stride(-1) != 1:
        ti = ti.contiguous()
    bias = None
    if blk_bias is not None:
        if tuple(blk_bias.shape) != tuple(topk_idx.shape):
            raise ValueError(f"blk_bias shape {tuple(blk_bias.shape)} != topk_idx {tuple(topk_idx.shape)}")
        bias = blk_bias.to(torch.float32)
        if bias.stride(-1) != 1:
            bias = bias.contiguous()
    bt = _i32(block_table)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    cu = _i32(cu_seqlens_q).contiguous()
    sl = _i32(seq_lens).contiguous()
    pl = _i32(prefix_lens).contiguous()
    R = sl.numel()
    if cu.numel() != R + 1 or pl.numel() != R or bt.shape[0] < R:
        raise ValueError(f"cu_seqlens_q [{cu.numel()}], prefix_lens [{pl.numel()}], block_table rows "
                         f"{bt.shape[0]} for {R} requests")
    if out is None:
        out = torch.empty(total_q, HQ, D, dtype=q.dtype, device=q.device)
    a = _lib.PagedFwdArgs()
    a.q = q.data_ptr(); a.q_sn, a.q_sh = q.stride(0), q.stride(1)
    a.k_cache = k_cache.data_ptr(); a.k_sp, a.k_st, a.k_sh = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.v_cache = v_cache.data_ptr(); a.v_sp, a.v_st, a.v_sh = v_cache.stride(0), v_cache.stride(1), v_cache.stride(2)
    a.topk = ti.data_ptr(); a.t_sh, a.t_sn = ti.stride(0), ti.stride(1)
    if bias is not None:
        a.bias = bias.data_ptr(); a.b_sh, a.b_sn = bias.stride(0), bias.stride(1)
    a.block_table = bt.data_ptr(); a.bt_sr = bt.stride(0)
    a.cu_seqlens_q, a.seq_lens, a.prefix_lens = cu.data_ptr(), sl.data_ptr(), pl.data_ptr()
    a.out = out.data_ptr(); a.o_sn, a.o_sh = out.stride(0), out.stride(1)
    a.R, a.max_query_len, a.HQ, a.HKV, a.D, a.S = R, int(max_query_len), HQ, HKV, D, ti.shape[-1]
    a.max_blocks, a.page_size, a.local_blocks = bt.shape[1], page, int(local_blocks)
    a.scale = float(scale)
    a.dtype = _lib.dtype_code(q.dtype)
    a.kv_fp8 = kv8
    _lib.check(_lib.lib().srswa_gather_fwd_paged(ctypes.byref(a), _lib.stream_ptr(q.device)),
               "srswa_gather_fwd_paged")
    return out


# ---------------------------------------------------------------------------
# head_cls summary cache over a paged index-key cache
# ---------------------------------------------------------------------------
def kbar_pages(keys_cache, head_cls, block_table, seq_lens, kbar, *, tail_blocks=0):
    """Write the summary row of every used page (or each request's last
    ``tail_blocks`` pages) into ``kbar`` [num_pages, D] fp32, in place.
    keys_cache [num_pages, page_size, D] (bf16/fp16/fp32); head_cls [D] or None
    (plain mean); block_table [R, max_blocks]; seq_lens [R]."""
    _require_cuda(keys_cache, head_cls, block_table, seq_lens, kbar)
    npages, page, D = keys_cache.shape
    if keys_cache.stride(-1) != 1 or kbar.stride(-1) != 1 or kbar.dtype != torch.float32:
        raise UnsupportedShape("keys / kbar rows must be contiguous, kbar fp32")
    hc = None if head_cls is None else head_cls.detach().to(torch.float32).contiguous()
    bt = _i32(block_table)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    sl = _i32(seq_lens).contiguous()
    a = _lib.KbarPagesArgs(keys=keys_cache.data_ptr(), k_sp=keys_cache.stride(0), k_st=keys_cache.stride(1),
                           head_cls=_lib.ptr(hc), block_table=bt.data_ptr(), bt_sr=bt.stride(0),
                           seq_lens=sl.data_ptr(), kbar=kbar.data_ptr(), kb_sp=kbar.stride(0),
                           R=bt.shape[0], max_blocks=bt.shape[1], page_size=page, D=D,
                           tail_blocks=int(tail_blocks), k_dtype=_lib.dtype_code(keys_cache.dtype))
    _lib.check(_lib.lib().srswa_kbar_pages(ctypes.byref(a), _lib.stream_ptr(kbar.device)), "srswa_kbar_pages")
    return kbar


def kbar_scores(q, kbar, block_table, seq_lens, *, width, page_size, local_blocks, dql=None, row_req=None,
                row_pos=None, cu_q=None, ctx=None, row_off=0, out=None):
    """Scores [nrows, width] fp32 of index queries q [nrows, D] against the
    cached page summaries (SCORE_NEG off the remote blocks).  Decode rows by
    default (request n // dql at seq_len - dql + n % dql); explicit per-row
    request / position tensors; or prefill rows (``row_req`` the row -> request
    map of every query, ``cu_q`` / ``ctx`` the per-request query offsets and
    cached lengths, ``row_off`` the first query of this chunk)."""
    _require_cuda(q, kbar, block_table, seq_lens, row_req, row_pos, cu_q, ctx, out)
    nrows, D = q.shape
    qf = q.to(torch.float32)
    if qf.stride(-1) != 1:
        qf = qf.contiguous()
    bt = _i32(block_table)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    sl = _i32(seq_lens).contiguous()
    rr = None if row_req is None else _i32(row_req).contiguous()
    rp = None if row_pos is None else _i32(row_pos).contiguous()
    cu = None if cu_q is None else _i32(cu_q).contiguous()
    cx = None if ctx is None else _i32(ctx).contiguous()
    if out is None:
        out = torch.empty(nrows, int(width), dtype=torch.float32, device=q.device)
    if out.stride(-1) != 1:
        raise UnsupportedShape("score rows must be contiguous")
    if out.shape[0] < nrows or out.shape[1] < int(width):
        raise ValueError(f"scores {tuple(out.shape)} smaller than {nrows} x {width}")
    if cu is not None and (rr is None or rr.numel() < int(row_off) + nrows or cu.numel() != sl.numel() + 1
                           or cx.numel() != sl.numel()):
        raise ValueError("prefill rows need row_req covering row_off + nrows rows, cu_q [R + 1], ctx [R]")
    if rp is not None and (rr is None or rr.numel() < nrows or rp.numel() < nrows):
        raise ValueError("explicit rows need row_req and row_pos of nrows entries")
    a = _lib.KbarScoresArgs(q=qf.data_ptr(), q_sn=qf.stride(0), kbar=kbar.data_ptr(), kb_sp=kbar.stride(0),
                            block_table=bt.data_ptr(), bt_sr=bt.stride(0), seq_lens=sl.data_ptr(),
                            row_req=_lib.ptr(rr), row_pos=_lib.ptr(rp), cu_q=_lib.ptr(cu), ctx=_lib.ptr(cx),
                            scores=out.data_ptr(), sc_sn=out.stride(0), nrows=nrows, R=bt.shape[0],
                            dql=int(dql or 0), max_blocks=bt.shape[1], width=int(width), page_size=int(page_size),
                            local_blocks=int(local_blocks), D=D, row_off=int(row_off))
    _lib.check(_lib.lib().srswa_kbar_scores(ctypes.byref(a), _lib.stream_ptr(q.device)), "srswa_kbar_scores")
    return out


def kbar_plan(keys_cache, head_cls, pages, tok, kbar):
    """Summaries of the listed pages (``pages`` int64 [n], ``tok`` their live
    keys, <= 0 skipped) written into ``kbar`` [num_pages, D] fp32 in place."""
    _require_cuda(keys_cache, head_cls, pages, tok, kbar)
    npages, page, D = keys_cache.shape
    if keys_cache.stride(-1) != 1 or kbar.stride(-1) != 1 or kbar.dtype != torch.float32:
        raise UnsupportedShape("keys / kbar rows must be contiguous, kbar fp32")
    hc = None if head_cls is None else head_cls.detach().to(torch.float32).contiguous()
    pg = pages.to(torch.int64).contiguous()
    tk = _i32(tok).contiguous()
    a = _lib.KbarPlanArgs(keys=keys_cache.data_ptr(), k_sp=keys_cache.stride(0), k_st=keys_cache.stride(1),
                          head_cls=_lib.ptr(hc), pages=pg.data_ptr(), tok=tk.data_ptr(), kbar=kbar.data_ptr(),
                          kb_sp=kbar.stride(0), n=pg.numel(), num_pages=min(npages, kbar.shape[0]),
                          page_size=page, D=D, k_dtype=_lib.dtype_code(keys_cache.dtype))
    _lib.check(_lib.lib().srswa_kbar_plan(ctypes.byref(a), _lib.stream_ptr(kbar.device)), "srswa_kbar_plan")
    return kbar


def route_serve(scores, image_allow, out_idx, out_bias, *, K, M, idx_scale, prior_floor, inv_sigma):
    """The serving router over fp32 block scores [rows, W] (see
    ``srswa_route_serve``): writes the first M slots of each row of
    ``out_idx`` (int32) / ``out_bias`` (fp32) in place."""
    _require_cuda(scores, image_allow, out_idx, out_bias)
    rows, W = scores.shape
    if scores.dtype != torch.float32 or scores.stride(-1) != 1:
        raise UnsupportedShape("scores must be fp32 with contiguous rows")
    if out_idx.dtype != torch.int32 or out_bias.dtype != torch.float32 or out_idx.stride(-1) != 1 \
            or out_bias.stride(-1) != 1:
        raise UnsupportedShape("out_idx int32 / out_bias fp32 with contiguous rows")
    if out_idx.shape[0] < rows or out_bias.shape[0] < rows or out_idx.shape[-1] < M or out_bias.shape[-1] < M:
        raise ValueError(f"outputs {tuple(out_idx.shape)} / {tuple(out_bias.shape)} too small for {rows} x {M}")
    img = None
    if image_allow is not None:
        img = image_allow.view(torch.int8) if image_allow.dtype in (torch.bool, torch.uint8) else image_allow
        if img.dtype != torch.int8:
            img = (img != 0).to(torch.int8)
        if img.stride(-1) != 1:
            img = img.contiguous()
        if img.shape[0] < rows or img.shape[-1] < W:
            raise ValueError(f"image_allow {tuple(image_allow.shape)} smaller than the scores {rows} x {W}")
    a = _lib.RouteServeArgs(scores=scores.data_ptr(), sc_sn=scores.stride(0),
                            img=_lib.ptr(img), img_sn=img.stride(0) if img is not None else 0,
                            out_idx=out_idx.data_ptr(), oi_sn=out_idx.stride(0),
                            out_bias=out_bias.data_ptr(), ob_sn=out_bias.stride(0),
                            rows=rows, W=W, K=int(K), M=int(M), idx_scale=float(idx_scale),
                            prior_floor=float(prior_floor), inv_sigma=float(inv_sigma))
    _lib.check(_lib.lib().srswa_route_serve(ctypes.byref(a), _lib.stream_ptr(scores.device)), "srswa_route_serve")


def win_bounds(allow, seq_lens, lo, hi, fit, *, max_block, block_size, local_blocks, dql, tile):
    """Remote page span (lo, hi) and the narrow-tile flag of every decode row
    (see ``srswa_win_bounds``), written into int32 ``lo`` / ``hi`` and int8 ``fit``."""
    _require_cuda(allow, seq_lens, lo, hi, fit)
    nd = int(lo.numel())
    al = allow.view(torch.int8) if allow.dtype in (torch.bool, torch.uint8) else allow
    if al.dtype != torch.int8:
        al = (al != 0).to(torch.int8)
    if al.stride(-1) != 1:
        al = al.contiguous()
    if lo.dtype != torch.int32 or hi.dtype != torch.int32 or fit.dtype != torch.int8 or not (
            lo.is_contiguous() and hi.is_contiguous() and fit.is_contiguous()):
        raise UnsupportedShape("lo / hi int32, fit int8, contiguous")
    sl = _i32(seq_lens).contiguous()
    if al.shape[0] < nd or sl.numel() * max(1, int(dql)) < nd or hi.numel() < nd or fit.numel() < nd:
        raise ValueError(f"win bounds: {nd} rows need allow rows {al.shape[0]}, seq_lens x dql "
                         f"{sl.numel()} x {dql}, hi {hi.numel()}, fit {fit.numel()}")
    a = _lib.WinBoundsArgs(allow=al.data_ptr(), a_sn=al.stride(0), seq_lens=sl.data_ptr(), lo=lo.data_ptr(),
                           hi=hi.data_ptr(), fit=fit.data_ptr(), rows=nd, W=int(max_block), WQ=al.shape[1],
                           block_size=int(block_size), local_blocks=int(local_blocks), dql=max(1, int(dql)),
                           tile=int(tile))
    _lib.check(_lib.lib().srswa_win_bounds(ctypes.byref(a), _lib.stream_ptr(lo.device)), "srswa_win_bounds")


# ---------------------------------------------------------------------------
# DASH router
# ---------------------------------------------------------------------------
def dash_route(block_scores, block_cand, p, *, attend_ids=False):
    """``_infer_route_select`` (HF/modeling_deepseekv2.py:338-362) on the GPU.

    block_scores [B, Lq, nblk] fp32 (``SCORE_NEG`` = not a remote block);
    block_cand [B, Lq, nblk] bool page mask or None; ``p`` the router's
    ``_infer_params`` dict (idx_scale, floor, sigma, K, topm).  Returns
    (topi [B, Lq, K] int64, bias [B, Lq, K] fp32, valid [B, Lq, K] bool);
    with ``attend_ids`` topi is int32 with -1 in the invalid slots instead
    (``torch.where(valid, topi, -1)``, the ids the gather-attention kernels take).
    Raises ``UnsupportedShape`` for a top-M window above 64 blocks."""
    _require_cuda(block_scores, block_cand)
    B, Lq, nblk = block_scores.shape
    sc = block_scores.to(torch.float32)
    if sc.stride(-1) != 1:
        sc = sc.contiguous()
    cd = None
    if block_cand is not None:
        cd = block_cand.to(torch.bool).expand(B, Lq, nblk)
        if cd.stride(-1) != 1:
            cd = cd.contiguous()
        cd = cd.view(torch.uint8)
    M = max(1, min(int(p["topm"]), nblk)) if int(p["topm"]) > 0 else nblk
    K = max(1, min(int(p["K"]), M))
    topi = torch.empty(B, Lq, K, dtype=torch.int32, device=sc.device)
    bias = torch.empty(B, Lq, K, dtype=torch.float32, device=sc.device)
    valid = torch.empty(B, Lq, K, dtype=torch.bool, device=sc.device)
    a = _lib.RouteArgs(
        scores=sc.data_ptr(), sc_sb=sc.stride(0), sc_sq=sc.stride(1),
        cand=_lib.ptr(cd), cd_sb=cd.stride(0) if cd is not None else 0, cd_sq=cd.stride(1) if cd is not None else 0,
        topi=topi.data_ptr(), ti_sb=topi.stride(0), ti_sq=topi.stride(1),
        bias=bias.data_ptr(), bi_sb=bias.stride(0), bi_sq=bias.stride(1),
        valid=valid.data_ptr(), va_sb=valid.stride(0), va_sq=valid.stride(1),
        B=B, Lq=Lq, nblk=nblk, K=int(p["K"]), topm=int(p["topm"]),
        idx_scale=float(p["idx_scale"]), floor=float(p["floor"]), sigma=float(p["sigma"]),
        mask_ids=1 if attend_ids else 0)
    _lib.check(_lib.lib().srswa_dash_route(ctypes.byref(a), _lib.stream_ptr(sc.device)), "srswa_dash_route")
    return (topi if attend_ids else topi.to(torch.int64)), bias, valid


# ---------------------------------------------------------------------------
# gather-attention forward (matrix cores)
# ---------------------------------------------------------------------------
def _seg_from_positions(position_ids, T, Sk, device):
    """seg[b, t] = (Sk - T + t) - position_ids[b, t]: the key index where query
    t's sample starts (HF/sparse_gather_triton.py:413-416, generalised to a
    query chunk at the tail of a prefix cache).  None when all zero."""
    if position_ids is None:
        return None
    qi = torch.arange(Sk - T, Sk, device=device, dtype=torch.int64)
    seg = (qi[None, :] - position_ids.to(device=device, dtype=torch.int64)).to(torch.int32).contiguous()
    return seg


def gather_fwd(q, k, v, block_indices, *, block_size, local_window, scale, seg=None, bias=None,
               out=None, need_lse=True, tail_split=True):
    """Fused gather attention forward.

    q [B, T, HQ, D]; k, v [B, Sk, HKV, D] (Sk >= T, queries are the last T
    keys); block_indices [B, HI, T, S] (-1 pad); seg [B, T] int sample starts
    (None = 0); bias [B, T, S] or [B, HI, T, S] per-slot bias on remote keys.
    tail_split=False runs every tile as one workgroup (no workspace).
    Returns (o [B, T, HQ, D], lse [B, T, HQ] fp32 or None)."""
    _require_cuda(q, k, v, block_indices, seg, bias)
    B, T, HQ, D = q.shape
    Bk, Sk, HKV, Dk = k.shape
    if Bk != B or Dk != D or tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"k/v shape {tuple(k.shape)} incompatible with q {tuple(q.shape)}")
    if q.dtype != k.dtype or k.dtype != v.dtype:
        raise ValueError("q, k, v must share a dtype")
    for t in (q, k, v):
        if t.stride(-1) != 1:
            raise UnsupportedShape("head dim must be contiguous")
    HI, S = block_indices.shape[1], block_indices.shape[-1]
    if tuple(block_indices.shape) != (B, HI, T, S):
        raise ValueError(f"block_indices shape {tuple(block_indices.shape)} != {(B, HI, T, S)}")
    idx = _i32(block_indices).contiguous()
    if bias is not None:
        if bias.dim() == 3:
            bias = bias.unsqueeze(1)
        bias = bias.to(torch.float32).expand(B, HI, T, S).contiguous()
    if seg is not None:
        seg = _i32(seg).contiguous()
    if out is None:
        out = torch.empty(B, T, HQ, D, dtype=q.dtype, device=q.device)
    lse = torch.empty(B, T, HQ, dtype=torch.float32, device=q.device) if need_lse else None
    a = _lib.FwdArgs()
    a.q = q.data_ptr(); a.q_sb, a.q_st, a.q_sh = q.stride(0), q.stride(1), q.stride(2)
    a.k = k.data_ptr(); a.k_sb, a.k_st, a.k_sh = k.stride(0), k.stride(1), k.stride(2)
    a.v = v.data_ptr(); a.v_sb, a.v_st, a.v_sh = v.stride(0), v.stride(1), v.stride(2)
    a.idx = idx.data_ptr(); a.idx_sb, a.idx_sh, a.idx_st = idx.stride(0), idx.stride(1), idx.stride(2)
    if bias is not None:
        a.bias = bias.data_ptr(); a.bias_sb, a.bias_sh, a.bias_st = bias.stride(0), bias.stride(1), bias.stride(2)
    if seg is not None:
        a.seg = seg.data_ptr(); a.seg_sb = seg.stride(0)
    a.out = out.data_ptr(); a.o_sb, a.o_st, a.o_sh = out.stride(0), out.stride(1), out.stride(2)
    if lse is not None:
        a.lse = lse.data_ptr(); a.lse_sb, a.lse_st, a.lse_sh = lse.stride(0), lse.stride(1), lse.stride(2)
    a.B, a.T, a.Sk, a.HQ, a.HKV, a.HI, a.D, a.S = B, T, Sk, HQ, HKV, HI, D, S
    a.block_size, a.local_window = int(block_size), max(1, int(local_window))
    a.scale = float(scale)
    a.dtype = _lib.dtype_code(q.dtype)
    # the tail split's workspace (0 bytes when the launch's last round is full)
    nws = _lib.lib().srswa_gather_fwd_workspace(ctypes.byref(a)) if tail_split else 0
    ws = _lib.scratch(q.device, nws)
    _lib.check(_lib.lib().srswa_gather_fwd_ws(ctypes.byref(a), _lib.ptr(ws), nws, _lib.stream_ptr(q.device)),
               "srswa_gather_fwd_ws")
    return out, lse


def gather_bwd(q, k, v, o, lse, do, block_indices, *, block_size, local_window, scale, seg=None,
               bias=None, need_dbias=False):
    """Backward of ``gather_fwd``.  Returns (dq, dk, dv, dbias_heads) with
    dbias_heads [B, HQ, T, S] (per query head) when ``need_dbias`` and a bias
    was used, else None.  Deterministic (no floating-point atomics)."""
    _require_cuda(q, k, v, o, lse, do, block_indices, seg, bias)
    B, T, HQ, D = q.shape
    Sk, HKV = k.shape[1], k.shape[2]
    HI, S = block_indices.shape[1], block_indices.shape[-1]
    idx = _i32(block_indices).contiguous()
    if bias is not None:
        if bias.dim() == 3:
            bias = bias.unsqueeze(1)
        bias = bias.to(torch.float32).expand(B, HI, T, S).contiguous()
    if seg is not None:
        seg = _i32(seg).contiguous()
    if do.stride(-1) != 1:
        do = do.contiguous()
    dq = torch.empty(B, T, HQ, D, dtype=q.dtype, device=q.device)
    dk = torch.empty(B, Sk, HKV, D, dtype=k.dtype, device=k.device)
    dv = torch.empty(B, Sk, HKV, D, dtype=v.dtype, device=v.device)
    dbh = None
    if need_dbias and bias is not None:
        dbh = torch.empty(B, HQ, T, S, dtype=torch.float32, device=q.device)
    a = _lib.BwdArgs()
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o), ("dq", dq), ("dk", dk), ("dv", dv)):
        setattr(a, name, t.data_ptr())
        setattr(a, name + "_sb", t.stride(0))
        setattr(a, name + "_st", t.stride(1))
        setattr(a, name + "_sh", t.stride(2))
    a.dout = do.data_ptr(); a.do_sb, a.do_st, a.do_sh = do.stride(0), do.stride(1), do.stride(2)
    a.lse = lse.data_ptr(); a.lse_sb, a.lse_st, a.lse_sh = lse.stride(0), lse.stride(1), lse.stride(2)
    a.idx = idx.data_ptr(); a.idx_sb, a.idx_sh, a.idx_st = idx.stride(0), idx.stride(1), idx.stride(2)
    if bias is not None:
        a.bias = bias.data_ptr(); a.bias_sb, a.bias_sh, a.bias_st = bias.stride(0), bias.stride(1), bias.stride(2)
    if seg is not None:
        a.seg = seg.data_ptr(); a.seg_sb = seg.stride(0)
    if dbh is not None:
        a.dbias = dbh.data_ptr(); a.db_sb, a.db_sh, a.db_st = dbh.stride(0), dbh.stride(1), dbh.stride(2)
    a.B, a.T, a.Sk, a.HQ, a.HKV, a.HI, a.D, a.S = B, T, Sk, HQ, HKV, HI, D, S
    a.block_size, a.local_window = int(block_size), max(1, int(local_window))
    a.scale = float(scale)
    a.dtype = _lib.dtype_code(q.dtype)
    L_ = _lib.lib()
    nbytes = L_.srswa_gather_bwd_workspace(ctypes.byref(a))
    scr = _lib.scratch(q.device, nbytes)
    st = L_.srswa_gather_bwd(ctypes.byref(a), _lib.ptr(scr), nbytes, _lib.stream_ptr(q.device))
    _lib.check(st, "srswa_gather_bwd")
    return dq, dk, dv, dbh


class GatherAttnFn(torch.autograd.Function):
    """Autograd glue of the fused gather attention (forward + backward on the
    matrix cores).  Inputs are [B, T, H, D] views; ``bias`` (optional) is the
    per-slot bias [B, T, S] or [B, HI, T, S] and receives a gradient."""

    @staticmethod
    def forward(ctx, q, k, v, sel, seg, bias, block_size, scale, local_window):
        o, lse = gather_fwd(q, k, v, sel, block_size=block_size, local_window=local_window,
                            scale=scale, seg=seg, bias=bias)
        ctx.save_for_backward(q, k, v, sel, seg, bias, o, lse)
        ctx.cfg = (block_size, scale, local_window)
        ctx.bias_shape = None if bias is None else tuple(bias.shape)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, sel, seg, bias, o, lse = ctx.saved_tensors
        block_size, scale, local_window = ctx.cfg
        need_db = bias is not None and ctx.needs_input_grad[5]
        dq, dk, dv, dbh = gather_bwd(q, k, v, o, lse, do, sel, block_size=block_size,
                                     local_window=local_window, scale=scale, seg=seg, bias=bias,
                                     need_dbias=need_db)
        dbias = None
        if dbh is not None:
            B, HQ, T, S = dbh.shape
            HI = sel.shape[1]
            db = dbh.view(B, HI, HQ // HI, T, S).sum(2)            # heads -> their index head
            # the forward broadcast the bias to [B, HI, T, S]: sum the gradient
            # over every broadcast dim (a [B, T, S] bias feeds all HI heads)
            shape4 = (B, 1, T, S) if len(ctx.bias_shape) == 3 else ctx.bias_shape
            db = db.sum_to_size(shape4)
            dbias = (db[:, 0] if len(ctx.bias_shape) == 3 else db).to(bias.dtype)
        return dq, dk, dv, None, None, dbias, None, None, None


def block_max_score(q, k, pos, seg, *, block_size, num_key_blocks, local_window):
    """Indexer block-max score (see srswa_block_max_score): q [B, C, D],
    k [B, Sk, D], pos / seg [B, C] -> fp32 [B, C, num_key_blocks]."""
    _require_cuda(q, k, pos, seg)
    B, C, D = q.shape
    Sk = k.shape[1]
    if q.dtype != k.dtype:
        raise ValueError("q and k must share a dtype")
    if q.stride(-1) != 1:
        q = q.contiguous()
    if k.stride(-1) != 1:
        k = k.contiguous()
    posi = _i32(pos).contiguous()
    segi = None if seg is None else _i32(seg).contiguous()
    out = torch.empty(B, C, int(num_key_blocks), dtype=torch.float32, device=q.device)
    a = _lib.BlockMaxArgs()
    a.q = q.data_ptr(); a.q_sb, a.q_sc = q.stride(0), q.stride(1)
    a.k = k.data_ptr(); a.k_sb, a.k_sk = k.stride(0), k.stride(1)
    a.pos = posi.data_ptr(); a.pos_sb, a.pos_sc = posi.stride(0), posi.stride(1)
    if segi is not None:
        a.seg = segi.data_ptr(); a.seg_sb, a.seg_sc = segi.stride(0), segi.stride(1)
    a.out = out.data_ptr(); a.o_sb, a.o_sc, a.o_sn = out.stride(0), out.stride(1), out.stride(2)
    a.B, a.C, a.Sk, a.D, a.nblk = B, C, Sk, D, int(num_key_blocks)
    a.block_size, a.local_window = int(block_size), max(1, int(local_window))
    a.dtype = _lib.dtype_code(q.dtype)
    _lib.check(_lib.lib().srswa_block_max_score(ctypes.byref(a), _lib.stream_ptr(q.device)),
               "srswa_block_max_score")
    return out
