"""Gather-KL of the indexer distillation loss (training) on the MI355X kernels.

* ``gather_kl(q_idx, idx_k, q_main, k_main, sel, pos, ...)`` -> (kl, valid):
  the KL of the n_idx_heads == 1 gather branch of ``select_and_kl_loss``
  (HF/_sparse_base_impl.py:3413-3478), generalised to several index heads;
  differentiable in ``q_idx`` and ``idx_k`` (the teacher has no gradient).
* ``KLChunkFn`` -- drop-in for ``_KLChunkFn`` (HF/_sparse_base_impl.py:2158-2190,
  core ``_kl_chunk_core`` :2071-2154): same ``apply`` arguments (block-level
  keep mask instead of ids) and return value.

Every tensor must live on the GPU; the kernels take bf16 / fp16 with a head
dimension of 64 or 128 and 64-key blocks (other cases raise
``UnsupportedShape``, and the patched model falls back to its own code).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import UnsupportedShape


def _cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("srswa.kl takes device (cuda/hip) tensors; there is no CPU path")


def _inner(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _keys(idx_k: torch.Tensor) -> torch.Tensor:
    """idx_k as [B, Sk, d] (the reference passes [B, 1, Sk, d])."""
    return idx_k[:, 0] if idx_k.dim() == 4 else idx_k


_SIDE: dict = {}


def side_channel(device):
    """(stream, fork event, join event) handles of ``device``, passed to the
    KL entry points so that their tile kernels run beside the block-major
    ones.  They belong to this module (the C library owns no stream or event):
    created once per device with the default stream priority, on the first
    call that asks for them -- make that call before any graph capture."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    sc = _SIDE.get(idx)
    if sc is None:
        with torch.cuda.device(idx):
            s = torch.cuda.Stream(device=idx)
            fork, join = torch.cuda.Event(), torch.cuda.Event()
            fork.record(s)                           # torch creates an event on its first record
            join.record(s)
        sc = _SIDE[idx] = (s, fork, join)
    return sc


def _side_fields(device, use: bool) -> dict:
    if not use:
        return dict(side_stream=None, fork_event=None, join_event=None)
    s, fork, join = side_channel(device)
    return dict(side_stream=s.cuda_stream, fork_event=fork.cuda_event, join_event=join.cuda_event)


def kl_forward(q_idx, idx_k, q_main, k_main, sel, pos, *, block_size, local_window, scaling, seg=None,
               with_dsel=True, row_sparse=True, side_stream=True, slots_are_blocks=False):
    """(kl [B, HI, T] fp32, valid [B, HI, T] bool, dsel [B, HI, T, K, 64] fp32 or None).
    ``slots_are_blocks``: sel [B, HI, T, ceil(Sk / 64)] lists block s in slot s
    (sel[..., s] == s, else -1), any number of blocks per row; dsel rows of
    unlisted slots are left unwritten.
    ``row_sparse``: tiles whose rows select unrelated blocks are computed
    block-major (srswa_gather_kl_fwd_ws); False runs every tile on the tile
    kernel (srswa_gather_kl_fwd).  ``side_stream``: the row-sparse call runs
    its tile kernels on this module's second stream (``side_channel``), forked
    from and joined back to the current stream; False keeps every kernel on
    the current stream."""
    _cuda(q_idx, idx_k, q_main, k_main, sel, pos, seg)
    q_idx, q_main, k_main = _inner(q_idx), _inner(q_main), _inner(k_main)
    ik = _inner(_keys(idx_k))
    B, HI, T, D = q_idx.shape
    HQ, HKV, Sk = q_main.shape[1], k_main.shape[1], ik.shape[1]
    if q_main.shape[-1] != D or k_main.shape[-1] != D or ik.shape[-1] != D:
        raise UnsupportedShape("gather kl: the index and main head dims must match")
    if q_idx.dtype != ik.dtype or q_idx.dtype != q_main.dtype or q_idx.dtype != k_main.dtype:
        raise UnsupportedShape("gather kl: all operands must share one dtype")
    s = sel.to(torch.int32).contiguous()
    K = s.shape[-1]
    ps = pos.to(device=q_idx.device, dtype=torch.int32).contiguous()
    sg = None if seg is None else seg.to(device=q_idx.device, dtype=torch.int32).contiguous()
    kl = torch.empty(B, HI, T, dtype=torch.float32, device=q_idx.device)
    valid = torch.empty(B, HI, T, dtype=torch.bool, device=q_idx.device)
    dsel = torch.empty(B, HI, T, K, 64, dtype=torch.float32, device=q_idx.device) if with_dsel else None
    a = _lib.KlArgs(
        q_idx=q_idx.data_ptr(), qi_sb=q_idx.stride(0), qi_sh=q_idx.stride(1), qi_st=q_idx.stride(2),
        idx_k=ik.data_ptr(), ik_sb=ik.stride(0), ik_st=ik.stride(1),
        q_main=q_main.data_ptr(), qm_sb=q_main.stride(0), qm_sh=q_main.stride(1), qm_st=q_main.stride(2),
        k_main=k_main.data_ptr(), km_sb=k_main.stride(0), km_sh=k_main.stride(1), km_st=k_main.stride(2),
        sel=s.data_ptr(), sel_sb=s.stride(0), sel_sh=s.stride(1), sel_st=s.stride(2),
        pos=ps.data_ptr(), pos_sb=ps.stride(0), seg=_lib.ptr(sg), seg_sb=0 if sg is None else sg.stride(0),
        kl=kl.data_ptr(), kl_sb=kl.stride(0), kl_sh=kl.stride(1),
        valid=valid.data_ptr(), va_sb=valid.stride(0), va_sh=valid.stride(1),
        dsel=_lib.ptr(dsel), ds_sb=0 if dsel is None else dsel.stride(0),
        ds_sh=0 if dsel is None else dsel.stride(1), ds_st=0 if dsel is None else dsel.stride(2),
        B=B, HI=HI, HQ=HQ, HKV=HKV, T=T, Sk=Sk, D=D, K=K, block_size=int(block_size),
        local_window=int(local_window), scaling=float(scaling), dtype=_lib.dtype_code(q_idx.dtype),
        slots_are_blocks=1 if slots_are_blocks else 0,
        **_side_fields(q_idx.device, side_stream and row_sparse))
    # with a workspace, tiles whose rows select unrelated blocks are taken by
    # the block-major (row-sparse) kernels instead of the tile kernel
    need = _lib.lib().srswa_gather_kl_fwd_workspace(ctypes.byref(a)) if row_sparse else 0
    if need == 0:                                    # the tile kernel alone (or an empty batch)
        _lib.check(_lib.lib().srswa_gather_kl_fwd(ctypes.byref(a), _lib.stream_ptr(q_idx.device)),
                   "srswa_gather_kl_fwd")
        return kl, valid, dsel
    scr = _lib.scratch(q_idx.device, need)
    _lib.check(_lib.lib().srswa_gather_kl_fwd_ws(ctypes.byref(a), _lib.ptr(scr), need, _lib.stream_ptr(q_idx.device)),
               "srswa_gather_kl_fwd_ws")
    return kl, valid, dsel


def kl_backward(grad, q_idx, idx_k, sel, dsel, *, block_size, side_stream=True, slots_are_blocks=False):
    """(d q_idx like q_idx, d idx_k like idx_k) for d loss / d kl = grad [B, HI, T].
    ``side_stream`` and ``slots_are_blocks`` as in ``kl_forward``."""
    _cuda(grad, q_idx, idx_k, sel, dsel)
    qi = _inner(q_idx)
    ik = _inner(_keys(idx_k))
    B, HI, T, D = qi.shape
    Sk = ik.shape[1]
    s = sel.to(torch.int32).contiguous()
    g = grad.to(torch.float32).contiguous()
    dq = torch.empty(B, HI, T, D, dtype=qi.dtype, device=qi.device)
    dk = torch.empty(B, Sk, D, dtype=ik.dtype, device=ik.device)
    a = _lib.KlBwdArgs(
        q_idx=qi.data_ptr(), qi_sb=qi.stride(0), qi_sh=qi.stride(1), qi_st=qi.stride(2),
        idx_k=ik.data_ptr(), ik_sb=ik.stride(0), ik_st=ik.stride(1),
        sel=s.data_ptr(), sel_sb=s.stride(0), sel_sh=s.stride(1), sel_st=s.stride(2),
        dsel=dsel.data_ptr(), ds_sb=dsel.stride(0), ds_sh=dsel.stride(1), ds_st=dsel.stride(2),
        grad=g.data_ptr(), g_sb=g.stride(0), g_sh=g.stride(1),
        dq_idx=dq.data_ptr(), dq_sb=dq.stride(0), dq_sh=dq.stride(1), dq_st=dq.stride(2),
        dk_idx=dk.data_ptr(), dk_sb=dk.stride(0), dk_st=dk.stride(1),
        B=B, HI=HI, T=T, Sk=Sk, D=D, K=s.shape[-1], block_size=int(block_size), dtype=_lib.dtype_code(qi.dtype),
        slots_are_blocks=1 if slots_are_blocks else 0, **_side_fields(qi.device, side_stream))
    need = ctypes.c_size_t()
    _lib.check(_lib.lib().srswa_gather_kl_bwd_workspace(ctypes.byref(a), ctypes.byref(need)),
               "srswa_gather_kl_bwd_workspace")
    scr = _lib.scratch(qi.device, need.value)
    _lib.check(_lib.lib().srswa_gather_kl_bwd(ctypes.byref(a), _lib.ptr(scr), need.value, _lib.stream_ptr(qi.device)),
               "srswa_gather_kl_bwd")
    return dq, dk.view(idx_k.shape)


class GatherKLFn(torch.autograd.Function):
    """(kl, valid) with the student-path gradient (the teacher is detached)."""

    @staticmethod
    def forward(ctx, q_idx, idx_k, q_main, k_main, sel, pos, seg, block_size, local_window, scaling,
                slots_are_blocks=False):
        kl, valid, dsel = kl_forward(q_idx, idx_k, q_main.detach(), k_main.detach(), sel, pos,
                                     block_size=block_size, local_window=local_window, scaling=scaling, seg=seg,
                                     with_dsel=q_idx.requires_grad or idx_k.requires_grad,
                                     slots_are_blocks=slots_are_blocks)
        ctx.save_for_backward(q_idx, idx_k, sel, dsel if dsel is not None else kl)
        ctx.block_size = block_size
        ctx.slots_are_blocks = slots_are_blocks
        ctx.mark_non_differentiable(valid)
        return kl, valid

    @staticmethod
    def backward(ctx, gkl, gvalid):
        q_idx, idx_k, sel, dsel = ctx.saved_tensors
        if gkl is None:
            return (None,) * 11
        dq, dk = kl_backward(gkl, q_idx, idx_k, sel, dsel, block_size=ctx.block_size,
                             slots_are_blocks=ctx.slots_are_blocks)
        return dq, dk, None, None, None, None, None, None, None, None, None


def gather_kl(q_idx, idx_k, q_main, k_main, sel, pos, *, block_size, local_window, scaling, seg=None,
              slots_are_blocks=False):
    """Per-row KL [B, HI, T] (fp32, differentiable in q_idx / idx_k) and its
    validity [B, HI, T] (bool).  q_idx [B, HI, T, d]; idx_k [B, Sk, d] or
    [B, 1, Sk, d]; q_main [B, HQ, T, d]; k_main [B, HKV, Sk, d]; sel
    [B, HI, T, K] block ids (-1 = empty), K <= 64, or with ``slots_are_blocks``
    [B, HI, T, ceil(Sk / 64)] with sel[..., s] in {s, -1}; pos [B, T] key
    positions of the rows; seg [B, T] first key of each row's sample (packed
    rows) or None."""
    return GatherKLFn.apply(q_idx, idx_k, q_main, k_main, sel, pos, seg, block_size, local_window, scaling,
                            slots_are_blocks)


class KLChunkFn:
    """Drop-in for ``_KLChunkFn``: ``apply(q_chunk, idx_k, q_main_chunk, k_main,
    keep_block, pos_chunk, block_size, scaling, group, kv_group, local_window=None,
    same_seg=None)`` -> kl [B, HI, C], differentiable in q_chunk and idx_k."""

    @staticmethod
    def apply(q_chunk, idx_k, q_main_chunk, k_main, keep_block, pos_chunk, block_size, scaling, group, kv_group,
              local_window=None, same_seg=None):
        del group, kv_group                    # implied by the head counts of the operands
        lw = block_size if local_window is None else local_window
        nblk = keep_block.shape[-1]
        # slot s holds block s (-1 where not kept): every block of the row's
        # keep mask, however many (the warmup stage keeps every KL-eligible
        # block), with no read-back; listed blocks outside the row's kept key
        # range are dropped here (the kernels would give them zero rows)
        ar = torch.arange(nblk, device=keep_block.device, dtype=torch.int32)
        seg = None
        if same_seg is not None:               # [B, 1, C, Sk]: first key of the row's sample
            seg = same_seg[:, 0].to(torch.int8).argmax(dim=-1)
        hi = (pos_chunk.to(torch.int64) - lw + 1).clamp(min=0)                       # [B, C]
        lo = seg.to(torch.int64) if seg is not None else torch.zeros_like(hi)
        in_range = (ar[None, None, :] * block_size < hi[..., None]) & (ar[None, None, :] * block_size + block_size >
                                                                       lo[..., None])
        keep = keep_block & in_range[:, None]
        sel = torch.where(keep, ar, torch.full_like(ar, -1))
        kl, _ = gather_kl(q_chunk, idx_k, q_main_chunk, k_main, sel, pos_chunk, block_size=block_size,
                          local_window=lw, scaling=scaling, seg=seg, slots_are_blocks=True)
        return kl
