"""The DASH training router's block scorers on the MI355X kernels, forward
and backward:

* ``HeadClsScoreFn`` / ``head_cls_scores(idx_q, idx_k, head_cls, position_ids,
  nblk, block_size, local_blocks)`` -> z [B, S, nblk] fp32: stage 0 "head_cls"
  of ``DashAttention._block_scores_headcls`` (HF/dash_attention.py:1079-1143),
  from the index queries / keys; differentiable in idx_q, idx_k and head_cls
  (``srswa_hc_score_fwd`` / ``srswa_hc_score_bwd``).
* ``BlockMaxScoreFn`` / ``block_max_scores(idx_q, idx_k, position_ids, nblk,
  block_size, local_window)`` -> z [B, S, nblk] fp32: stage 0 "indexer" of
  ``DashAttention._block_scores`` (HF/dash_attention.py:1036-1050), the
  clamped remote block maxima, differentiable in idx_q and idx_k with torch's
  amax rule (``srswa_bm_score_fwd`` / ``srswa_bm_score_bwd``).
* ``block_scores_headcls`` / ``block_scores``: the drop-ins for the two
  methods.  The index projections, RMSNorms, RoPE, nan_to_num and gradient
  hooks (:1063-1078, :1011-1034) are the model's own torch modules, run as
  there; the scoring is the kernels'.

Every tensor must live on the GPU; head dims 64 / 128; block sizes 16, 32,
64, 128 for head_cls and 16, 32, 64 for block-max (else ``UnsupportedShape``
and the patched model runs its own method).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import UnsupportedShape

SCORE_NEG = -1.0e9
BLOCK_SIZES = (16, 32, 64, 128)
BM_BLOCK_SIZES = (16, 32, 64)


def _check(idx_q, idx_k, block_size):
    for t in (idx_q, idx_k):
        if not t.is_cuda:
            raise RuntimeError("srswa.train_scores takes device (cuda/hip) tensors; there is no CPU path")
    if idx_q.dim() != 3 or idx_k.shape != idx_q.shape:
        raise UnsupportedShape(f"idx_q / idx_k must both be [B, S, d] (got {tuple(idx_q.shape)}, "
                               f"{tuple(idx_k.shape)})")
    if idx_q.shape[-1] not in (64, 128) or int(block_size) not in BLOCK_SIZES:
        raise UnsupportedShape(f"head dim {idx_q.shape[-1]} / block size {block_size} not covered")


def _f32(t: torch.Tensor) -> torch.Tensor:
    t = t.float() if t.dtype != torch.float32 else t
    return t if t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(s % 4 == 0 for s in t.stride()[:-1]) \
        else t.contiguous()


def _positions(position_ids: torch.Tensor, B: int, S: int) -> torch.Tensor:
    p = position_ids
    if p.dim() == 1:
        p = p[None]
    return p.to(torch.int32).expand(B, S)


class HeadClsScoreFn(torch.autograd.Function):
    """z [B, S, nblk] of the head_cls stage 0, with the reference's gradient
    into idx_q, idx_k and head_cls."""

    @staticmethod
    def forward(ctx, idx_q, idx_k, head_cls, pos, nblk, block_size, local_blocks):
        q, k, hc = _f32(idx_q), _f32(idx_k), head_cls.float().contiguous()
        B, S, D = q.shape
        kbar = torch.empty(B, nblk, D, dtype=torch.float32, device=q.device)
        z = torch.empty(B, S, nblk, dtype=torch.float32, device=q.device)
        a = _lib.HcScoreArgs(
            q=q.data_ptr(), q_sb=q.stride(0), q_st=q.stride(1), k=k.data_ptr(), k_sb=k.stride(0), k_st=k.stride(1),
            head_cls=hc.data_ptr(), pos=pos.data_ptr(), pos_sb=pos.stride(0), pos_st=pos.stride(1),
            kbar=kbar.data_ptr(), kb_sb=kbar.stride(0), z=z.data_ptr(), z_sb=z.stride(0), z_st=z.stride(1),
            B=B, S=S, D=D, nblk=int(nblk), block_size=int(block_size), local_blocks=int(local_blocks))
        _lib.check(_lib.lib().srswa_hc_score_fwd(ctypes.byref(a), _lib.stream_ptr(q.device)), "srswa_hc_score_fwd")
        ctx.save_for_backward(q, k, hc, pos, kbar, z)
        ctx.meta = (int(nblk), int(block_size), int(local_blocks))
        return z

    @staticmethod
    def backward(ctx, gz):
        q, k, hc, pos, kbar, z = ctx.saved_tensors
        nblk, block_size, local_blocks = ctx.meta
        B, S, D = q.shape
        g = gz.float().contiguous()
        dq = torch.empty(B, S, D, dtype=torch.float32, device=q.device)
        # keys past nblk * block_size take no part in the scores (their rows stay 0)
        dk = (torch.zeros if nblk * block_size < S else torch.empty)(B, S, D, dtype=torch.float32, device=q.device)
        dhc = torch.empty(D, dtype=torch.float32, device=q.device)
        a = _lib.HcScoreBwdArgs(
            q=q.data_ptr(), q_sb=q.stride(0), q_st=q.stride(1), k=k.data_ptr(), k_sb=k.stride(0), k_st=k.stride(1),
            head_cls=hc.data_ptr(), pos=pos.data_ptr(), pos_sb=pos.stride(0), pos_st=pos.stride(1),
            kbar=kbar.data_ptr(), kb_sb=kbar.stride(0), z=z.data_ptr(), z_sb=z.stride(0), z_st=z.stride(1),
            gz=g.data_ptr(), gz_sb=g.stride(0), gz_st=g.stride(1),
            dq=dq.data_ptr(), dq_sb=dq.stride(0), dq_st=dq.stride(1),
            dk=dk.data_ptr(), dk_sb=dk.stride(0), dk_st=dk.stride(1), dhc=dhc.data_ptr(),
            B=B, S=S, D=D, nblk=nblk, block_size=block_size, local_blocks=local_blocks)
        need = ctypes.c_size_t()
        _lib.check(_lib.lib().srswa_hc_score_bwd_workspace(ctypes.byref(a), ctypes.byref(need)),
                   "srswa_hc_score_bwd_workspace")
        scr = _lib.scratch(q.device, need.value)
        _lib.check(_lib.lib().srswa_hc_score_bwd(ctypes.byref(a), _lib.ptr(scr), need.value, _lib.stream_ptr(q.device)),
                   "srswa_hc_score_bwd")
        return dq, dk, dhc, None, None, None, None


def head_cls_scores(idx_q, idx_k, head_cls, position_ids, nblk, block_size, local_blocks):
    """[B, S, nblk] fp32 remote block scores of the head_cls stage 0 (see the
    module docstring); idx_q, idx_k [B, S, d], head_cls [d], position_ids
    [B, S] (or [S])."""
    _check(idx_q, idx_k, block_size)
    B, S, _ = idx_q.shape
    if S == 0 or B == 0 or nblk <= 0:
        raise UnsupportedShape("empty scoring")
    pos = _positions(position_ids, B, S)
    return HeadClsScoreFn.apply(idx_q, idx_k, head_cls, pos, int(nblk), int(block_size), int(local_blocks))


def index_qk(router, hidden_states, position_embeddings, rope_fn, sanitize_grad):
    """The router's fp32 index queries / keys [B, S, d]: the projections,
    RMSNorms, RoPE and nan_to_num of HF/dash_attention.py:1063-1078 (and
    :1011-1034), run on the model's own modules, with the same gradient hooks."""
    B, S, _ = hidden_states.shape
    d = router.index_dim
    hs = torch.nan_to_num(hidden_states, nan=0.0, posinf=0.0, neginf=0.0)
    idx_q = router.q_norm(router.q_proj(hs).view(B, S, 1, d)).transpose(1, 2)
    idx_k = router.k_norm(router.k_proj(hs).view(B, S, 1, d)).transpose(1, 2)
    if rope_fn is not None and position_embeddings is not None:
        cos, sin = position_embeddings
        idx_q, idx_k = rope_fn(idx_q, idx_k, cos[..., :d], sin[..., :d])
    idx_q = torch.nan_to_num(idx_q[:, 0].float(), nan=0.0, posinf=0.0, neginf=0.0)
    idx_k = torch.nan_to_num(idx_k[:, 0].float(), nan=0.0, posinf=0.0, neginf=0.0)
    if sanitize_grad is not None:
        if idx_q.requires_grad:
            idx_q.register_hook(sanitize_grad)
        if idx_k.requires_grad:
            idx_k.register_hook(sanitize_grad)
    return idx_q, idx_k


def block_scores_headcls(router, hidden_states, position_embeddings, position_ids, nblk, *, rope_fn=None,
                         sanitize_grad=None):
    """Drop-in for ``DashAttention._block_scores_headcls`` (HF/dash_attention.py:
    1053-1143): [B, S, nblk] fp32, the model's index projections feeding the
    head_cls scoring kernels."""
    if not hidden_states.is_cuda:
        raise UnsupportedShape("host tensors")
    d = router.index_dim
    if d not in (64, 128) or int(router.block_size) not in BLOCK_SIZES:
        raise UnsupportedShape(f"index dim {d} / block size {router.block_size} not covered")
    B, S, _ = hidden_states.shape
    if position_ids is None:
        position_ids = torch.arange(S, device=hidden_states.device)[None].expand(B, -1)
    idx_q, idx_k = index_qk(router, hidden_states, position_embeddings, rope_fn, sanitize_grad)
    return head_cls_scores(idx_q, idx_k, router.head_cls.to(torch.float32), position_ids, nblk,
                           router.block_size, router.local_blocks)


class BlockMaxScoreFn(torch.autograd.Function):
    """z [B, S, nblk] of the block-max stage 0 with torch's amax gradient
    into idx_q and idx_k."""

    @staticmethod
    def forward(ctx, idx_q, idx_k, pos, nblk, block_size, local_window):
        q, k = _f32(idx_q), _f32(idx_k)
        B, S, D = q.shape
        z = torch.empty(B, S, nblk, dtype=torch.float32, device=q.device)
        code = torch.empty(B, nblk, S, dtype=torch.int32, device=q.device)
        # written only where several keys share a maximum: never read elsewhere
        tiemask = torch.empty(B, S, nblk, dtype=torch.int64, device=q.device)
        a = _lib.BmScoreArgs(
            q=q.data_ptr(), q_sb=q.stride(0), q_st=q.stride(1), k=k.data_ptr(), k_sb=k.stride(0), k_st=k.stride(1),
            pos=pos.data_ptr(), pos_sb=pos.stride(0), pos_st=pos.stride(1),
            z=z.data_ptr(), z_sb=z.stride(0), z_st=z.stride(1), code=code.data_ptr(), tiemask=tiemask.data_ptr(),
            B=B, S=S, D=D, nblk=int(nblk), block_size=int(block_size), local_window=int(local_window))
        _lib.check(_lib.lib().srswa_bm_score_fwd(ctypes.byref(a), _lib.stream_ptr(q.device)), "srswa_bm_score_fwd")
        ctx.save_for_backward(q, k, pos, code, tiemask)
        ctx.meta = (int(nblk), int(block_size), int(local_window))
        return z

    @staticmethod
    def backward(ctx, gz):
        q, k, pos, code, tiemask = ctx.saved_tensors
        nblk, block_size, local_window = ctx.meta
        B, S, D = q.shape
        g = gz.float().contiguous()
        dq = torch.empty(B, S, D, dtype=torch.float32, device=q.device)
        dk = (torch.zeros if nblk * block_size < S else torch.empty)(B, S, D, dtype=torch.float32, device=q.device)
        a = _lib.BmScoreBwdArgs(
            q=q.data_ptr(), q_sb=q.stride(0), q_st=q.stride(1), k=k.data_ptr(), k_sb=k.stride(0), k_st=k.stride(1),
            pos=pos.data_ptr(), pos_sb=pos.stride(0), pos_st=pos.stride(1), code=code.data_ptr(),
            tiemask=tiemask.data_ptr(), gz=g.data_ptr(), gz_sb=g.stride(0), gz_st=g.stride(1),
            dq=dq.data_ptr(), dq_sb=dq.stride(0), dq_st=dq.stride(1),
            dk=dk.data_ptr(), dk_sb=dk.stride(0), dk_st=dk.stride(1),
            B=B, S=S, D=D, nblk=nblk, block_size=block_size, local_window=local_window)
        need = ctypes.c_size_t()
        _lib.check(_lib.lib().srswa_bm_score_bwd_workspace(ctypes.byref(a), ctypes.byref(need)),
                   "srswa_bm_score_bwd_workspace")
        scr = _lib.scratch(q.device, need.value)
        _lib.check(_lib.lib().srswa_bm_score_bwd(ctypes.byref(a), _lib.ptr(scr), need.value, _lib.stream_ptr(q.device)),
                   "srswa_bm_score_bwd")
        return dq, dk, None, None, None, None


def block_max_scores(idx_q, idx_k, position_ids, nblk, block_size, local_window):
    """[B, S, nblk] fp32 remote block maxima of the block-max stage 0 (see the
    module docstring); idx_q, idx_k [B, S, d], position_ids [B, S] (or [S])."""
    _check(idx_q, idx_k, block_size)
    if int(block_size) not in BM_BLOCK_SIZES:
        raise UnsupportedShape(f"block size {block_size} not covered by the block-max scorer")
    B, S, _ = idx_q.shape
    if S == 0 or B == 0 or nblk <= 0 or int(nblk) * int(block_size) < S:
        raise UnsupportedShape("empty scoring or fewer blocks than keys")
    pos = _positions(position_ids, B, S)
    return BlockMaxScoreFn.apply(idx_q, idx_k, pos, int(nblk), int(block_size), int(local_window))


def block_scores(router, hidden_states, position_embeddings, position_ids, nblk, *, rope_fn=None,
                 sanitize_grad=None):
    """Drop-in for ``DashAttention._block_scores`` (HF/dash_attention.py:
    1005-1050): [B, S, nblk] fp32, the model's index projections feeding the
    block-max scoring kernels."""
    if not hidden_states.is_cuda:
        raise UnsupportedShape("host tensors")
    d = router.index_dim
    B, S, _ = hidden_states.shape
    if d not in (64, 128) or int(router.block_size) not in BM_BLOCK_SIZES or int(nblk) * int(router.block_size) < S:
        raise UnsupportedShape(f"index dim {d} / block size {router.block_size} not covered")
    if position_ids is None:
        position_ids = torch.arange(S, device=hidden_states.device)[None].expand(B, -1)
    idx_q, idx_k = index_qk(router, hidden_states, position_embeddings, rope_fn, sanitize_grad)
    return block_max_scores(idx_q, idx_k, position_ids, nblk, router.block_size, router.local_window)
