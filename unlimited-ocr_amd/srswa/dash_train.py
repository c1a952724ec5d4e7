"""The DASH router of the training step on the MI355X kernels:
``DashAttention._route`` and ``DashAttention._select_and_bias``
(HF/dash_attention.py:1145-1204), differentiable like the reference (the
entmax prior carries the LM loss's gradient from the bias back to the block
scores, :1309-1316).

* ``route(self, block_scores, image_block_mask, block_cand)`` -> (prior, cand):
  candidates under the per-query block mask or the page-agnostic image-block
  mask with the per-row fallback, then 1.5-entmax over every block
  (``srswa_dash_route_train``; backward ``srswa_dash_route_train_bwd``, the
  Jacobian-vector product of ``_Entmax15.backward`` :799-806).  The one-shot
  per-layer calibration of the reference (:1166-1169) runs as there, on the
  candidates, before the prior.
* ``select_and_bias(self, prior, cand, nblk)`` -> (topi, bias, valid): the K
  largest masked priors (ties -> the lower block id; the reference's
  ``topk`` leaves their order open, and entmax's exact zeros tie whenever its
  support is narrower than K) and the centred log-prior bias
  (``srswa_dash_select_train``; backward ``srswa_dash_select_train_bwd``).

Every tensor must live on the GPU; fp32 / bf16 / fp16 scores, at most 8192
blocks per row and K <= 64 (else ``UnsupportedShape`` and the patched model
runs its own method)."""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from ._lib import UnsupportedShape

SCORE_NEG = -1.0e9
MAX_BLOCKS = 8192


def _rows2d(t: torch.Tensor, nblk: int) -> torch.Tensor:
    """[..., nblk] as a [rows, nblk] view with unit column stride (copied if needed)."""
    t2 = t.reshape(-1, nblk)
    return t2 if t2.stride(-1) == 1 else t2.contiguous()


def _u8(t: torch.Tensor) -> torch.Tensor:
    """bool / uint8 masks are read in place as bytes (0 = false)."""
    if t.dtype == torch.bool:
        return t.view(torch.uint8) if t.is_contiguous() else t.contiguous().view(torch.uint8)
    return t.to(torch.uint8) if t.dtype != torch.uint8 else t


def candidates(block_scores, image_block_mask, block_cand, image_only):
    """bool [B, S, nblk] candidate blocks of ``_route`` (HF/dash_attention.py:
    1157-1165) in torch ops on the device, for the calibration hook only."""
    remote = block_scores > (SCORE_NEG * 0.5)
    cand = remote
    if block_cand is not None:
        cand = remote & block_cand
    elif image_only and image_block_mask is not None:
        cand = remote & image_block_mask[:, None, :]
    return torch.where(~cand.any(dim=-1, keepdim=True), remote, cand)


def route_forward(block_scores, block_cand, image_mask, scale, neg):
    """(prior like block_scores, cand bool) of ``srswa_dash_route_train``."""
    if not block_scores.is_cuda:
        raise RuntimeError("srswa.dash_train takes device tensors; there is no CPU path")
    if block_scores.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise UnsupportedShape("dash route: scores must be fp32 / bf16 / fp16")
    shape = block_scores.shape
    nblk = int(shape[-1])
    if nblk > MAX_BLOCKS:
        raise UnsupportedShape(f"dash route: {nblk} blocks per row (at most {MAX_BLOCKS})")
    sc = _rows2d(block_scores, nblk)
    rows = sc.shape[0]
    prior = torch.empty(rows, nblk, dtype=sc.dtype, device=sc.device)
    cand = torch.empty(rows, nblk, dtype=torch.bool, device=sc.device)
    bc = None if block_cand is None else _rows2d(_u8(block_cand.expand(shape).contiguous()), nblk)
    im = None
    if bc is None and image_mask is not None:
        im = _u8(image_mask).reshape(-1, nblk)
        im = im if im.stride(-1) == 1 else im.contiguous()
    rows_per_seq = rows // max(1, im.shape[0]) if im is not None else 1
    a = _lib.DashRouteTrainArgs(
        scores=sc.data_ptr(), sc_sr=sc.stride(0),
        block_cand=_lib.ptr(bc), bc_sr=0 if bc is None else bc.stride(0),
        img=_lib.ptr(im), img_sb=0 if im is None else im.stride(0),
        prior=prior.data_ptr(), p_sr=prior.stride(0), cand=cand.data_ptr(), c_sr=cand.stride(0),
        rows=rows, nblk=nblk, rows_per_seq=rows_per_seq, scale=float(scale), neg=float(neg),
        dtype=_lib.dtype_code(sc.dtype))
    _lib.check(_lib.lib().srswa_dash_route_train(ctypes.byref(a), _lib.stream_ptr(sc.device)),
               "srswa_dash_route_train")
    return prior.view(shape), cand.view(shape)


def route_backward(d_prior, prior, cand, scale):
    nblk = int(prior.shape[-1])
    dp = _rows2d(d_prior.to(prior.dtype), nblk)
    pr = _rows2d(prior, nblk)
    cd = _rows2d(cand, nblk)
    ds = torch.empty(pr.shape, dtype=pr.dtype, device=pr.device)
    a = _lib.DashRouteTrainBwdArgs(
        d_prior=dp.data_ptr(), dp_sr=dp.stride(0), prior=pr.data_ptr(), p_sr=pr.stride(0),
        cand=cd.data_ptr(), c_sr=cd.stride(0), d_scores=ds.data_ptr(), ds_sr=ds.stride(0),
        rows=pr.shape[0], nblk=nblk, scale=float(scale), dtype=_lib.dtype_code(pr.dtype))
    _lib.check(_lib.lib().srswa_dash_route_train_bwd(ctypes.byref(a), _lib.stream_ptr(pr.device)),
               "srswa_dash_route_train_bwd")
    return ds.view(prior.shape)


def _select_args(prior, cand, K, floor, sigma):
    nblk = int(prior.shape[-1])
    pr = _rows2d(prior, nblk)
    cd = _rows2d(cand, nblk)
    return pr, cd, _lib.DashSelectTrainArgs(
        prior=pr.data_ptr(), p_sr=pr.stride(0), cand=cd.data_ptr(), c_sr=cd.stride(0),
        rows=pr.shape[0], nblk=nblk, K=int(K), floor=float(floor), inv_sigma=float(1.0 / sigma),
        dtype=_lib.dtype_code(pr.dtype))


def select_forward(prior, cand, K, floor, sigma):
    """(topi int64, bias like prior, valid bool), each [..., K]."""
    if int(K) > 64 or int(K) > int(prior.shape[-1]) or int(prior.shape[-1]) > MAX_BLOCKS:
        raise UnsupportedShape(f"dash select: K = {K} over {prior.shape[-1]} blocks")
    pr, cd, a = _select_args(prior, cand, K, floor, sigma)
    rows = pr.shape[0]
    topi = torch.empty(rows, int(K), dtype=torch.int64, device=pr.device)
    bias = torch.empty(rows, int(K), dtype=pr.dtype, device=pr.device)
    valid = torch.empty(rows, int(K), dtype=torch.bool, device=pr.device)
    a.topi, a.ti_sr = topi.data_ptr(), topi.stride(0)
    a.bias, a.b_sr = bias.data_ptr(), bias.stride(0)
    a.valid, a.v_sr = valid.data_ptr(), valid.stride(0)
    _lib.check(_lib.lib().srswa_dash_select_train(ctypes.byref(a), _lib.stream_ptr(pr.device)),
               "srswa_dash_select_train")
    out = (*prior.shape[:-1], int(K))
    return topi.view(out), bias.view(out), valid.view(out)


def select_backward(d_bias, prior, cand, topi, floor, sigma):
    pr, cd, a = _select_args(prior, cand, topi.shape[-1], floor, sigma)
    ti = topi.reshape(pr.shape[0], -1).contiguous()
    db = d_bias.to(pr.dtype).reshape(pr.shape[0], -1).contiguous()
    dp = torch.empty(pr.shape, dtype=pr.dtype, device=pr.device)
    a.topi, a.ti_sr = ti.data_ptr(), ti.stride(0)
    a.d_bias, a.db_sr = db.data_ptr(), db.stride(0)
    a.d_prior, a.dp_sr = dp.data_ptr(), dp.stride(0)
    _lib.check(_lib.lib().srswa_dash_select_train_bwd(ctypes.byref(a), _lib.stream_ptr(pr.device)),
               "srswa_dash_select_train_bwd")
    return dp.view(prior.shape)


class RouteTrainFn(torch.autograd.Function):
    """(prior, cand) of block scores; differentiable in block_scores."""

    @staticmethod
    def forward(ctx, block_scores, block_cand, image_mask, scale, neg):
        prior, cand = route_forward(block_scores, block_cand, image_mask, scale, neg)
        ctx.set_materialize_grads(False)     # no zero tensor for the bool output's gradient
        ctx.save_for_backward(prior, cand)
        ctx.scale = scale
        ctx.mark_non_differentiable(cand)
        return prior, cand

    @staticmethod
    def backward(ctx, d_prior, d_cand):
        prior, cand = ctx.saved_tensors
        if d_prior is None:
            return None, None, None, None, None
        return route_backward(d_prior, prior, cand, ctx.scale), None, None, None, None


class SelectTrainFn(torch.autograd.Function):
    """(topi, bias, valid) of the prior; differentiable in prior through bias."""

    @staticmethod
    def forward(ctx, prior, cand, K, floor, sigma):
        topi, bias, valid = select_forward(prior, cand, K, floor, sigma)
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(prior, cand, topi)
        ctx.floor, ctx.sigma = floor, sigma
        ctx.mark_non_differentiable(topi, valid)
        return topi, bias, valid

    @staticmethod
    def backward(ctx, d_topi, d_bias, d_valid):
        prior, cand, topi = ctx.saved_tensors
        if d_bias is None:
            return None, None, None, None, None
        return select_backward(d_bias, prior, cand, topi, ctx.floor, ctx.sigma), None, None, None, None


def route(self, block_scores, image_block_mask, block_cand=None, *, sched=None):
    """``DashAttention._route`` on the kernels (``self`` the DashAttention);
    ``sched``: the model package's per-layer scheduler (``_SCHED``)."""
    if not block_scores.is_cuda:
        raise UnsupportedShape("dash route: host tensors")
    if int(block_scores.shape[-1]) > MAX_BLOCKS:
        raise UnsupportedShape("dash route: too many blocks")
    if sched is not None and sched.needs_calib(self._sched_id, self.training):
        cand = candidates(block_scores, image_block_mask, block_cand, self.image_only)
        sched.calibrate(self._sched_id, block_scores.detach(), cand, self._neg, math.sqrt(self.index_dim))
    img = image_block_mask if (block_cand is None and self.image_only and image_block_mask is not None) else None
    return RouteTrainFn.apply(block_scores, block_cand, img, float(self._cur_idx_scale()), float(self._neg))


def select_and_bias(self, prior, cand, nblk, *, k_budget):
    """``DashAttention._select_and_bias`` on the kernels; ``k_budget``: the
    current top-k budget (the package's ``_KS.k``)."""
    if not prior.is_cuda:
        raise UnsupportedShape("dash select: host tensors")
    K = max(1, min(int(k_budget), int(nblk)))
    return SelectTrainFn.apply(prior, cand, K, float(self._cur_prior_floor()), float(self.sigma))
