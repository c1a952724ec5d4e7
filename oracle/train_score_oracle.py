"""DASH training block-scorer CPU oracle -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker.

Restates, in plain torch with autograd, the two stage-0 scorers of the DASH
training router from their index queries / keys (the output of the layer's
projections, RMSNorms, RoPE and nan_to_num, which the model runs itself):

* ``headcls_scores``  -- ``DashAttention._block_scores_headcls``
  HF/dash_attention.py:1079-1143 (the head_cls softmax summary per block, then
  the remote-only summary scores), including the gradient hook on the score
  matmul output (:1131-1132);
* ``blockmax_scores`` -- ``DashAttention._block_scores`` HF/dash_attention.py:
  1036-1050 (clamped token scores, remote-only, amax per block).

``sanitize_grad`` restates ``_sanitize_grad`` (HF/dash_attention.py:749-755).
Everything runs in the dtype of its inputs (float64 for the pinned checks).

Pinning (``tests/test_train_score_pins.py``): with head_cls = 0 the summary is
the block mean and the scores equal the pinned mean-pool oracle
(``srswa_oracle.meanpool_block_scores``) and a pure-Python brute force; the
scores are invariant to permuting a block's keys; a head_cls that is a large
multiple of one key's direction makes the summary that key; gradcheck of both
scorers in float64; the block-max forward and its gradient against a
pure-Python brute force (one-hot on the arg-max key, split evenly between
tied keys, nothing through clamped or masked scores).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

SCORE_NEG = -1.0e9      # _SCORE_NEG, HF/dash_attention.py:741
ACT_CLAMP = 1.0e4       # _ACT_CLAMP, HF/dash_attention.py:747
GRAD_CLAMP = 1.0e4      # _GRAD_CLAMP, HF/dash_attention.py:746


def sanitize_grad(g):
    """nan_to_num + bound (HF/dash_attention.py:749-755)."""
    if g is None:
        return None
    return torch.nan_to_num(g, nan=0.0, posinf=0.0, neginf=0.0).clamp(-GRAD_CLAMP, GRAD_CLAMP)


def headcls_summary(idx_k, head_cls, nblk, block_size):
    """(k_bar [B, nblk, d], chunk_valid [B, nblk]) of HF/dash_attention.py:1088-1119."""
    B, S, d = idx_k.shape
    bs = int(block_size)
    inv_sqrt_d = 1.0 / math.sqrt(d)
    Sp = nblk * bs
    if Sp > S:
        kk = F.pad(idx_k, (0, 0, 0, Sp - S))
        real = F.pad(torch.ones(B, S, dtype=torch.bool), (0, Sp - S), value=False)
    else:
        kk = idx_k[:, :Sp]
        real = torch.ones(B, Sp, dtype=torch.bool)
    kk = kk.reshape(B, nblk, bs, d)
    vmask = real.view(B, nblk, bs)
    hc = head_cls.to(kk.dtype).view(1, 1, 1, d)
    aw = (kk * hc).sum(-1) * inv_sqrt_d
    aw = aw.clamp(-ACT_CLAMP, ACT_CLAMP)
    neg = torch.finfo(aw.dtype).min
    row_max = torch.where(vmask, aw, aw.new_full((), neg)).amax(dim=-1, keepdim=True)
    row_max = torch.where(vmask.any(dim=-1, keepdim=True), row_max, torch.zeros_like(row_max))
    aw = aw - row_max
    e = torch.exp(aw) * vmask.to(aw.dtype)
    w = e / e.sum(dim=-1, keepdim=True).clamp_min(1e-6)
    k_bar = (w.unsqueeze(-1) * kk).sum(dim=2)
    k_bar = torch.nan_to_num(k_bar, nan=0.0, posinf=0.0, neginf=0.0)
    return k_bar, vmask.any(dim=-1)


def headcls_scores(idx_q, idx_k, head_cls, position_ids, nblk, block_size, local_blocks, hooks=True):
    """[B, S, nblk] remote block scores of ``_block_scores_headcls``
    (HF/dash_attention.py:1079-1143) from idx_q, idx_k [B, S, d], head_cls [d]
    and position_ids [B, S]; ``hooks`` keeps the gradient hook of the score
    matmul output (:1131-1132)."""
    d = idx_k.shape[-1]
    inv_sqrt_d = 1.0 / math.sqrt(d)
    k_bar, chunk_valid = headcls_summary(idx_k, head_cls, nblk, block_size)
    z = torch.matmul(idx_q, k_bar.transpose(-1, -2))                      # [B, S, nblk]
    if hooks and z.requires_grad:
        z.register_hook(sanitize_grad)
    z = z * inv_sqrt_d
    z = z.clamp(-ACT_CLAMP, ACT_CLAMP)
    qblk = position_ids.long() // int(block_size)
    blk_ids = torch.arange(nblk)
    remote_ok = blk_ids[None, None, :] <= (qblk[:, :, None] - int(local_blocks))
    keep = remote_ok & chunk_valid[:, None, :]
    return z.masked_fill(~keep, SCORE_NEG)


def blockmax_scores(idx_q, idx_k, position_ids, nblk, block_size, local_window):
    """[B, S, nblk] remote block scores of ``_block_scores``
    (HF/dash_attention.py:1036-1050): token scores clamped to +-1e4, keys in
    the query's causal local window or after it masked to -1e9, amax per
    block (the last block padded with -1e9)."""
    B, S, _ = idx_k.shape
    bs = int(block_size)
    kpos = torch.arange(S)
    Sp = nblk * bs
    sc = torch.matmul(idx_q, idx_k.transpose(-1, -2))
    sc = sc.clamp(-ACT_CLAMP, ACT_CLAMP)
    pos = position_ids.long()
    future = kpos[None, None, :] > pos[:, :, None]
    local = (kpos[None, None, :] > (pos[:, :, None] - int(local_window))) & ~future
    sc = sc.masked_fill(future | local, SCORE_NEG)
    if Sp > S:
        sc = F.pad(sc, (0, Sp - S), value=SCORE_NEG)
    else:
        sc = sc[..., :Sp]
    sc = sc.reshape(B, S, nblk, bs)
    return sc.amax(dim=-1)


def index_qk(router, hidden_states, position_embeddings, rope_fn):
    """The router's index queries / keys [B, S, d] with their gradient hooks:
    HF/dash_attention.py:1063-1078 (the same lines open ``_block_scores``,
    :1011-1034)."""
    B, S, _ = hidden_states.shape
    d = router.index_dim
    hs = torch.nan_to_num(hidden_states, nan=0.0, posinf=0.0, neginf=0.0)
    idx_q = router.q_norm(router.q_proj(hs).view(B, S, 1, d)).transpose(1, 2)
    idx_k = router.k_norm(router.k_proj(hs).view(B, S, 1, d)).transpose(1, 2)
    if rope_fn is not None and position_embeddings is not None:
        cos, sin = position_embeddings
        idx_q, idx_k = rope_fn(idx_q, idx_k, cos[..., :d], sin[..., :d])
    dt = torch.promote_types(idx_q.dtype, torch.float32)
    idx_q = torch.nan_to_num(idx_q[:, 0].to(dt), nan=0.0, posinf=0.0, neginf=0.0)
    idx_k = torch.nan_to_num(idx_k[:, 0].to(dt), nan=0.0, posinf=0.0, neginf=0.0)
    if idx_q.requires_grad:
        idx_q.register_hook(sanitize_grad)
    if idx_k.requires_grad:
        idx_k.register_hook(sanitize_grad)
    return idx_q, idx_k


def headcls_method(router, hidden_states, position_embeddings, position_ids, nblk, rope_fn=None):
    """The whole of ``DashAttention._block_scores_headcls`` (HF/dash_attention.py:
    1053-1143) on a router object: index projections then ``headcls_scores``."""
    idx_q, idx_k = index_qk(router, hidden_states, position_embeddings, rope_fn)
    return headcls_scores(idx_q, idx_k, router.head_cls.to(idx_k.dtype), position_ids, nblk, router.block_size,
                          router.local_blocks)


def blockmax_method(router, hidden_states, position_embeddings, position_ids, nblk, rope_fn=None):
    """The whole of ``DashAttention._block_scores`` (HF/dash_attention.py:
    1005-1050) on a router object: index projections then ``blockmax_scores``."""
    idx_q, idx_k = index_qk(router, hidden_states, position_embeddings, rope_fn)
    return blockmax_scores(idx_q, idx_k, position_ids, nblk, router.block_size, router.local_window)
