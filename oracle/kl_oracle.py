"""Gather-KL (indexer distillation) CPU oracle -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker.

Restates the KL term of the DASH/"sparse" stage training step: per query row
the teacher distribution over its selected remote keys (the main branch's
softmax, averaged over the index head's group of query heads, no gradient)
against the indexer's (student) log-softmax over the same keys:

* dense form: ``_kl_chunk_core`` HF/_sparse_base_impl.py:2071-2154 (wrapped by
  ``_KLChunkFn`` :2158-2190 for multi-index-head configs);
* gather form: the n_idx_heads == 1 branch of ``select_and_kl_loss``
  HF/_sparse_base_impl.py:3413-3478, and its reduction :3497-3498, 3516.

Rounding points kept from the reference: both matmuls return the input dtype
(bf16) before ``.float()``; the teacher logits are scaled after that rounding;
softmax / log-softmax / KL in fp32 (here: the dtype of the computation, float64
for the pinned checks).

Pinning (``tests/test_kl_pins.py``): the dense form equals an independent
restatement of the gather form; KL >= 0; KL == 0 when the student logits equal
a single teacher head's; the row reduction; and ``torch.autograd.gradcheck`` of
the differentiable student path in float64.
"""

from __future__ import annotations

import torch

NEG = -1e9


def _round(x: torch.Tensor, dtype) -> torch.Tensor:
    """x rounded to ``dtype`` and back (None: no rounding)."""
    return x if dtype is None else x.to(dtype).to(x.dtype)


def keep_mask(sel, pos, Sk: int, block_size: int, local_window: int, seg=None):
    """bool [B, HI, T, Sk]: key j kept for row (b, ih, t) when its block is
    selected, j <= pos, j is outside the token window (j < pos - LW + 1) and
    (packed rows) j >= seg.  HF/_sparse_base_impl.py:2106-2122, :3424-3440."""
    B, HI, T, K = sel.shape
    kb = torch.zeros(B, HI, T, -(-Sk // block_size) + 1, dtype=torch.bool)
    safe = torch.where(sel >= 0, sel.long(), torch.full_like(sel.long(), kb.shape[-1] - 1))
    kb.scatter_(-1, safe, True)
    keep = kb[..., :-1].repeat_interleave(block_size, dim=-1)[..., :Sk]
    j = torch.arange(Sk)
    p = pos.long()[:, None, :, None]
    local_start = (p - (local_window - 1)).clamp(min=0)
    keep = keep & (j <= p) & (j < local_start)
    if seg is not None:
        keep = keep & (j >= seg.long()[:, None, :, None])
    return keep


def gather_kl_dense(q_idx, idx_k, q_main, k_main, sel, pos, *, block_size, local_window, scaling,
                    seg=None, round_dtype=torch.bfloat16):
    """Per-row KL [B, HI, T] and validity [B, HI, T] (dense form).

    q_idx [B, HI, T, d], idx_k [B, Sk, d], q_main [B, HQ, T, Dh],
    k_main [B, HKV, Sk, Dh], sel [B, HI, T, K] block ids (-1 = empty),
    pos [B, T] key positions of the rows, seg [B, T] or None.
    Computed in the dtype of the inputs; ``q_idx`` / ``idx_k`` may require grad."""
    B, HI, T, _ = q_idx.shape
    HQ, HKV = q_main.shape[1], k_main.shape[1]
    Sk = idx_k.shape[1]
    group, kv_rep = HQ // HI, HQ // HKV
    keep = keep_mask(sel, pos, Sk, block_size, local_window, seg)
    s_idx = _round(torch.einsum("bhtd,bsd->bhts", q_idx, idx_k), round_dtype)
    s_idx = s_idx.masked_fill(~keep, NEG)
    log_p_idx = torch.log_softmax(s_idx, dim=-1)
    with torch.no_grad():
        p = torch.zeros_like(s_idx)
        for h in range(HQ):
            s_h = _round(torch.einsum("btd,bsd->bts", q_main[:, h], k_main[:, h // kv_rep]), round_dtype) * scaling
            s_h = s_h.masked_fill(~keep[:, h // group], NEG)
            p[:, h // group] += torch.softmax(s_h, dim=-1)
        p = p / group
    log_p = torch.log(p.clamp_min(1e-12))
    term = torch.where(keep, p * (log_p - log_p_idx), torch.zeros_like(p))
    return term.sum(-1), keep.any(-1)


def kl_loss(kl, valid):
    """sum(kl * valid) / (sum(valid) + 1e-6), HF/_sparse_base_impl.py:3497-3498, 3516."""
    v = valid.to(kl.dtype)
    return (kl * v).sum() / (v.sum() + 1e-6)
