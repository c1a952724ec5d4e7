"""Drop-in replacement of hf-model-code/sparse_gather_e2e_triton.py on MI355X.

``SPARSE_E2E_SENTINEL`` and ``triton_gather_attention_e2e``
(HF/sparse_gather_e2e_triton.py:355-407) with the reference's signature and
None-fallback gates, backed by the gfx950 kernels: the per-slot bias
``blk_bias_slots`` [B, T, S] is read by the kernels directly (no dense
[B, T, M] scatter) and receives its gradient (sum of dS over the remote keys
of each selected block, summed over heads) without atomics.
"""

from __future__ import annotations

import torch

from . import ops
from ._lib import UnsupportedShape
from .sparse_gather_triton import _local_meta

SPARSE_E2E_SENTINEL = 1


def triton_gather_attention_e2e(query_states, key_states, value_states, block_indices,
                                blk_bias_slots, position_ids, attention_mask, block_size, scale,
                                local_window=None):
    """query_states [B, HQ, T, D]; key/value_states [B, Hkv, T, D]; block_indices
    [B, 1, T, S]; blk_bias_slots [B, T, S]; position_ids [B, T] (must be arange).
    Returns [B, HQ, T, D] or None (reference gates)."""
    if attention_mask is not None:
        return None
    if block_indices.shape[1] != 1:
        return None
    B, HQ, T, D = query_states.shape
    if key_states.shape[2] != T:
        return None
    if position_ids is None or position_ids.dim() != 2 or position_ids.shape[-1] != T:
        return None
    ar = torch.arange(T, device=position_ids.device)
    if not bool((position_ids == ar).all()):
        return None
    lw, _ = _local_meta(block_size, local_window)
    q = query_states.transpose(1, 2)
    k = key_states.transpose(1, 2)
    v = value_states.transpose(1, 2)
    try:
        o = ops.GatherAttnFn.apply(q, k, v, block_indices, None, blk_bias_slots, block_size, scale, lw)
    except UnsupportedShape:
        return None
    return o.transpose(1, 2)
