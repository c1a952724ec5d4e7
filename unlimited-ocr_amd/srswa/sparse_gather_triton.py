"""Drop-in replacement of hf-model-code/sparse_gather_triton.py on MI355X.

Same module-level names and call signatures as the reference:
``SPARSE_BLOCK_SIZE_SENTINEL``, ``triton_gather_attention`` (HF/sparse_gather_triton.py:379-434)
and ``triton_block_max_score`` (HF/sparse_gather_triton.py:488-524), backed by
the gfx950 HIP kernels of libsrswa.so instead of Triton.  Return conventions
are the reference's: ``triton_gather_attention`` returns ``None`` for inputs
the fused path does not take (attention mask present, index-head count not
tiling the heads, malformed position ids, a dtype/shape the kernels do not
cover) so the caller falls back to its eager path.  Differences, all
supersets: a query chunk at the tail of a longer KV cache (q_len < k_len) is
accepted instead of returning None; index heads need only divide the query
heads (the reference also requires them to divide the kv heads,
HF/sparse_gather_triton.py:405-407: each query head here picks its own index
and kv head); and duplicate block ids are collapsed inside the kernels (no
host-side sort).
"""

from __future__ import annotations

import torch

from . import ops
from ._lib import UnsupportedShape

SPARSE_BLOCK_SIZE_SENTINEL = 128


def _local_meta(block_size, local_window):
    """(window length, physical blocks it can touch) -- HF/sparse_gather_triton.py:298-305."""
    lw = block_size if local_window is None else int(local_window)
    lw = max(1, lw)
    return lw, (lw + block_size - 1) // block_size + 1


def triton_gather_attention(query_states, key_states, value_states, block_indices, position_ids,
                            attention_mask, block_size, scale, local_window=None):
    """Fused gather attention.  query_states [B, HQ, T, D]; key/value_states
    [B, Hkv, Sk, D] (Sk >= T: the queries are the last T keys); block_indices
    [B, HI, T, S] (-1 = padding); position_ids [B, T].  Returns [B, HQ, T, D]
    (a transposed view, like the reference) or None when unsupported."""
    if attention_mask is not None:
        return None
    B, HQ, T, D = query_states.shape
    HI = block_indices.shape[1]
    if HI < 1 or HQ % HI != 0:
        return None
    if key_states.shape[2] < T:
        return None
    if position_ids is None or position_ids.dim() != 2 or position_ids.shape[-1] != T:
        return None
    Sk = key_states.shape[2]
    lw, _ = _local_meta(block_size, local_window)
    seg = ops._seg_from_positions(position_ids, T, Sk, query_states.device)
    q = query_states.transpose(1, 2)
    k = key_states.transpose(1, 2)
    v = value_states.transpose(1, 2)
    try:
        o = ops.GatherAttnFn.apply(q, k, v, block_indices, seg, None, block_size, scale, lw)
    except UnsupportedShape:
        return None
    return o.transpose(1, 2)


def triton_block_max_score(q, k, pos, seg, block_size, num_key_blocks, local_window=None):
    """Block-level max of q.k over non-local, causal, same-segment keys.

    q [B, C, D], k [B, Sk, D], pos / seg [B, C] -> [B, C, num_key_blocks] fp32
    (-inf where a block has no valid key).  HF/sparse_gather_triton.py:488-524."""
    assert q.dim() == 3 and k.dim() == 3, "expects [B, C, D] / [B, Sk, D]"
    lw = block_size if local_window is None else max(1, int(local_window))
    return ops.block_max_score(q, k, pos, seg, block_size=block_size,
                               num_key_blocks=num_key_blocks, local_window=lw)
