"""Bind the MI355X kernels into a loaded Unlimited-OCR model package.

The reference swaps implementations by rebinding module attributes
(HF/modeling_deepseekv2.py:246-247); this module does the same for the
functions of the hot path that live inside the model code rather than in the
two kernel files (those are replaced file-for-file by
``srswa.sparse_gather_triton`` / ``srswa.sparse_gather_e2e_triton``):

* ``_decode_attend``       (HF/modeling_deepseekv2.py:454-481) -> ``srswa.ops.decode_attend``
* ``_block_scores_infer``  (HF/modeling_deepseekv2.py:380-430), stage0 "head_cls"
                           -> the head_cls / mean-pool indexer kernel
* ``_infer_route_select``  (HF/modeling_deepseekv2.py:338-362) -> ``srswa.ops.dash_route``

Every replacement keeps the reference signature and return convention, runs
the HIP kernels for device tensors, and hands host tensors (or a case the
kernels do not cover) to the original function -- the model code's own
eager path, exactly as the reference's wrappers fall back.
"""

from __future__ import annotations

import torch

from . import ops
from ._lib import UnsupportedShape

SCORE_NEG = -1.0e9


def head_cls_block_scores(idx_q, idx_k, q_pos, nblk, block_size, local_blocks, head_cls=None):
    """[B, Lq, nblk] fp32 remote block scores of one router (single index head):
    idx_q [B, Lq, d], idx_k [B, S, d], q_pos [B, Lq]; the semantics of
    ``_block_scores_infer`` stage0 == "head_cls"."""
    q = idx_q.unsqueeze(1)                               # [B, 1, Lq, d]
    _, scores = ops.index_meanpool_topk(q, idx_k, q_pos, block_size=block_size,
                                        local_blocks=local_blocks, topk=0, head_cls=head_cls,
                                        nblk=nblk, return_scores=True)
    return scores[:, 0]


def apply(modeling_deepseekv2) -> list:
    """Rebind the hot-path functions of a loaded ``modeling_deepseekv2`` module
    (the reference's DASH overlay).  Returns the names rebound; calling it
    twice is harmless (the originals are kept once)."""
    mod = modeling_deepseekv2
    done = []
    orig_decode = getattr(mod, "_srswa_orig_decode_attend", None) or getattr(mod, "_decode_attend", None)
    if orig_decode is not None:
        mod._srswa_orig_decode_attend = orig_decode

        def _decode_attend(q, k_all, v_all, topi, bias, valid, q_pos, block_size, local_window, scale):
            if q.is_cuda:
                try:
                    return ops.decode_attend(q, k_all, v_all, topi, bias, valid, q_pos, block_size,
                                             local_window, scale)
                except UnsupportedShape:
                    pass
            return orig_decode(q, k_all, v_all, topi, bias, valid, q_pos, block_size, local_window, scale)

        mod._decode_attend = _decode_attend
        done.append("_decode_attend")

    orig_scores = getattr(mod, "_srswa_orig_block_scores_infer", None) or getattr(mod, "_block_scores_infer", None)
    if orig_scores is not None:
        mod._srswa_orig_block_scores_infer = orig_scores

        def _block_scores_infer(router, idx_q, idx_k, q_pos, nblk):
            if idx_q.is_cuda and getattr(router, "stage0", None) == "head_cls":
                try:
                    hc = router.head_cls.detach().float()
                    hc = None if not bool(hc.any()) else hc      # zero head_cls == mean pooling
                    return head_cls_block_scores(idx_q, idx_k, q_pos, nblk, router.block_size,
                                                 router.local_blocks, hc)
                except UnsupportedShape:
                    pass
            return orig_scores(router, idx_q, idx_k, q_pos, nblk)

        mod._block_scores_infer = _block_scores_infer
        done.append("_block_scores_infer")

    orig_route = getattr(mod, "_srswa_orig_infer_route_select", None) or getattr(mod, "_infer_route_select", None)
    if orig_route is not None:
        mod._srswa_orig_infer_route_select = orig_route

        def _infer_route_select(block_scores, block_cand, p):
            if block_scores.is_cuda:
                try:
                    return ops.dash_route(block_scores, block_cand, p)
                except UnsupportedShape:
                    pass
            return orig_route(block_scores, block_cand, p)

        mod._infer_route_select = _infer_route_select
        done.append("_infer_route_select")
    return done


def restore(modeling_deepseekv2) -> None:
    """Undo ``apply``."""
    mod = modeling_deepseekv2
    if hasattr(mod, "_srswa_orig_decode_attend"):
        mod._decode_attend = mod._srswa_orig_decode_attend
        del mod._srswa_orig_decode_attend
    if hasattr(mod, "_srswa_orig_block_scores_infer"):
        mod._block_scores_infer = mod._srswa_orig_block_scores_infer
        del mod._srswa_orig_block_scores_infer
    if hasattr(mod, "_srswa_orig_infer_route_select"):
        mod._infer_route_select = mod._srswa_orig_infer_route_select
        del mod._srswa_orig_infer_route_select
