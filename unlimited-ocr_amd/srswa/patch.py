"""Bind the MI355X kernels into a loaded Unlimited-OCR model package.

The reference swaps implementations by rebinding module attributes
(HF/modeling_deepseekv2.py:246-247); this module does the same for the
functions of the hot path that live inside the model code rather than in the
two kernel files (those are replaced file-for-file by
``srswa.sparse_gather_triton`` / ``srswa.sparse_gather_e2e_triton``):

* ``_decode_attend``       (HF/modeling_deepseekv2.py:454-481) -> ``srswa.ops.decode_attend``
* ``_block_scores_infer``  (HF/modeling_deepseekv2.py:380-430): stage0 "head_cls"
                           -> the head_cls / mean-pool indexer kernel; stage0
                           "indexer" -> the block-max kernel
                           (``srswa.indexer.block_scores_indexer``)
* ``_infer_route_select``  (HF/modeling_deepseekv2.py:338-362) -> ``srswa.ops.dash_route``
* page isolation and the Page2D indexer RoPE of ``_sparse_base_impl`` (reached as
  ``modeling_deepseekv2._base``): ``DeepseekV2Indexer._build_kl_candidate_mask``
  (HF/_sparse_base_impl.py:2706-2737), ``_build_page_aware_ids`` (:2404-2502),
  ``_build_page_rope_pos`` (:2511-2570), ``DeepseekV2IndexerRotary2D.forward``
  (:2046-2061) and the module's ``_llama_apply_rotary_pos_emb`` (:39-41)
  -> ``srswa.page_isolation``; with ``modeling_unlimitedocr`` given, also its
  ``_uocr_dash_decode_allow`` (HF/modeling_unlimitedocr.py:481-528)
* ``DashAttention._route`` / ``_select_and_bias`` (HF/dash_attention.py:1145-1204),
  the training router -> ``srswa.dash_train``
* ``DashAttention._block_scores_headcls`` / ``_block_scores``
  (HF/dash_attention.py:1053-1143 / 1005-1050), the training router's stage-0
  scorers -> ``srswa.train_scores``
* ``_KLChunkFn`` (HF/_sparse_base_impl.py:2158-2190), the KL of the indexer
  distillation loss -> ``srswa.kl.KLChunkFn``
* ``DeepseekV2Indexer.select_and_kl_loss`` (HF/_sparse_base_impl.py:3240-3516),
  the indexer's training selection and KL -> ``srswa.indexer.select_and_kl_loss``,
  and ``DeepseekV2Indexer.forward`` (:3065-3105), its block selection
  -> ``srswa.indexer.indexer_forward``

Every replacement keeps the reference signature and return convention, runs
the HIP kernels for device tensors, and hands host tensors (or a case the
kernels do not cover) to the original function -- the model code's own
eager path, exactly as the reference's wrappers fall back.
"""

from __future__ import annotations

import sys

import torch

from . import dash_train, indexer, kl, ops, page_isolation, train_scores
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


_HC_ZERO: dict = {}


def _head_cls_or_none(param):
    """head_cls as fp32, or None while it is all zero (zero head_cls weights
    every valid key of a block equally: the mean-pool kernel path).  The zero
    test reads the device once per parameter version (an optimizer step bumps
    the version), not on every decode step."""
    key = (id(param), param.data_ptr(), param._version)
    zero = _HC_ZERO.get(key)
    if zero is None:
        if len(_HC_ZERO) > 256:
            _HC_ZERO.clear()
        zero = _HC_ZERO[key] = not bool(param.detach().any())
    return None if zero else param.detach().float()


def _rebind(owner, name: str, make, done: list, label: str) -> None:
    """owner.name = make(original); the original is kept once as
    owner._srswa_orig_<name> so ``restore`` can put it back."""
    keep = "_srswa_orig_" + name
    orig = getattr(owner, keep, None) or getattr(owner, name, None)
    if orig is None:
        return
    setattr(owner, keep, orig)
    setattr(owner, name, make(orig))
    done.append(label)


def _unbind(owner, name: str) -> None:
    keep = "_srswa_orig_" + name
    if owner is not None and keep in vars(owner):
        setattr(owner, name, vars(owner)[keep])
        delattr(owner, keep)


def _page_isolation(mod, base, done: list) -> None:
    indexer_cls = getattr(base, "DeepseekV2Indexer", None)
    if indexer_cls is not None:
        def make_mask(orig):
            def _build_kl_candidate_mask(self, pos_chunk, num_key_blocks, image_token_mask, batch, cq,
                                         image_token_page_ids=None, query_token_page_ids=None):
                if pos_chunk.is_cuda:
                    try:
                        return page_isolation.build_kl_candidate_mask(
                            self, pos_chunk, num_key_blocks, image_token_mask, batch, cq,
                            image_token_page_ids, query_token_page_ids)
                    except UnsupportedShape:
                        pass
                return orig(self, pos_chunk, num_key_blocks, image_token_mask, batch, cq,
                            image_token_page_ids, query_token_page_ids)
            return _build_kl_candidate_mask
        _rebind(indexer_cls, "_build_kl_candidate_mask", make_mask, done, "DeepseekV2Indexer._build_kl_candidate_mask")
    if indexer_cls is not None:
        def make_ids(orig):
            def _build_page_aware_ids(self, source_input_ids, img_context_token_id, page_token_id, key_length):
                # the first call prints the reference's one-shot diagnostic
                if getattr(self, "_page_aware_diag_logged", False) and source_input_ids is not None:
                    try:
                        return page_isolation.build_page_aware_ids(
                            self, source_input_ids, img_context_token_id, page_token_id, key_length,
                            page_scope_prefill=bool(getattr(base, "_PAGE_SCOPE_PREFILL", True)))
                    except UnsupportedShape:
                        pass
                return orig(self, source_input_ids, img_context_token_id, page_token_id, key_length)
            return _build_page_aware_ids
        _rebind(indexer_cls, "_build_page_aware_ids", make_ids, done, "DeepseekV2Indexer._build_page_aware_ids")

        def make_pos(orig):
            def _build_page_rope_pos(self, source_input_ids, key_length):
                if getattr(self, "_page_rope_diag_logged", False) and source_input_ids is not None:
                    try:
                        return page_isolation.build_page_rope_pos(self, source_input_ids, key_length)
                    except UnsupportedShape:
                        pass
                return orig(self, source_input_ids, key_length)
            return _build_page_rope_pos
        _rebind(indexer_cls, "_build_page_rope_pos", make_pos, done, "DeepseekV2Indexer._build_page_rope_pos")
    rot_cls = getattr(base, "DeepseekV2IndexerRotary2D", None)
    if rot_cls is not None:
        def make_rot(orig):
            def forward(self, x, tok_pos, page_pos):
                if x.is_cuda:
                    try:
                        return page_isolation.rotary2d_forward(self, x, tok_pos, page_pos)
                    except UnsupportedShape:
                        pass
                return orig(self, x, tok_pos, page_pos)
            return forward
        _rebind(rot_cls, "forward", make_rot, done, "DeepseekV2IndexerRotary2D.forward")
    for owner in (base, mod):
        if owner is not None and hasattr(owner, "_llama_apply_rotary_pos_emb"):
            def make_rope(orig):
                def _llama_apply_rotary_pos_emb(q, k, cos, sin, position_ids=None, unsqueeze_dim=1):
                    return page_isolation.apply_rotary_pos_emb(q, k, cos, sin, position_ids, unsqueeze_dim,
                                                               orig=orig)
                return _llama_apply_rotary_pos_emb
            _rebind(owner, "_llama_apply_rotary_pos_emb", make_rope, done,
                    f"{getattr(owner, '__name__', 'module')}._llama_apply_rotary_pos_emb")


def _kl_chunk(base, done: list) -> None:
    if base is None or not hasattr(base, "_KLChunkFn"):
        return

    def make(orig):
        class _KLChunkFn:
            """``_KLChunkFn`` on the gather-KL kernels; host tensors and shapes
            the kernels do not take use the original."""

            @staticmethod
            def apply(q_chunk, idx_k, q_main_chunk, k_main, keep_block, pos_chunk, block_size, scaling, group,
                      kv_group, local_window=None, same_seg=None):
                if q_chunk.is_cuda:
                    try:
                        return kl.KLChunkFn.apply(q_chunk, idx_k, q_main_chunk, k_main, keep_block, pos_chunk,
                                                  block_size, scaling, group, kv_group, local_window, same_seg)
                    except UnsupportedShape:
                        pass
                return orig.apply(q_chunk, idx_k, q_main_chunk, k_main, keep_block, pos_chunk, block_size, scaling,
                                  group, kv_group, local_window, same_seg)
        return _KLChunkFn
    _rebind(base, "_KLChunkFn", make, done, "_KLChunkFn")


def _select_and_kl(base, done: list) -> None:
    indexer_cls = getattr(base, "DeepseekV2Indexer", None)
    if indexer_cls is None:
        return

    def make(orig):
        def select_and_kl_loss(self, hidden_states, query_states, key_states, position_embeddings, position_ids,
                               scaling, image_token_mask=None, image_token_page_ids=None, query_token_page_ids=None):
            try:
                return indexer.select_and_kl_loss(self, hidden_states, query_states, key_states, position_embeddings,
                                                  position_ids, scaling, image_token_mask, image_token_page_ids,
                                                  query_token_page_ids, pk=getattr(base, "_pk", None))
            except UnsupportedShape:
                pass
            return orig(self, hidden_states, query_states, key_states, position_embeddings, position_ids, scaling,
                        image_token_mask=image_token_mask, image_token_page_ids=image_token_page_ids,
                        query_token_page_ids=query_token_page_ids)
        return select_and_kl_loss
    _rebind(indexer_cls, "select_and_kl_loss", make, done, "DeepseekV2Indexer.select_and_kl_loss")

    def make_fwd(orig):
        def forward(self, hidden_states, position_embeddings, past_key_values, position_ids, image_token_mask=None):
            try:
                return indexer.indexer_forward(self, hidden_states, position_embeddings, past_key_values,
                                               position_ids, image_token_mask)
            except UnsupportedShape:
                pass
            return orig(self, hidden_states, position_embeddings, past_key_values, position_ids,
                        image_token_mask=image_token_mask)
        return forward
    _rebind(indexer_cls, "forward", make_fwd, done, "DeepseekV2Indexer.forward")


def _dash_router(mod, done: list) -> None:
    dash_cls = getattr(mod, "DashAttention", None)
    if dash_cls is None:
        return
    dash_mod = sys.modules.get(getattr(dash_cls, "__module__", ""), None)

    def make_route(orig):
        def _route(self, block_scores, image_block_mask, block_cand=None):
            try:
                return dash_train.route(self, block_scores, image_block_mask, block_cand,
                                        sched=getattr(dash_mod, "_SCHED", None))
            except UnsupportedShape:
                pass
            return orig(self, block_scores, image_block_mask, block_cand)
        return _route

    def make_select(orig):
        def _select_and_bias(self, prior, cand, nblk):
            ks = getattr(dash_mod, "_KS", None)
            if ks is not None:
                try:
                    return dash_train.select_and_bias(self, prior, cand, nblk, k_budget=ks.k)
                except UnsupportedShape:
                    pass
            return orig(self, prior, cand, nblk)
        return _select_and_bias
    def make_headcls(orig):
        def _block_scores_headcls(self, hidden_states, position_embeddings, position_ids, nblk):
            if hidden_states.is_cuda:
                try:
                    return train_scores.block_scores_headcls(
                        self, hidden_states, position_embeddings, position_ids, nblk,
                        rope_fn=getattr(dash_mod, "_rope_fn", None),
                        sanitize_grad=getattr(dash_mod, "_sanitize_grad", None))
                except UnsupportedShape:
                    pass
            return orig(self, hidden_states, position_embeddings, position_ids, nblk)
        return _block_scores_headcls

    def make_blockmax(orig):
        def _block_scores(self, hidden_states, position_embeddings, position_ids, nblk):
            if hidden_states.is_cuda:
                try:
                    return train_scores.block_scores(
                        self, hidden_states, position_embeddings, position_ids, nblk,
                        rope_fn=getattr(dash_mod, "_rope_fn", None),
                        sanitize_grad=getattr(dash_mod, "_sanitize_grad", None))
                except UnsupportedShape:
                    pass
            return orig(self, hidden_states, position_embeddings, position_ids, nblk)
        return _block_scores

    _rebind(dash_cls, "_route", make_route, done, "DashAttention._route")
    _rebind(dash_cls, "_select_and_bias", make_select, done, "DashAttention._select_and_bias")
    _rebind(dash_cls, "_block_scores_headcls", make_headcls, done, "DashAttention._block_scores_headcls")
    _rebind(dash_cls, "_block_scores", make_blockmax, done, "DashAttention._block_scores")


def apply(modeling_deepseekv2, modeling_unlimitedocr=None) -> list:
    """Rebind the hot-path functions of a loaded ``modeling_deepseekv2`` module
    (the reference's DASH overlay), of its ``_sparse_base_impl`` (``_base``)
    and, when given, of ``modeling_unlimitedocr``.  Returns the names rebound;
    calling it twice is harmless (the originals are kept once)."""
    mod = modeling_deepseekv2
    done = []
    _page_isolation(mod, getattr(mod, "_base", None), done)
    _kl_chunk(getattr(mod, "_base", None), done)
    _select_and_kl(getattr(mod, "_base", None), done)
    _dash_router(mod, done)
    if modeling_unlimitedocr is not None:
        def make_allow(orig):
            def _uocr_dash_decode_allow(indexer, input_ids, cache):
                if input_ids.is_cuda:
                    try:
                        return page_isolation.uocr_dash_decode_allow(indexer, input_ids, cache)
                    except UnsupportedShape:
                        pass
                return orig(indexer, input_ids, cache)
            return _uocr_dash_decode_allow
        _rebind(modeling_unlimitedocr, "_uocr_dash_decode_allow", make_allow, done, "_uocr_dash_decode_allow")
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
            stage0 = getattr(router, "stage0", None)
            if idx_q.is_cuda and stage0 == "head_cls":
                try:
                    return head_cls_block_scores(idx_q, idx_k, q_pos, nblk, router.block_size,
                                                 router.local_blocks, _head_cls_or_none(router.head_cls))
                except UnsupportedShape:
                    pass
            elif idx_q.is_cuda and stage0 == "indexer":
                try:
                    return indexer.block_scores_indexer(router, idx_q, idx_k, q_pos, nblk)
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


def restore(modeling_deepseekv2, modeling_unlimitedocr=None) -> None:
    """Undo ``apply``."""
    mod = modeling_deepseekv2
    base = getattr(mod, "_base", None)
    for owner, name in ((getattr(base, "DeepseekV2Indexer", None), "_build_kl_candidate_mask"),
                        (getattr(base, "DeepseekV2Indexer", None), "_build_page_aware_ids"),
                        (getattr(base, "DeepseekV2Indexer", None), "_build_page_rope_pos"),
                        (getattr(base, "DeepseekV2Indexer", None), "select_and_kl_loss"),
                        (getattr(base, "DeepseekV2Indexer", None), "forward"),
                        (getattr(mod, "DashAttention", None), "_route"),
                        (getattr(mod, "DashAttention", None), "_select_and_bias"),
                        (getattr(mod, "DashAttention", None), "_block_scores_headcls"),
                        (getattr(mod, "DashAttention", None), "_block_scores"),
                        (getattr(base, "DeepseekV2IndexerRotary2D", None), "forward"),
                        (base, "_llama_apply_rotary_pos_emb"), (mod, "_llama_apply_rotary_pos_emb"),
                        (base, "_KLChunkFn"),
                        (modeling_unlimitedocr, "_uocr_dash_decode_allow")):
        _unbind(owner, name)
    if hasattr(mod, "_srswa_orig_decode_attend"):
        mod._decode_attend = mod._srswa_orig_decode_attend
        del mod._srswa_orig_decode_attend
    if hasattr(mod, "_srswa_orig_block_scores_infer"):
        mod._block_scores_infer = mod._srswa_orig_block_scores_infer
        del mod._srswa_orig_block_scores_infer
    if hasattr(mod, "_srswa_orig_infer_route_select"):
        mod._infer_route_select = mod._srswa_orig_infer_route_select
        del mod._srswa_orig_infer_route_select
