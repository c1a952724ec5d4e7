"""HF-model drop-ins for page isolation and the Page2D indexer RoPE.

Each function keeps the signature and return convention of the reference
function it replaces and runs the MI355X kernels on device tensors; host
tensors (and layouts the kernels do not take) go to the original function,
which ``srswa.patch`` passes in as ``orig``:

* ``build_kl_candidate_mask``  -- ``DeepseekV2Indexer._build_kl_candidate_mask``
  (HF/_sparse_base_impl.py:2706-2737, with ``_build_page_aware_image_block_mask``
  :2629-2649 and ``_build_image_block_allow_mask`` :2392-2402)
* ``rotary2d_forward``         -- ``DeepseekV2IndexerRotary2D.forward`` (HF/_sparse_base_impl.py:2046-2061)
* ``apply_rotary_pos_emb``     -- transformers' llama ``apply_rotary_pos_emb`` as the
  indexer imports it (HF/_sparse_base_impl.py:39-41, applied at :3049)
* ``uocr_dash_decode_allow``   -- ``_uocr_dash_decode_allow`` (HF/modeling_unlimitedocr.py:481-528)
* ``build_page_aware_ids``     -- ``DeepseekV2Indexer._build_page_aware_ids`` (HF/_sparse_base_impl.py:2404-2502)
* ``build_page_rope_pos``      -- ``DeepseekV2Indexer._build_page_rope_pos`` with ``_page_rope_offsets``
  (HF/_sparse_base_impl.py:2511-2570)

The two prompt-wide builders print a one-shot diagnostic in the reference;
their first call on a model goes to the original (which prints it and sets
the model's flag), every later call runs the kernels.
"""

from __future__ import annotations

import torch

from . import page_ops
from ._lib import UnsupportedShape


@torch.no_grad()
def build_kl_candidate_mask(self, pos_chunk, num_key_blocks, image_token_mask, batch, cq,
                            image_token_page_ids=None, query_token_page_ids=None):
    """[B, 1, cq, num_key_blocks] bool remote-candidate blocks per query:
    same-page image blocks (page-aware ids), all image blocks (flat image
    mask), or all blocks; a query with no candidate is open to every block."""
    device = pos_chunk.device
    nblk = int(num_key_blocks)
    bs = int(self.block_size)
    if self.image_bucket_constraint and image_token_page_ids is not None and query_token_page_ids is not None:
        ids = image_token_page_ids.to(device)
        bounds = page_ops.page_block_bounds(ids, nblk=nblk, block_size=bs)
        cand = page_ops.page_candidate_mask(bounds, ids, query_token_page_ids.to(device), pos_chunk,
                                            nblk=nblk, block_size=bs)
    elif image_token_mask is not None:
        # every image block: page 0 for image tokens, one query page 0 for all rows
        ids = torch.where(image_token_mask.to(device=device, dtype=torch.bool), 0, -1).to(torch.int32)
        bounds = page_ops.page_block_bounds(ids, nblk=nblk, block_size=bs)
        qpage = torch.zeros(batch, 1, dtype=torch.int32, device=device)
        pos = torch.zeros(batch, cq, dtype=torch.int32, device=device)
        cand = page_ops.page_candidate_mask(bounds, ids, qpage, pos, nblk=nblk, block_size=bs)
    else:
        return torch.ones(batch, 1, cq, nblk, dtype=torch.bool, device=device)
    return cand.unsqueeze(1)


@torch.no_grad()
def rotary2d_forward(self, x, tok_pos, page_pos):
    """tok_pos / page_pos [B, S] int -> cos / sin [B, S, dim] in x.dtype."""
    B, S = tok_pos.shape
    inv_tok = self.inv_tok.to(device=x.device, dtype=torch.float32)
    inv_page = self.inv_page.to(device=x.device, dtype=torch.float32)
    tok = tok_pos.to(x.device).reshape(-1)
    page = page_pos.to(x.device).reshape(-1)
    cos, sin = page_ops.page2d_cos_sin(tok, page, inv_tok, inv_page, dim=int(self.dim),
                                       page_mod=int(getattr(self, "page_mod", 0) or 0), dtype=x.dtype)
    return cos.view(B, S, -1), sin.view(B, S, -1)


def apply_rotary_pos_emb(q, k, cos, sin, position_ids=None, unsqueeze_dim=1, *, orig=None):
    """(q * cos + rotate_half(q) * sin, the same for k): q / k [B, H, S, hd],
    cos / sin [B, S, hd] broadcast over heads (``unsqueeze_dim`` = 1)."""
    del position_ids
    if q.is_cuda and unsqueeze_dim == 1 and cos.dim() == 3:
        try:
            return page_ops.rope_bhsd(q, k, cos, sin)
        except UnsupportedShape:
            pass
    if orig is None:
        raise UnsupportedShape("apply_rotary_pos_emb: layout not covered and no original to fall back to")
    return orig(q, k, cos, sin, unsqueeze_dim=unsqueeze_dim)


@torch.no_grad()
def uocr_dash_decode_allow(indexer, input_ids, cache):
    """Prefill (q_len > 1): records per KV block the [min, max] image page it
    holds, the prompt page count and the marker count; returns None.  Decode
    (q_len == 1): [B, nblk] bool candidate blocks of the query token's page
    (every block when its page is unknown or has no image block)."""
    img_id, pg_id = indexer.image_token_id, indexer.page_token_id
    if img_id is None or pg_id is None:
        return None
    bs = int(indexer.block_size)
    ids = input_ids
    B, L = ids.shape
    if L > 1:
        # per-token image page by the reference's scans, per-block bounds on the device
        img = ids == img_id
        cum = torch.cumsum((ids == pg_id).long(), dim=-1)
        run = torch.cumsum(img.long(), dim=-1)
        per_page = max(1, int(indexer.per_page_image_tokens))
        page = torch.where(cum > 0, cum - 1, (run - 1) // per_page)
        page = torch.where(img, page, torch.full_like(page, -1))
        pp = torch.where(img, cum, torch.zeros_like(cum)).cummax(dim=-1).values[:, -1]
        nblk = -(-L // bs)
        bounds = page_ops.page_block_bounds(page, nblk=nblk, block_size=bs)
        cache._uocr_pg = {"bounds": bounds, "bmin": bounds[..., 0], "bmax": bounds[..., 1], "pp": pp,
                          "mcum": cum[:, -1].clone()}
        return None
    st = getattr(cache, "_uocr_pg", None)
    if st is None:
        return None
    if "bounds" not in st:       # recorded by the original prefill branch
        st["bounds"] = torch.stack((st["bmin"], st["bmax"]), dim=-1).to(torch.int32).contiguous()
    st["mcum"] = st["mcum"] + (ids[:, -1] == pg_id).long()
    qp = st["mcum"] - 1 - st["pp"]
    qp = torch.where(qp >= 0, qp, torch.full_like(qp, -1))[:, None]
    total = int(cache.get_seq_length()) + L
    nblk = -(-total // bs)
    out = page_ops.page_candidate_mask(st["bounds"], None, qp, None, nblk=nblk, block_size=bs, range_test=True)
    return out[:, 0]


@torch.no_grad()
def build_page_aware_ids(self, source_input_ids, img_context_token_id, page_token_id, key_length, *,
                         page_scope_prefill=True):
    """(image_token_mask, image_token_page_ids, query_token_page_ids) [B,
    key_length], or (None, None, None) as the reference (nothing to
    constrain); one read-back of the per-row counts for that test, as the
    reference's own ``.sum() == 0`` checks."""
    if source_input_ids is None or img_context_token_id is None or page_token_id is None:
        return None, None, None
    if source_input_ids.ndim != 2:
        return None, None, None
    device = self.q_proj.weight.device
    if device.type != "cuda":
        raise UnsupportedShape("host model")
    img, ipage, qpage, counts = page_ops.page_aware_ids(
        source_input_ids, image_token_id=int(img_context_token_id), page_token_id=int(page_token_id),
        key_length=int(key_length), per_page=max(1, int(self.per_page_image_tokens)),
        page_scope_prefill=page_scope_prefill, device=device)
    nq, ni = (int(x) for x in counts.sum(0).tolist())
    if ni == 0 or nq == 0:
        return None, None, None
    return img, ipage, qpage


@torch.no_grad()
def build_page_rope_pos(self, source_input_ids, key_length):
    """(tok_pos, page_pos) [B, key_length] int64 for the 2-axis indexer RoPE,
    or the reference's bail (``self._page_rope_bail``) where it bails; sets
    ``self._page_rope_meta`` as ``_page_rope_offsets`` does."""
    if source_input_ids is None or getattr(source_input_ids, "ndim", 0) != 2:
        return self._page_rope_bail("no source_input_ids")
    if self.image_token_id is None or self.page_token_id is None:
        return self._page_rope_bail("image_token_id / page_token_id unavailable")
    device = self.q_proj.weight.device
    if device.type != "cuda":
        raise UnsupportedShape("host model")
    page, pre, info = page_ops.page_rope_pos(source_input_ids, image_token_id=int(self.image_token_id),
                                             page_token_id=int(self.page_token_id), key_length=int(key_length),
                                             device=device)
    inf = info.cpu()                                   # the reference's data-dependent checks
    if not bool(inf[:, 2].any()) or not bool(inf[:, 3].any()):
        return self._page_rope_bail("row has no image token / no <PAGE> marker")
    if not bool((inf[:, 0] > 0).all()):
        return self._page_rope_bail("non-marker mode (prompt carries no <PAGE>)")
    n_pg = int(inf[:, 1].max()) + 1
    tok, pf_cnt = page_ops.page_rope_tok(page, pre, n_pg)
    page = page.to(torch.int64)
    self._page_rope_meta = {"pf_cnt": pf_cnt, "n_pg": n_pg}
    if getattr(self, "rope_page_span", 0) > 0:
        # the span-normalisation ablation of _page_rope_offsets, on the kernel's counts
        in_prefill = pre.bool()
        pf_k = pf_cnt.gather(1, page)
        s_span = float(self.rope_page_span)
        scaled_pre = torch.round(tok.float() * s_span / pf_k.clamp(min=1).float())
        post = s_span + (tok - pf_k).float()
        scaled = torch.where(in_prefill, scaled_pre, post).to(torch.int64)
        tok = torch.where(page > 0, scaled, tok)
    return tok, page
