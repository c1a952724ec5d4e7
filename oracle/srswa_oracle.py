"""SR-SWA CPU oracle -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or, in bench.py,
as the timed CPU baseline).  The product path (``unlimited-ocr_amd/srswa``)
never imports it and raises when its HIP library is missing.

Each function restates, on the CPU in plain torch, the reference algorithm of
one function on the Sparse-Reference Sliding-Window Attention hot path and
cites the reference file:line it follows.  Citation prefixes:

* ``HF/x.py:N``  -> ``hf-model-code/x.py`` line N of the reference.
* ``WHL!p:N``    -> ``sglang/srt/p`` line N inside the reference's SGLang wheel.

Everything runs in the dtype of its inputs (pass float64 for the pinned checks,
float32 to mirror the reference's fp32 CPU path).  No function here ever calls
into the GPU library.

Pinning (what checks each function beyond restating it) lives in
``tests/test_oracle_pins.py``: brute-force set enumeration in pure Python,
textbook special cases (``F.scaled_dot_product_attention`` causal / banded),
closed forms, invariants and ``torch.autograd.gradcheck``.  Every public
function below has at least one such check; none is "parity unpinned".
"""

from __future__ import annotations

import math

import torch

# --- constants (HF/dash_attention.py:733-746; HF/sparse_gather_triton.py:32;
#     HF/sparse_gather_e2e_triton.py:33) -------------------------------------
SCORE_NEG = -1.0e9
MASK_NEG = -1.0e9
ACT_CLAMP = 1.0e4
ENTMAX_NEG = -1.0e4          # HF/modeling_deepseekv2.py:66
SPARSE_BLOCK_SIZE_SENTINEL = 128
SPARSE_E2E_SENTINEL = 1


def local_meta(block_size: int, local_window):
    """Window length in tokens and the number of physical blocks it can touch.

    HF/sparse_gather_triton.py:298-305 (``_local_meta``)."""
    lw = block_size if local_window is None else int(local_window)
    lw = max(1, lw)
    nlb = (lw + block_size - 1) // block_size + 1
    return lw, nlb


def dedup_slots(sel: torch.Tensor, valid: torch.Tensor | None = None) -> torch.Tensor:
    """Collapse repeated block ids of one row to a single slot (later repeats -> -1).

    HF/sparse_gather_triton.py:418-428 and HF/sparse_gather_e2e_triton.py:387-394
    dedup by sort+scatter; which of the equal slots survives is the (unstable)
    sort's choice there.  Here the FIRST slot holding an id survives, which is
    what the HIP kernels do.  Slots with ``valid == False`` or a negative id
    never count as a holder.
    """
    sel = sel.long()
    ok = sel >= 0
    if valid is not None:
        ok = ok & valid.bool()
    S = sel.shape[-1]
    same = sel[..., :, None] == sel[..., None, :]                  # [..., S, S]
    earlier = torch.ones(S, S, dtype=torch.bool).tril(diagonal=-1)  # j < i
    dup = (same & earlier & ok[..., None, :]).any(-1)
    return sel.masked_fill(dup | ~ok, -1)


def _slot_bitmap(sel: torch.Tensor, nblk: int) -> torch.Tensor:
    """[..., S] ids (-1 pad) -> [..., nblk] bool membership (ids >= nblk dropped).

    HF/_sparse_base_impl.py:3525-3529 (``build_block_mask`` bitmap)."""
    safe = sel.long().clamp(min=0)
    safe = safe.masked_fill((sel < 0) | (sel >= nblk), nblk)
    bm = torch.zeros(*sel.shape[:-1], nblk + 1, dtype=torch.bool)
    bm.scatter_(-1, safe, True)
    return bm[..., :nblk]


def _expand_heads(x: torch.Tensor, n_to: int) -> torch.Tensor:
    n_from = x.shape[1]
    if n_from == n_to:
        return x
    assert n_to % n_from == 0
    return x.repeat_interleave(n_to // n_from, dim=1)


# ---------------------------------------------------------------------------
# gather attention (prefill / training semantics)
# ---------------------------------------------------------------------------
def gather_keep_masks(block_indices, position_ids, key_length, block_size, local_window):
    """(keep, remote) [B, HI, T, Sk] bool for the fused gather attention.

    Query t sits at key index ``qi = Sk - T + t`` (T == Sk in the reference,
    the tail of a prefix cache otherwise); ``seg = qi - position_ids[t]`` is its
    sample start (HF/sparse_gather_triton.py:413-416).  With
    ``ls = max(qi - LW + 1, seg)``:

    * local  keys: ``ls <= j <= qi``                      (HF/sparse_gather_triton.py:95-111)
    * remote keys: ``j`` in a selected (deduped) block,
      ``seg <= j < ls`` and ``j <= qi``                   (HF/sparse_gather_triton.py:78-94)

    ``keep = local | remote`` equals ``build_block_mask``'s
    ``(block_keep | local_keep) & ~token_future`` (& same-segment when packed),
    HF/_sparse_base_impl.py:3518-3557.
    """
    B, HI, T, S = block_indices.shape
    Sk = int(key_length)
    lw, _ = local_meta(block_size, local_window)
    nblk = -(-Sk // block_size)
    sel = dedup_slots(block_indices)
    bitmap = _slot_bitmap(sel, nblk)                                 # [B,HI,T,nblk]
    j = torch.arange(Sk)
    selected = bitmap[..., j // block_size]                          # [B,HI,T,Sk]
    qi = (Sk - T) + torch.arange(T)
    seg = qi[None, :] - position_ids.long()                          # [B,T]
    qi_ = qi.view(1, 1, T, 1)
    seg_ = seg[:, None, :, None]
    ls = torch.maximum(qi_ - lw + 1, seg_)
    causal = j.view(1, 1, 1, Sk) <= qi_
    local = causal & (j >= ls)
    remote = selected & causal & (j < ls) & (j >= seg_)
    return local | remote, remote


def bias_slots_to_dense(bias_slots, block_indices, nblk):
    """[B,T,S] per-slot bias -> dense [B,T,nblk] keyed by block id (0 elsewhere).

    HF/sparse_gather_e2e_triton.py:396-400.  Duplicate / padding slots are
    dropped (the first slot holding an id wins, as in ``dedup_slots``).
    Differentiable w.r.t. ``bias_slots``."""
    sel = dedup_slots(block_indices)
    idx = sel.clamp(min=0).masked_fill((sel < 0) | (sel >= nblk), nblk)
    B, T, S = bias_slots.shape
    dense = bias_slots.new_zeros(B, T, nblk + 1).scatter(-1, idx, bias_slots)
    return dense[..., :nblk]


def gather_attention(q, k, v, block_indices, position_ids, block_size, scale,
                     local_window=None, blk_bias_dense=None):
    """Dense restatement of the fused gather attention forward.

    q [B,HQ,T,D]; k, v [B,Hkv,Sk,D] (Sk >= T); block_indices [B,HI,T,S]
    (-1 pad); position_ids [B,T]; optional ``blk_bias_dense`` [B,T,nblk] added
    to REMOTE logits only.  Returns (o [B,HQ,T,Dv], lse [B,HQ,T]); a row with
    no kept key gives o = 0 and lse = -inf.

    Follows HF/sparse_gather_triton.py:35-122 (K1) and, with bias,
    HF/sparse_gather_e2e_triton.py:36-121 (K5): logit = scale*q.k (+ bias on
    remote keys), one softmax over the disjoint union window | remote.  The
    eager equivalents are HF/_sparse_base_impl.py:1803-1836 and
    HF/dash_attention.py:1230-1260.
    """
    B, HQ, T, D = q.shape
    Sk = k.shape[2]
    HI = block_indices.shape[1]
    nblk = -(-Sk // block_size)
    keep, remote = gather_keep_masks(block_indices, position_ids, Sk, block_size, local_window)
    keep = _expand_heads(keep, HQ)
    remote = _expand_heads(remote, HQ)
    kk = _expand_heads(k, HQ)
    vv = _expand_heads(v, HQ)
    s = torch.matmul(q, kk.transpose(-1, -2)) * scale
    if blk_bias_dense is not None:
        kb = blk_bias_dense[:, None, :, torch.arange(Sk) // block_size]   # [B,1,T,Sk]
        s = s + torch.where(remote, kb.to(s.dtype), torch.zeros((), dtype=s.dtype))
    s = s.masked_fill(~keep, float("-inf"))
    m = s.amax(-1, keepdim=True).detach()
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    p = torch.exp(s - m)
    l = p.sum(-1, keepdim=True)
    o = torch.matmul(p, vv) / torch.where(l > 0, l, torch.ones_like(l))
    lse = (m + torch.log(l)).squeeze(-1)
    _ = HI
    return o, lse


def gather_attention_e2e(q, k, v, block_indices, blk_bias_slots, position_ids,
                         block_size, scale, local_window=None):
    """Restatement of ``triton_gather_attention_e2e`` (HF/sparse_gather_e2e_triton.py:355-407):
    per-slot bias [B,T,S] scattered to blocks, added to remote logits; single index head."""
    Sk = k.shape[2]
    nblk = -(-Sk // block_size)
    dense = bias_slots_to_dense(blk_bias_slots, block_indices[:, 0], nblk)
    o, _ = gather_attention(q, k, v, block_indices, position_ids, block_size, scale,
                            local_window, blk_bias_dense=dense)
    return o


def build_block_mask(block_indices, key_length, block_size, local_window, position_ids,
                     num_heads):
    """``DeepseekV2Indexer.build_block_mask`` (HF/_sparse_base_impl.py:3518-3557)
    without an attention mask: bool keep [B, num_heads, T, key_length]."""
    keep, _ = gather_keep_masks(block_indices, position_ids, key_length, block_size,
                                local_window)
    return _expand_heads(keep, num_heads)


# ---------------------------------------------------------------------------
# decode attention
# ---------------------------------------------------------------------------
def decode_attend(q, k_all, v_all, topi, bias, valid, q_pos, block_size, local_window, scale):
    """Bias-aware block-sparse decode attention in fp32 (or the input's wider dtype).

    Restates ``_decode_attend`` (HF/modeling_deepseekv2.py:454-481) with the
    index head made explicit: ``topi``/``bias``/``valid`` may be [B,Lq,K] (one
    index head shared by all heads, as in the reference) or [B,HI,Lq,K].

    Remote keys of a selected valid block get its bias; the token-level window
    ``(q_pos - local_window, q_pos]`` gets bias 0 and wins on overlap; keys after
    ``q_pos`` are dropped.  Duplicate valid ids: the first slot's bias is used
    (the reference's scatter leaves the winner unspecified).
    q [B,H,Lq,D]; k_all, v_all [B,Hkv,S,D]; q_pos [B,Lq].  Returns [B,H,Lq,Dv].
    """
    B, H, Lq, D = q.shape
    S = k_all.shape[2]
    dt = torch.promote_types(q.dtype, torch.float32)
    if topi.dim() == 3:
        topi, bias, valid = topi[:, None], bias[:, None], valid[:, None]
    HI = topi.shape[1]
    nblk = (S + block_size - 1) // block_size
    kpos = torch.arange(S)
    sel = dedup_slots(topi, valid)                                   # [B,HI,Lq,K]
    src = torch.where(sel >= 0, bias.to(dt), torch.full((), MASK_NEG, dtype=dt))
    idx = sel.clamp(min=0).masked_fill(sel < 0, nblk)
    blk = torch.full((B, HI, Lq, nblk + 1), MASK_NEG, dtype=dt)
    blk = blk.scatter(-1, idx, src)[..., :nblk]
    base = blk.index_select(-1, kpos // block_size)                  # [B,HI,Lq,S]
    qp = q_pos.long()[:, None, :, None]
    causal = kpos.view(1, 1, 1, S) <= qp
    local = causal & (kpos > (qp - local_window))
    keep = causal & (local | (base > MASK_NEG * 0.5))
    m = torch.where(local, torch.zeros_like(base), base).masked_fill(~keep, float("-inf"))
    m = _expand_heads(m, H)
    kk = _expand_heads(k_all.to(dt), H)
    vv = _expand_heads(v_all.to(dt), H)
    s = torch.matmul(q.to(dt), kk.transpose(-1, -2)) * scale + m
    return torch.matmul(torch.softmax(s, dim=-1), vv)


def paged_decode_attend(q, k_cache, v_cache, topk, bias, block_table, seq_lens, dql, local_blocks, scale):
    """The serving decode over a paged cache: ``dash_sparse_attn_decode``
    (WHL!layers/attention/unlimited_dash_ops/attend_triton.py:307-518, 600-715).

    q [R*dql, H, D]; k_cache, v_cache [num_pages, page, Hkv, D] (one page per
    block); topk / bias [Hkv, R*dql, K] (per kv head; -1 = empty); block_table
    [R, max_blocks]; seq_lens [R].  Query i of request r sits at
    ``seq_lens[r] - dql + i``; window = the last ``local_blocks * page`` keys up
    to it, unbiased; remote = keys of the listed blocks below the window.  The
    same attention as ``decode_attend`` on the request's cache gathered page by
    page (a repeated id counts once, as there).  Returns [R*dql, H, D]."""
    R = block_table.shape[0]
    page = k_cache.shape[1]
    Hkv, H, D = k_cache.shape[2], q.shape[1], q.shape[2]
    nb = block_table.shape[1]
    out = []
    for r in range(R):
        pages = block_table[r].long()
        kr = k_cache[pages].reshape(nb * page, Hkv, D).transpose(0, 1)[None]       # [1,Hkv,S,D]
        vr = v_cache[pages].reshape(nb * page, Hkv, v_cache.shape[-1]).transpose(0, 1)[None]
        L = int(seq_lens[r])
        kr, vr = kr[:, :, :L], vr[:, :, :L]
        rows = slice(r * dql, (r + 1) * dql)
        qr = q[rows].transpose(0, 1)[None]                                           # [1,H,dql,D]
        ti = topk[:, rows].long()[None]                                              # [1,Hkv,dql,K]
        ti = ti.masked_fill(ti >= -(-L // page), -1)     # blocks past seq_len hold no key (pos < kv_len)
        bi = bias[:, rows][None] if bias is not None else torch.zeros(ti.shape, dtype=torch.float64)
        valid = ti >= 0
        q_pos = (L - dql + torch.arange(dql))[None]
        o = decode_attend(qr, kr, vr, ti, bi, valid, q_pos, page, local_blocks * page, scale)
        # a row with no key at all (no window, nothing selected) is 0, not NaN:
        # attend_triton.py:495-497 scales by 0 when its lse stays -inf
        o = torch.nan_to_num(o, nan=0.0)
        out.append(o[0].transpose(0, 1))                                             # [dql,H,D]
    return torch.cat(out, 0)


def paged_prefill_attend(q, k_cache, v_cache, topk, bias, block_table, cu_seqlens_q, seq_lens, prefix_lens,
                         local_blocks, scale):
    """The serving prefill over a paged cache: ``dash_sparse_attn`` /
    ``_dash_sparse_fwd_kernel`` (K10, WHL!layers/attention/unlimited_dash_ops/
    attend_triton.py:76-292, 521-597), query by query in its two passes.

    q [total_q, H, D]; k_cache, v_cache [num_pages, page, Hkv, D]; topk / bias
    [Hkv, total_q, K] (bias None = 0); block_table [R, max_blocks]; request r
    owns query rows cu_seqlens_q[r] .. cu_seqlens_q[r + 1), row t at position
    qp = prefix_lens[r] + t.  Per query head (kv head h // (H / Hkv)):
      remote pass: the first count(id >= 0) slots, in slot order (:162-177),
        keys c + n of each slot's block with c + n <= qp - LB * page and
        c + n < seq_lens[r] (:183-211), logit scale * q.k + bias[slot];
      window pass (LB > 0): blocks qp // page - o, o = 0 .. LB, keys in
        [qp - LB * page + 1, qp] below seq_lens[r] (:231-263), logit scale * q.k.
    One softmax over everything; returns [total_q, H, Dv] in fp64 (or the
    promoted input dtype).  A row with no key at all is 0 here (the reference's
    final acc * exp2(m - lse) is NaN there: -inf - -inf); with a window it
    always holds its own key."""
    page = k_cache.shape[1]
    Hkv, H = k_cache.shape[2], q.shape[1]
    G = H // Hkv
    LW = int(local_blocks) * page
    dt = torch.promote_types(q.dtype, torch.float32)
    out = torch.zeros(q.shape[0], H, v_cache.shape[-1], dtype=dt)
    for r in range(block_table.shape[0]):
        sl, pre = int(seq_lens[r]), int(prefix_lens[r])
        pages = block_table[r].long()
        for n in range(int(cu_seqlens_q[r]), int(cu_seqlens_q[r + 1])):
            qp = pre + n - int(cu_seqlens_q[r])
            for h in range(H):
                kh = h // G
                ids = topk[kh, n].tolist()
                real = sum(1 for i in ids if i >= 0)
                keys, bvals = [], []
                for si in range(real):
                    c = ids[si] * page
                    kk = [j for j in range(c, c + page) if j <= qp - LW and j < sl]
                    keys += kk
                    bvals += [0.0 if bias is None else float(bias[kh, n, si])] * len(kk)
                if local_blocks > 0:
                    kk = [j for j in range(max(qp - LW + 1, 0), qp + 1) if j < sl]
                    keys += kk
                    bvals += [0.0] * len(kk)
                if not keys:
                    continue
                kt = torch.tensor(keys)
                kv = k_cache[pages[kt // page], kt % page, kh].to(dt)
                vv = v_cache[pages[kt // page], kt % page, kh].to(dt)
                s = (kv @ q[n, h].to(dt)) * scale + torch.tensor(bvals, dtype=dt)
                out[n, h] = torch.softmax(s, 0) @ vv
    return out


def decode_attend_gather(q, k_cache, v_cache, block_idx, q_pos, block_size, local_window,
                         scale, bias=None):
    """Gather-form decode for caches too large for the dense form.

    q [B,H,D]; k_cache, v_cache [B,L,H,D] (the BASELINE's contiguous layout);
    block_idx [B,H,K] per-head selected blocks (-1 pad); q_pos [B].  Reads only
    the window keys ``(q_pos-LW, q_pos]`` and the remote keys of the selected
    blocks, then the same softmax as ``decode_attend`` (identical read set /
    weights, HF/modeling_deepseekv2.py:454-481).  Returns [B,H,Dv] in the
    promoted fp32/fp64 dtype.
    """
    B, H, D = q.shape
    dt = torch.promote_types(q.dtype, torch.float32)
    out = torch.empty(B, H, v_cache.shape[-1], dtype=dt)
    for b in range(B):
        qp = int(q_pos[b])
        ws = max(qp - int(local_window) + 1, 0)
        for h in range(H):
            ids = dedup_slots(block_idx[b, h][None])[0].tolist()
            keys, bvals = [], []
            for si, bid in enumerate(ids):
                if bid < 0:
                    continue
                lo, hi = bid * block_size, min((bid + 1) * block_size, ws, qp + 1)
                if hi > lo:
                    keys.append(torch.arange(lo, hi))
                    bv = 0.0 if bias is None else float(bias[b, h, si])
                    bvals.append(torch.full((hi - lo,), bv, dtype=dt))
            keys.append(torch.arange(ws, qp + 1))
            bvals.append(torch.zeros(qp + 1 - ws, dtype=dt))
            kp = torch.cat(keys)
            kb = k_cache[b, kp, h].to(dt)
            vb = v_cache[b, kp, h].to(dt)
            s = (kb @ q[b, h].to(dt)) * scale + torch.cat(bvals)
            out[b, h] = torch.softmax(s, 0) @ vb
    return out


# ---------------------------------------------------------------------------
# indexer: block scoring and top-k
# ---------------------------------------------------------------------------
def meanpool_block_scores(q, k, q_pos, block_size, local_blocks, head_cls=None):
    """head_cls / mean-pool remote block scores, per index head.

    q [B,HI,Lq,d]; k [B,HI,S,d] (S = cached keys); q_pos [B,Lq] absolute
    positions.  Returns [B,HI,Lq,nblk] with ``SCORE_NEG`` on non-remote blocks.

    Restates ``_block_scores_infer`` stage0 == "head_cls"
    (HF/modeling_deepseekv2.py:391-417; same math as
    HF/dash_attention.py:1053-1143 and WHL!layers/attention/unlimited_dash_ops/dash_stage0.py:25-58):
    ``w = softmax_valid(clamp(k.hc/sqrt d))`` (hc = 0 -> mean of the block's real
    keys), ``k_bar = sum w k``, ``z = clamp(q.k_bar/sqrt d, +-1e4)``, remote iff
    ``blk <= q_pos // BS - local_blocks`` and the block holds a real key.
    """
    B, HI, S, d = k.shape
    bs = int(block_size)
    nblk = -(-S // bs)
    Sp = nblk * bs
    inv_sqrt_d = 1.0 / math.sqrt(d)
    kk = torch.nn.functional.pad(k, (0, 0, 0, Sp - S))
    real = torch.nn.functional.pad(torch.ones(B, HI, S, dtype=torch.bool), (0, Sp - S), value=False)
    kk = kk.view(B, HI, nblk, bs, d)
    vmask = real.view(B, HI, nblk, bs)
    hc = torch.zeros(d, dtype=kk.dtype) if head_cls is None else head_cls.to(kk.dtype)
    aw = ((kk * hc.view(1, 1, 1, 1, d)).sum(-1) * inv_sqrt_d).clamp(-ACT_CLAMP, ACT_CLAMP)
    neg = torch.finfo(aw.dtype).min
    row_max = torch.where(vmask, aw, torch.full((), neg, dtype=aw.dtype)).amax(-1, keepdim=True)
    row_max = torch.where(vmask.any(-1, keepdim=True), row_max, torch.zeros_like(row_max))
    e = torch.exp(aw - row_max) * vmask.to(aw.dtype)
    w = e / e.sum(-1, keepdim=True).clamp_min(1e-6)
    k_bar = torch.nan_to_num((w.unsqueeze(-1) * kk).sum(dim=3), nan=0.0, posinf=0.0, neginf=0.0)
    chunk_valid = vmask.any(-1)                                      # [B,HI,nblk]
    z = torch.matmul(q.to(k_bar.dtype), k_bar.transpose(-1, -2)) * inv_sqrt_d
    z = z.clamp(-ACT_CLAMP, ACT_CLAMP)
    qblk = q_pos.long()[:, None, :, None] // bs
    blk = torch.arange(nblk).view(1, 1, 1, nblk)
    keep = (blk <= qblk - int(local_blocks)) & chunk_valid[:, :, None, :]
    return z.masked_fill(~keep, SCORE_NEG)


def kbar_summaries(keys, valid, head_cls=None):
    """``_summary_keys`` (WHL!layers/attention/unlimited_dash_ops/dash_stage0.py:25-43):
    [nb, bs, d] keys, [nb, bs] real-key mask -> [nb, d] head_cls softmax-weighted
    means (the plain mean when head_cls is None); a block without keys -> 0."""
    d = keys.shape[-1]
    inv_sqrt_d = 1.0 / math.sqrt(d)
    hc = torch.zeros(d, dtype=keys.dtype) if head_cls is None else head_cls.to(keys.dtype)
    aw = ((keys * hc).sum(-1) * inv_sqrt_d).clamp(-ACT_CLAMP, ACT_CLAMP)
    neg = torch.finfo(aw.dtype).min
    row_max = torch.where(valid, aw, torch.full((), neg, dtype=aw.dtype)).amax(-1, keepdim=True)
    row_max = torch.where(valid.any(-1, keepdim=True), row_max, torch.zeros_like(row_max))
    e = torch.exp(aw - row_max) * valid.to(aw.dtype)
    w = e / e.sum(-1, keepdim=True).clamp_min(1e-6)
    return torch.nan_to_num((w.unsqueeze(-1) * keys).sum(1), nan=0.0, posinf=0.0, neginf=0.0)


def kbar_pages(keys_cache, head_cls, block_table, seq_lens, kbar, tail_blocks=0):
    """``KBarCache.put`` for every used page (headcls_scores_prefill,
    dash_stage0.py:62-103) or ``refresh_tail`` (:123-148, tail_blocks > 0):
    kbar[block_table[r, b]] = summary of the block's real keys for the
    request's blocks b < ceil(seq_len / page) (only the last tail_blocks).
    keys_cache [num_pages, page, d]; returns the updated copy of kbar."""
    kbar = kbar.clone()
    page = keys_cache.shape[1]
    for r in range(block_table.shape[0]):
        sl = int(seq_lens[r])
        nb = min(-(-sl // page), block_table.shape[1])
        blks = range(max(nb - tail_blocks, 0), nb) if tail_blocks > 0 else range(nb)
        for b in blks:
            pg = int(block_table[r, b])
            valid = (torch.arange(page) < sl - b * page)[None]
            kbar[pg] = kbar_summaries(keys_cache[pg][None].to(kbar.dtype), valid, head_cls)[0]
    return kbar


def kbar_scores(q, kbar, block_table, seq_lens, width, page, local_blocks, dql=None, row_req=None,
                row_pos=None):
    """``headcls_scores_decode`` (dash_stage0.py:151-199; prefill rows as
    ``_score_rows``, :45-58) off the summary cache: row n of request r at
    position pos scores block b as clamp(q . kbar[block_table[r, b]] / sqrt d,
    +-1e4) when b <= pos // page - local_blocks and b * page < seq_lens[r], else
    SCORE_NEG.  Decode rows (row_req / row_pos None): r = n // dql, pos =
    seq_lens[r] - dql + n % dql.  Returns [nrows, width]."""
    n_rows, d = q.shape
    out = torch.full((n_rows, width), SCORE_NEG, dtype=kbar.dtype)
    for n in range(n_rows):
        r = int(row_req[n]) if row_req is not None else n // dql
        sl = int(seq_lens[r])
        pos = int(row_pos[n]) if row_pos is not None else sl - dql + n % dql
        if pos < 0:
            continue
        for b in range(min(width, block_table.shape[1])):
            if b <= pos // page - local_blocks and b * page < sl:
                z = (q[n].to(kbar.dtype) @ kbar[int(block_table[r, b])]) / math.sqrt(d)
                out[n, b] = z.clamp(-ACT_CLAMP, ACT_CLAMP)
    return out


def block_max_scores(q, k, pos, seg, block_size, num_key_blocks, local_window=None):
    """Fused indexer block-max score: ``max_{j in blk, seg <= j < local_start} q.k_j``.

    q [B,C,D]; k [B,Sk,D]; pos, seg [B,C]; unscaled; -inf where a block has no
    valid key.  ``local_start = max(pos - LW + 1, 0)``.  Restates
    ``triton_block_max_score`` (HF/sparse_gather_triton.py:445-524), which
    matches the eager ``token_future | local_token`` masking of
    ``DeepseekV2Indexer.forward`` (HF/_sparse_base_impl.py:3076-3094).
    """
    B, C, D = q.shape
    Sk = k.shape[1]
    bs = int(block_size)
    nblk = int(num_key_blocks)
    lw = bs if local_window is None else max(1, int(local_window))
    s = torch.matmul(q, k.transpose(-1, -2))                          # [B,C,Sk]
    j = torch.arange(Sk).view(1, 1, Sk)
    ls = (pos.long() - (lw - 1)).clamp(min=0)[:, :, None]
    valid = (j < ls) & (j >= seg.long()[:, :, None])
    s = s.masked_fill(~valid, float("-inf"))
    width = nblk * bs
    if width > Sk:
        s = torch.nn.functional.pad(s, (0, width - Sk), value=float("-inf"))
    else:
        s = s[..., :width]
    return s.view(B, C, nblk, bs).amax(-1)


def indexer_forward_ids(idx_q, idx_k, position_ids, block_size, local_window, topk, chunk=0, img_blk=None):
    """``DeepseekV2Indexer.forward`` (HF/_sparse_base_impl.py:3065-3105) from its
    projections: idx_q [B, HI, T, d], idx_k [B, 1, Sk, d], position_ids [B, T];
    per chunk the q . k scores with future and local-window keys at -inf,
    padded to whole blocks, block amax; blocks outside ``img_blk`` [B, nblk]
    (bool, or None) at -inf; then the top-k (ties -> lower id), -1 where -inf.
    int64 [B, HI, T, topk]."""
    B, HI, T, _ = idx_q.shape
    Sk = idx_k.shape[2]
    nblk = -(-Sk // block_size)
    kpos = torch.arange(Sk)
    step = chunk if chunk and chunk > 0 else T
    out = []
    for c0 in range(0, T, step):
        c1 = min(c0 + step, T)
        sc = torch.matmul(idx_q[:, :, c0:c1], idx_k.transpose(-1, -2))
        pos = position_ids[:, c0:c1].long()
        future = kpos[None, None, None, :] > pos[:, None, :, None]
        start = (pos - (local_window - 1)).clamp(min=0)
        local = (kpos[None, None, None, :] >= start[:, None, :, None]) & (kpos[None, None, None, :] <= pos[:, None, :, None])
        sc = sc.masked_fill(future | local, float("-inf"))
        pad = nblk * block_size - Sk
        if pad:
            sc = torch.nn.functional.pad(sc, (0, pad), value=float("-inf"))
        out.append(sc.view(B, HI, c1 - c0, nblk, block_size).amax(-1))
    bsc = torch.cat(out, dim=2)
    if img_blk is not None:
        bsc = bsc.masked_fill(~img_blk[:, None, None, :], float("-inf"))
    if topk == 0:
        return torch.empty(B, HI, T, 0, dtype=torch.long)
    return topk_blocks(bsc, topk, invalid_at=float("-inf")), bsc


def indexer_infer_block_scores(idx_q, idx_k, q_pos, nblk, block_size, local_window, q_chunk=2048):
    """The stage0 == "indexer" branch of ``_block_scores_infer``
    (HF/modeling_deepseekv2.py:419-430): idx_q [B, Lq, d], idx_k [B, S, d],
    q_pos [B, Lq]; q . k clamped to +-ACT_CLAMP, future keys and keys
    j > pos - local_window at SCORE_NEG, padded with SCORE_NEG to nblk blocks,
    block amax.  [B, Lq, nblk]."""
    B, S, _ = idx_k.shape
    kpos = torch.arange(S)
    out = []
    for c0 in range(0, idx_q.shape[1], q_chunk):
        c1 = min(c0 + q_chunk, idx_q.shape[1])
        sc = torch.matmul(idx_q[:, c0:c1], idx_k.transpose(-1, -2)).clamp(-ACT_CLAMP, ACT_CLAMP)
        pos = q_pos[:, c0:c1].long()
        future = kpos[None, None, :] > pos[:, :, None]
        local = (kpos[None, None, :] > (pos[:, :, None] - local_window)) & ~future
        sc = sc.masked_fill(future | local, SCORE_NEG)
        if nblk * block_size > S:
            sc = torch.nn.functional.pad(sc, (0, nblk * block_size - S), value=SCORE_NEG)
        out.append(sc.view(B, c1 - c0, nblk, block_size).amax(-1))
    return torch.cat(out, dim=1)


def topk_blocks(scores, k, invalid_at=SCORE_NEG * 0.5):
    """k best blocks per row: descending score, ties -> lower block id.

    Restates ``block_scores.topk(k)`` + ``masked_fill(score == -inf, -1)``
    (HF/_sparse_base_impl.py:3100-3105) and the top-K of
    ``_infer_route_select`` (HF/modeling_deepseekv2.py:346-355) with the tie
    order fixed.  Slots past the number of valid entries (score > invalid_at;
    -inf, NaN and sentinels are invalid) are -1.  Returns int64 [..., k].
    """
    n = scores.shape[-1]
    kk = min(int(k), n)
    s = scores.double()
    s = torch.where(torch.isnan(s), torch.full((), float("-inf"), dtype=s.dtype), s)   # +-inf kept as they are
    order = torch.sort(-s, dim=-1, stable=True).indices[..., :kk]
    top = s.gather(-1, order)
    out = order.masked_fill(~(top > invalid_at), -1)
    if kk < k:
        pad = torch.full((*out.shape[:-1], k - kk), -1, dtype=out.dtype)
        out = torch.cat([out, pad], -1)
    return out


def near_tie_rows(scores, k, rel=1e-4, invalid_at=SCORE_NEG * 0.5, floor=1.0):
    """bool [...]: rows whose k-th and (k+1)-th best valid scores differ by less
    than ``rel * max(floor, |s_k|)`` -- there the selected SET is not determined by
    fp32 summation order and bit-exact comparison is reported separately.
    ``floor`` = 1 for scores of order one and above; 0 makes the gap purely
    relative (scores far below one, e.g. config 1's 1/sqrt(D)-scaled inputs)."""
    s = scores.double()
    s = torch.where(torch.isnan(s), torch.full((), float("-inf"), dtype=s.dtype), s)   # +-inf kept as they are
    s = torch.where(s > invalid_at, s, torch.full((), float("-inf"), dtype=s.dtype))
    n = s.shape[-1]
    if k >= n:
        return torch.zeros(s.shape[:-1], dtype=torch.bool)
    top = torch.sort(s, dim=-1, descending=True).values
    sk, sk1 = top[..., k - 1], top[..., k]
    fin = torch.isfinite(sk) & torch.isfinite(sk1)
    return fin & ((sk - sk1).abs() < rel * torch.clamp(sk.abs(), min=float(floor)))


# ---------------------------------------------------------------------------
# DASH router (entmax-1.5 prior -> hard top-K -> centred log-prior bias)
# ---------------------------------------------------------------------------
def entmax15(x, dim=-1):
    """1.5-entmax by the sort-based exact threshold (Peters, Niculae & Martins 2019).

    HF/dash_attention.py:764-814 (``_entmax_threshold_and_support`` + forward)."""
    x = x.transpose(dim, -1)
    x = (x - x.amax(-1, keepdim=True)) / 2
    xs = torch.sort(x, dim=-1, descending=True).values
    n = x.shape[-1]
    rho = torch.arange(1, n + 1, dtype=x.dtype)
    mean = xs.cumsum(-1) / rho
    mean_sq = (xs ** 2).cumsum(-1) / rho
    ss = rho * (mean_sq - mean ** 2)
    delta = (1 - ss) / rho
    tau = mean - torch.sqrt(torch.clamp(delta, min=0))
    support = (tau <= xs).sum(-1, keepdim=True).clamp(min=1)
    tau_star = tau.gather(-1, support - 1)
    y = torch.clamp(x - tau_star, min=0) ** 2
    return y.transpose(dim, -1)


class Entmax15Ref(torch.autograd.Function):
    """``entmax15`` with the reference's own backward (``_Entmax15.backward``,
    HF/dash_attention.py:797-806): g = sqrt(y), dx = dy g - g sum(dy g) / sum(g)."""

    @staticmethod
    def forward(ctx, x, dim):
        y = entmax15(x, dim)
        ctx.dim = dim
        ctx.save_for_backward(y)
        return y

    @staticmethod
    def backward(ctx, dy):
        (y,) = ctx.saved_tensors
        g = y.sqrt()
        dx = dy * g
        q = (dx.sum(ctx.dim) / g.sum(ctx.dim).clamp_min(1e-12)).unsqueeze(ctx.dim)
        return dx - q * g, None


def dash_route_train(block_scores, image_block_mask, block_cand, idx_scale, neg=ENTMAX_NEG, image_only=True):
    """``DashAttention._route`` (HF/dash_attention.py:1145-1174) without its
    calibration hook: (prior [B, S, nblk], cand bool); differentiable in
    block_scores."""
    remote = block_scores > (SCORE_NEG * 0.5)
    cand = remote
    if block_cand is not None:
        cand = remote & block_cand
    elif image_only and image_block_mask is not None:
        cand = remote & image_block_mask[:, None, :]
    cand = torch.where(~cand.any(dim=-1, keepdim=True), remote, cand)
    x = torch.where(cand, block_scores * idx_scale, block_scores.new_full((), neg))
    x = torch.nan_to_num(x, nan=neg, posinf=neg, neginf=neg)
    return Entmax15Ref.apply(x, -1), cand


def dash_select_and_bias(prior, cand, K, floor, sigma):
    """``DashAttention._select_and_bias`` (HF/dash_attention.py:1176-1204):
    the K largest of the masked prior (non-candidates -1; ties -> lower block
    id), valid = a candidate slot, bias = (log(max(p, floor)) - mean over the
    valid slots) / sigma, 0 elsewhere, clamped to +-1e4.  (topi, bias, valid);
    bias differentiable in prior."""
    sel = prior.masked_fill(~cand, -1.0)
    topi = torch.sort(-sel.detach(), dim=-1, stable=True).indices[..., :K]
    bias, valid = dash_bias_given(prior, cand, topi, floor, sigma)
    return topi, bias, valid


def dash_bias_given(prior, cand, topi, floor, sigma):
    """The bias / valid of ``_select_and_bias`` (HF/dash_attention.py:1196-1203)
    for given slot ids: topv = the masked prior at topi.  (bias, valid)."""
    sel = prior.masked_fill(~cand, -1.0)
    topv = sel.gather(-1, topi)
    valid = topv >= 0.0
    logp = torch.log(topv.clamp_min(floor))
    cnt = valid.sum(dim=-1, keepdim=True).clamp(min=1)
    mu = torch.where(valid, logp, torch.zeros_like(logp)).sum(dim=-1, keepdim=True) / cnt
    bias = (logp - mu) * (1.0 / sigma)
    bias = torch.where(valid, bias, torch.zeros_like(bias)).clamp(-ACT_CLAMP, ACT_CLAMP)
    return bias, valid


def infer_route_select(block_scores, block_cand, idx_scale, floor, sigma, K, topm):
    """``_infer_route_select`` (HF/modeling_deepseekv2.py:338-362): top-M window,
    entmax-1.5 prior, first K slots, centred log-prior bias.  Top-M ties -> lower id."""
    remote = block_scores > (SCORE_NEG * 0.5)
    cand = remote if block_cand is None else (remote & block_cand)
    cand = torch.where(~cand.any(-1, keepdim=True), remote, cand)
    x = torch.where(cand, block_scores * idx_scale, torch.full((), ENTMAX_NEG, dtype=block_scores.dtype))
    x = torch.nan_to_num(x, nan=ENTMAX_NEG, posinf=ENTMAX_NEG, neginf=ENTMAX_NEG)
    nblk = x.shape[-1]
    M = max(1, min(int(topm), nblk)) if int(topm) > 0 else nblk
    xi = torch.sort(-x.double(), dim=-1, stable=True).indices[..., :M]
    xv = x.gather(-1, xi)
    prior = entmax15(xv, dim=-1)
    is_cand = cand.gather(-1, xi)
    Kc = max(1, min(int(K), M))
    xi, prior, valid = xi[..., :Kc], prior[..., :Kc], is_cand[..., :Kc]
    logp = torch.log(prior.clamp_min(floor))
    cnt = valid.sum(-1, keepdim=True).clamp(min=1)
    mu = torch.where(valid, logp, torch.zeros_like(logp)).sum(-1, keepdim=True) / cnt
    bias = torch.where(valid, (logp - mu) * (1.0 / sigma), torch.zeros_like(logp))
    return xi, bias.float(), valid
