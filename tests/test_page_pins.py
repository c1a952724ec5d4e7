"""Pins of the page-isolation / Page2D RoPE oracle (oracle/page_oracle.py).

Each check compares the oracle against a different formulation of the same
reference semantics: whole-sequence scans (cumsum / cummax) against the
token-by-token state machine, brute-force set membership against the min/max
block test, transformers' llama rotary evaluated by torch against the numpy
rounding schedule, and identities of the cos / sin table."""

import math

import numpy as np
import pytest
import torch

from oracle import page_oracle as P

IMG, PG = 128815, 128816


def _document(rng, pages, with_markers=True, placeholder=False, img_tokens=(20, 40), text=(3, 9)):
    """A prompt of `pages` image pages (optionally each led by a <PAGE>
    marker), an instruction, then a response with one <PAGE> per page."""
    toks = [0]
    for _ in range(pages):
        if with_markers:
            toks.append(PG)
        n = int(rng.integers(*img_tokens))
        toks += [P.MM_PAD_SHIFT + 7 if placeholder else IMG] * n
    toks += list(rng.integers(10, 1000, size=int(rng.integers(*text))))
    for _ in range(pages + 1):                      # one extra marker past the last page
        toks.append(PG)
        toks += list(rng.integers(10, 1000, size=int(rng.integers(*text))))
    return np.array(toks, np.int64)


def _scan_expectation(ids, per_page, marker_id=PG, max_pages=64):
    """Whole-sequence restatement with scans: PageIsolationState.step
    (WHL!…/page_state.py:232-282, every token generated) and the decode
    coordinates of PageCoordState.step (WHL!…/page2d_rope.py:559-604)."""
    is_img = (ids >= P.MM_PAD_SHIFT) | (ids == IMG)
    is_mark = ids == marker_id if marker_id is not None else np.zeros_like(is_img)
    marker = np.cumsum(is_mark).astype(np.int64)
    run = np.cumsum(is_img).astype(np.int64)
    img_page = np.where(marker > 0, marker - 1, (run - 1) // per_page)
    img_page = np.where(is_img, img_page, -1)
    pp = np.maximum.accumulate(np.where(is_img, marker, 0))
    resp = marker - 1 - pp
    q_page = np.where(is_img, img_page, np.where(resp >= 0, resp, -1))
    cpage = np.clip(np.minimum(np.maximum(marker - pp, 0), pp), 0, max_pages - 1)
    tok = np.array([int(np.sum(cpage[:t] == cpage[t])) for t in range(len(ids))])   # earlier tokens, same page
    return dict(img_page=img_page, marker=marker, run=run, pp=pp, q_page=q_page, cpage=cpage, tok=tok)


@pytest.mark.parametrize("variant", ["markers", "per_page", "placeholder", "no_marker_id"])
def test_decode_meta_stepwise_equals_scans(variant):
    rng = np.random.default_rng({"markers": 1, "per_page": 2, "placeholder": 3, "no_marker_id": 4}[variant])
    bs, per_page, max_pages = 16, 24, 64
    marker_id = None if variant == "no_marker_id" else PG
    docs = [_document(rng, int(rng.integers(1, 5)), with_markers=variant != "per_page",
                      placeholder=variant == "placeholder") for _ in range(3)]
    T = max(len(d) for d in docs)
    docs = [np.concatenate([d, rng.integers(10, 1000, size=T - len(d))]) for d in docs]   # equal length
    R = len(docs)
    nblk = -(-T // bs)
    perm = rng.permutation(R * nblk + 5)
    bt = perm[:R * nblk].reshape(R, nblk).astype(np.int64)
    n_slots = (R * nblk + 5) * bs
    st = P.SlotState(n_slots)
    st.img_page[:] = 7                        # stale pages from an earlier request
    cs = P.CoordState(R + 1, max_pages)
    coord_row = np.arange(R) + 1              # row 0 unused
    q_seen = np.zeros((R, T), np.int32)
    tok_seen = np.zeros((R, T), np.int64)
    page_seen = np.zeros((R, T), np.int64)
    for t in range(T):
        ids = np.array([d[t] for d in docs])
        seq = np.full(R, t + 1)
        slot = bt[np.arange(R), t // bs] * bs + t % bs
        q, tok, page = P.decode_meta_step(ids, bt, seq, slot, coord_row, st, cs, IMG, marker_id, per_page, bs)
        q_seen[:, t], tok_seen[:, t], page_seen[:, t] = q, tok, page
    for r in range(R):
        ex = _scan_expectation(docs[r], per_page, marker_id, max_pages)
        np.testing.assert_array_equal(q_seen[r], ex["q_page"])
        np.testing.assert_array_equal(page_seen[r], ex["cpage"])
        np.testing.assert_array_equal(tok_seen[r], ex["tok"])
        slots = bt[r, np.arange(T) // bs] * bs + np.arange(T) % bs
        np.testing.assert_array_equal(st.img_page[slots], ex["img_page"])
        np.testing.assert_array_equal(st.marker_cum[slots], ex["marker"])
        np.testing.assert_array_equal(st.img_run[slots], ex["run"])
        np.testing.assert_array_equal(st.prompt_pages[slots], ex["pp"])
        # the unused tail of the last block was reset, the stale 7s elsewhere untouched
        last = bt[r, (T - 1) // bs] * bs
        tail = np.arange(last + T % bs, last + bs) if T % bs else np.arange(0)
        assert (st.img_page[tail] == -1).all()


def test_decode_meta_no_marker_variant_uses_per_page_buckets():
    ids = np.array([0] + [IMG] * 50, np.int64)
    ex = _scan_expectation(ids, 20, None)
    assert list(ex["img_page"][1:]) == [i // 20 for i in range(50)]


def _contiguous_slots(rng, R, nblk, bs):
    """Per-slot image pages of documents whose pages are contiguous runs longer
    than a block (the real layout): a block holds at most two consecutive pages."""
    pages = []
    for _ in range(R):
        seq = []
        p = 0
        while len(seq) < nblk * bs:
            kind = rng.integers(0, 3)
            n = int(rng.integers(bs + 1, 3 * bs))
            seq += [-1] * n if kind == 0 else [p] * n
            p += int(kind != 0)
        pages.append(seq[:nblk * bs])
    return np.array(pages, np.int32)


def test_decode_allow_equals_token_membership():
    rng = np.random.default_rng(5)
    R, nblk, bs = 4, 12, 16
    per_req = _contiguous_slots(rng, R, nblk, bs)
    num_blocks = R * nblk + 3
    perm = rng.permutation(num_blocks)
    bt = perm[:R * nblk].reshape(R, nblk)
    s_page = np.full(num_blocks * bs, -1, np.int32)
    for r in range(R):
        for w in range(nblk):
            s_page[bt[r, w] * bs:(bt[r, w] + 1) * bs] = per_req[r, w * bs:(w + 1) * bs]
    seq = np.array([nblk * bs, 5 * bs + 3, 1, 9 * bs])
    for max_block in (nblk, nblk + 5, nblk - 4):
        for qp in (np.array([0, 1, 2, -1]), np.array([3, 0, 0, 1]), np.array([50, 2, 1, 0])):
            got = P.decode_allow(bt, s_page, qp, seq, max_block, num_blocks, bs)
            W = min(max_block, nblk)
            for r in range(R):
                same = np.zeros(max_block, bool)
                for w in range(W):
                    if w * bs < seq[r] and qp[r] >= 0:
                        same[w] = qp[r] in set(s_page[bt[r, w] * bs:(bt[r, w] + 1) * bs].tolist())
                exp = np.ones(max_block, bool) if not same.any() else same
                np.testing.assert_array_equal(got[r].astype(bool), exp)


def test_local_union_equals_clamped_index_scatter():
    rng = np.random.default_rng(6)
    R, max_block, bs = 5, 20, 16
    for lb in (1, 2, 4, 25):
        allow = rng.integers(0, 2, size=(R, 14)).astype(np.int8)
        seq = np.array([1, 17, 160, 320, 999])
        out = np.full((R, 24), 9, np.int8)
        P.local_union(allow, seq, out, max_block, bs, lb)
        for r in range(R):
            q_blk = (seq[r] - 1) // bs
            win = {min(max(q_blk - j, 0), max_block - 1) for j in range(lb)}      # the torch scatter form
            exp = [int((w < 14 and allow[r, w]) or w in win) for w in range(max_block)]
            assert list(out[r, :max_block]) == exp
            assert (out[r, max_block:] == 9).all()


def test_block_bounds_and_candidates_brute_force():
    rng = np.random.default_rng(7)
    B, L, bs, nblk, cq = 2, 150, 16, 11, 9
    ids = np.where(rng.random((B, L)) < 0.4, rng.integers(0, 6, size=(B, L)), -1)   # any pattern, gaps included
    qtp = rng.integers(-1, 7, size=(B, L))
    pos = rng.integers(-5, L + 10, size=(B, cq))
    bounds = P.block_bounds(ids, nblk, bs)
    cand = P.candidate_mask_page_aware(ids, qtp, pos, nblk, bs)
    for b in range(B):
        for k in range(nblk):
            vals = [int(v) for v in ids[b, k * bs:min((k + 1) * bs, L)] if v >= 0]
            assert tuple(bounds[b, k]) == ((min(vals), max(vals)) if vals else (-1, -1))
        for i in range(cq):
            qp = int(qtp[b, min(max(int(pos[b, i]), 0), L - 1)])
            same = [qp >= 0 and any(int(v) == qp for v in ids[b, k * bs:min((k + 1) * bs, L)])
                    for k in range(nblk)]
            exp = same if any(same) else [True] * nblk
            assert list(cand[b, i]) == exp
    img = rng.random((B, L)) < 0.05
    img[1] = False
    ci = P.candidate_mask_image(img, nblk, bs, cq)
    for b in range(B):
        blk = [bool(img[b, k * bs:min((k + 1) * bs, L)].any()) for k in range(nblk)]
        exp = blk if any(blk) else [True] * nblk
        assert all(list(ci[b, i]) == exp for i in range(cq))


def test_range_test_is_exact_on_contiguous_pages():
    rng = np.random.default_rng(8)
    bs, nblk = 16, 14
    ids = _contiguous_slots(rng, 3, nblk, bs).astype(np.int64)
    bounds = P.block_bounds(ids, nblk, bs)
    for b in range(3):
        for k in range(nblk):
            lo, hi = bounds[b, k]
            assert hi - lo <= 1                  # at most two consecutive pages per block
            for qp in range(-1, 8):
                tok_level = qp >= 0 and qp in set(ids[b, k * bs:(k + 1) * bs].tolist())
                assert tok_level == (lo >= 0 and lo <= qp <= hi and qp >= 0)


@pytest.mark.parametrize("mode", ["resample", "truncate"])
def test_cos_sin_angles_layout_and_identities(mode):
    dim, pairs = 128, 8
    inv_tok, inv_page = P.page2d_freqs(dim, 10000.0, 256.0, pairs, mode)
    rng = np.random.default_rng(9)
    tok = rng.integers(0, 200000, size=40)
    page = rng.integers(-3, 500, size=40)
    for page_mod in (0, 2, 7):
        c, s = P.page2d_cos_sin(tok, page, inv_tok, inv_page, dim, page_mod)
        assert np.abs(c * c + s * s - 1).max() < 1e-12
        # torch's fp32 angle (the reference builds t.float() * inv_tok in fp32)
        t = torch.from_numpy(tok).float()[:, None] * torch.from_numpy(inv_tok)[None, :]
        pm = torch.from_numpy(page)
        if page_mod:
            pm = torch.remainder(pm, page_mod)
        p = pm.float()[:, None] * torch.from_numpy(inv_page)[None, :]
        ang = torch.cat((t, p), 1).double().numpy()
        np.testing.assert_array_equal(np.cos(ang), c[:, :dim // 2])
        np.testing.assert_array_equal(c[:, :dim // 2], c[:, dim // 2:])       # cat(ang, ang)
        np.testing.assert_array_equal(s[:, :dim // 2], s[:, dim // 2:])
        # token columns ignore the page, page columns ignore the token
        c2, _ = P.page2d_cos_sin(tok, page + 1, inv_tok, inv_page, dim, page_mod)
        np.testing.assert_array_equal(c[:, :dim // 2 - pairs], c2[:, :dim // 2 - pairs])
        c3, _ = P.page2d_cos_sin(tok + 1, page, inv_tok, inv_page, dim, page_mod)
        np.testing.assert_array_equal(c[:, dim // 2 - pairs:dim // 2], c3[:, dim // 2 - pairs:dim // 2])
        if page_mod:
            c4, _ = P.page2d_cos_sin(tok, page + page_mod, inv_tok, inv_page, dim, page_mod)
            np.testing.assert_array_equal(c, c4)
    # page axis at frequency 1: page p rotates the first page pair by exactly p radians
    c, s = P.page2d_cos_sin(np.zeros(3, np.int64), np.array([0, 1, 2]), inv_tok, inv_page, dim, 0)
    assert abs(c[1, dim // 2 - pairs] - math.cos(1.0)) < 1e-15 and abs(s[2, dim // 2 - pairs] - math.sin(2.0)) < 1e-15


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_rope_matches_llama_apply_rotary_pos_emb(dtype):
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    g = torch.Generator().manual_seed(10)
    B, H, S, hd = 2, 3, 17, 64
    q = (torch.randn(B, H, S, hd, generator=g) * 3).to(tdt)
    k = (torch.randn(B, 1, S, hd, generator=g) * 3).to(tdt)
    ang = torch.rand(B, S, hd // 2, generator=g) * 1000
    emb = torch.cat((ang, ang), -1)
    cos, sin = emb.cos().to(tdt), emb.sin().to(tdt)
    qe, ke = apply_rotary_pos_emb(q, k, cos, sin)
    oq = P.rope_apply(q.float().numpy(), cos.float().numpy()[:, None], sin.float().numpy()[:, None], dtype)
    ok = P.rope_apply(k.float().numpy(), cos.float().numpy()[:, None], sin.float().numpy()[:, None], dtype)
    np.testing.assert_array_equal(oq, qe.float().numpy())
    np.testing.assert_array_equal(ok, ke.float().numpy())


def test_rope_identities():
    rng = np.random.default_rng(11)
    x = P.round_to(rng.standard_normal((5, 4, 32)).astype(np.float32), "bf16")
    one, zero = np.ones((5, 1, 32), np.float32), np.zeros((5, 1, 32), np.float32)
    np.testing.assert_array_equal(P.rope_apply(x, one, zero, "bf16"), x)                   # angle 0
    rot = np.concatenate([-x[..., 16:], x[..., :16]], -1)
    np.testing.assert_array_equal(P.rope_apply(x, zero, one, "bf16"), rot)                 # angle pi/2
    th = rng.random((5, 1, 16)).astype(np.float32) * 6
    c, s = np.cos(np.concatenate([th, th], -1)), np.sin(np.concatenate([th, th], -1))
    y = P.rope_apply(x, c, s, "f32")
    back = P.rope_apply(y, c, -s, "f32")
    assert np.abs(back - x).max() < 1e-5
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)


# ------------------------------------------------------------ multi-token steps
def _layout(rng, docs, chunks, bs, n_extra_pages=5):
    """Per-request block tables and the slots of every position."""
    R = len(docs)
    L = max(len(d) for d in docs)
    nblk = -(-L // bs) + 1
    perm = rng.permutation(R * nblk + n_extra_pages)
    bt = perm[:R * nblk].reshape(R, nblk).astype(np.int64)
    n_slots = (R * nblk + n_extra_pages) * bs
    return bt, n_slots


def _step_inputs(docs, pos, lens, bt, bs):
    """One serving step: request r contributes docs[r][pos[r]:pos[r]+lens[r]]."""
    ids, slots, q_start = [], [], [0]
    for r, d in enumerate(docs):
        for t in range(pos[r], pos[r] + lens[r]):
            ids.append(d[t])
            slots.append(bt[r, t // bs] * bs + t % bs)
        q_start.append(q_start[-1] + lens[r])
    return np.array(ids, np.int64), np.array(slots, np.int64), np.array(q_start, np.int64)


@pytest.mark.parametrize("seed", [11, 12])
def test_page_step_chunked_equals_token_by_token(seed):
    """PageIsolationState.step's whole-step scans (oracle.page_step), run over
    whole prompts in random chunk sizes, give the q_page / per-slot state of the
    token-by-token state machine (the same step one token at a time, a
    different formulation: no scans), and on generated tokens the pinned
    one-token decode restatement."""
    rng = np.random.default_rng(seed)
    bs, per_page = 16, 24
    docs = [_document(rng, int(rng.integers(1, 4)), with_markers=bool(r % 2 == 0)) for r in range(3)]
    bt, n_slots = _layout(rng, docs, None, bs)
    R = len(docs)
    st_a, st_b = P.SlotState(n_slots), P.SlotState(n_slots)
    L = [len(d) for d in docs]
    q_a = [np.zeros(n, np.int32) for n in L]
    q_b = [np.zeros(n, np.int32) for n in L]
    # (a) random chunks, all requests in one step each time
    pos = [0] * R
    while any(pos[r] < L[r] for r in range(R)):
        lens = [min(int(rng.integers(0, 40)), L[r] - pos[r]) for r in range(R)]
        ids, slots, q_start = _step_inputs(docs, pos, lens, bt, bs)
        if len(ids) == 0:
            continue
        q = P.page_step(ids, q_start, np.array(pos), bt, slots, st_a, IMG, PG, per_page, bs)
        for r in range(R):
            q_a[r][pos[r]:pos[r] + lens[r]] = q[q_start[r]:q_start[r + 1]]
            pos[r] += lens[r]
    # (b) token by token as a plain state machine
    n = n_slots
    for r in range(R):
        m = run = pp = 0
        for t in range(L[r]):
            tid = int(docs[r][t])
            img = tid >= P.MM_PAD_SHIFT or tid == IMG
            m += int(tid == PG)
            run += int(img)
            if img:
                pp = max(pp, m)
            ip = (m - 1 if m > 0 else (run - 1) // per_page) if img else -1
            q_b[r][t] = ip if img else (m - 1 if m > pp else -1)
            sl = bt[r, t // bs] * bs + t % bs
            st_b.img_page[sl], st_b.marker_cum[sl], st_b.img_run[sl], st_b.prompt_pages[sl] = ip, m, run, pp
        end = L[r]
        if end % bs:
            last = bt[r, (end - 1) // bs] * bs
            st_b.img_page[last + end % bs:last + bs] = -1
    for r in range(R):
        np.testing.assert_array_equal(q_a[r], q_b[r])
        slots = bt[r, np.arange(L[r]) // bs] * bs + np.arange(L[r]) % bs
        for f in ("img_page", "marker_cum", "img_run", "prompt_pages"):
            np.testing.assert_array_equal(getattr(st_a, f)[slots], getattr(st_b, f)[slots], err_msg=f)
    # (c) generated tokens: page_step with every token generated equals the
    # pinned one-token decode restatement
    st_c, st_d = P.SlotState(n_slots), P.SlotState(n_slots)
    cs = P.CoordState(R, 64)
    T = min(L)
    for t in range(T):
        ids = np.array([d[t] for d in docs], np.int64)
        slots = bt[np.arange(R), t // bs] * bs + t % bs
        qs = np.arange(R + 1, dtype=np.int64)
        qc = P.page_step(ids, qs, np.full(R, t), bt, slots, st_c, IMG, PG, per_page, bs, num_decode_tokens=R)
        qd, _, _ = P.decode_meta_step(ids, bt, np.full(R, t + 1), slots, np.arange(R), st_d, cs, IMG, PG,
                                      per_page, bs)
        np.testing.assert_array_equal(qc, qd)


def test_coord_step_chunked_equals_token_by_token():
    """PageCoordState.step's scans + stable-sort ranks (oracle.coord_step) over
    random chunks equal a per-token state machine with per-page counters, and
    on generated tokens the pinned one-token decode coordinates."""
    rng = np.random.default_rng(13)
    docs = [_document(rng, int(rng.integers(1, 4))) for _ in range(3)]
    R, pages = len(docs), 32
    L = [len(d) for d in docs]
    cs = P.CoordState(R + 2, pages)
    rows = np.array([2, 0, 3])
    tok_a = [np.zeros(n, np.int64) for n in L]
    page_a = [np.zeros(n, np.int64) for n in L]
    pos = [0] * R
    gen_start = np.array([L[r] - 6 for r in range(R)])   # the last 6 tokens are generated
    while any(pos[r] < L[r] for r in range(R)):
        lens = [min(int(rng.integers(0, 30)), L[r] - pos[r]) for r in range(R)]
        ids, _, q_start = _step_inputs(docs, pos, lens, np.zeros((R, 64), np.int64), 16)
        if len(ids) == 0:
            continue
        tok, page, _, _ = P.coord_step(ids, q_start, np.array(pos), rows, cs, IMG, PG, gen_start=gen_start)
        for r in range(R):
            tok_a[r][pos[r]:pos[r] + lens[r]] = tok[q_start[r]:q_start[r + 1]]
            page_a[r][pos[r]:pos[r] + lens[r]] = page[q_start[r]:q_start[r + 1]]
            pos[r] += lens[r]
    for r in range(R):
        m = pp = 0
        cnt = np.zeros(pages, np.int64)
        for t in range(L[r]):
            tid = int(docs[r][t])
            img = tid >= P.MM_PAD_SHIFT or tid == IMG
            m += int(tid == PG)
            if img:
                pp = max(pp, m)
            gen = t >= gen_start[r]
            pre = (not gen) and (img or m > pp)
            pg = min(max(m if pre else min(max(m - pp, 0), pp), 0), pages - 1)
            assert page_a[r][t] == pg and tok_a[r][t] == cnt[pg], (r, t)
            cnt[pg] += 1
        np.testing.assert_array_equal(cs.cnt[rows[r]], cnt)


def _ids_batch(rng, B, marker_rows=True):
    docs = [_document(rng, int(rng.integers(1, 4)), with_markers=marker_rows or b % 2 == 1) for b in range(B)]
    L = max(len(d) for d in docs)
    return np.stack([np.concatenate([d, np.full(L - len(d), 5)]) for d in docs]), L


@pytest.mark.parametrize("scope", [True, False])
def test_page_aware_ids_per_token_state_machine(scope):
    """_build_page_aware_ids (oracle.page_aware_ids) against a per-row walk
    that counts markers / image tokens as it goes (two passes: find the last
    image token, then assign)."""
    rng = np.random.default_rng(14)
    ids, L = _ids_batch(rng, 4, marker_rows=False)
    klen = L + 7                                            # padded with -1 past the ids
    img, ipage, q = P.page_aware_ids(ids, IMG, PG, klen, 24, page_scope_prefill=scope)
    for b in range(len(ids)):
        row = list(ids[b]) + [-1] * 7
        last = max([i for i, v in enumerate(row) if v == IMG], default=-1)
        npp = sum(1 for v in row[:last + 1] if v == PG) if last >= 0 else 0
        cum = run = 0
        for i, v in enumerate(row):
            cum += int(v == PG)
            run += int(v == IMG)
            assert img[b, i] == (v == IMG)
            exp_ip = ((cum - 1) if npp > 0 else (run - 1) // 24) if v == IMG else -1
            assert ipage[b, i] == exp_ip
            if i <= last:
                eq = cum - 1 if scope else -1
            else:
                eq = cum - 1 - (npp if npp > 0 else 0)
            assert q[b, i] == (eq if eq >= 0 else -1), (b, i)
    none = P.page_aware_ids(np.full((2, 30), 7), IMG, PG, 30, 24)
    assert none == (None, None, None)


def test_page_rope_pos_brute_force():
    """_build_page_rope_pos + the running counts (oracle.page_rope_pos):
    tok = earlier tokens of the row in the same page, pf_cnt = prefill tokens
    per page, both by brute force; bails where the reference bails."""
    rng = np.random.default_rng(15)
    ids, L = _ids_batch(rng, 3)
    tok, page, pf = P.page_rope_pos(ids, IMG, PG, L)
    for b in range(len(ids)):
        row = list(ids[b])
        last = max(i for i, v in enumerate(row) if v == IMG)
        for i in range(L):
            assert tok[b, i] == sum(1 for j in range(i) if page[b, j] == page[b, i])
        for p in range(pf.shape[1]):
            assert pf[b, p] == sum(1 for j in range(last + 1) if page[b, j] == p)
    assert P.page_rope_pos(np.full((1, 20), 3), IMG, PG, 20) is None
    no_mark = np.array([[0] + [IMG] * 10 + [5] * 4])
    assert P.page_rope_pos(no_mark, IMG, PG, 15) is None
