"""Page isolation + Page2D RoPE kernels (srswa_page_* / srswa_page2d_*) vs the
CPU oracle (oracle/page_oracle.py):

* integer work -- decode page state and coordinates, decode allow masks, the
  local union, block bounds and the page-aware candidate masks -- bit-exact;
* the rotary application bit-exact in bf16 / fp16 / fp32 (each product and
  the sum rounded to the dtype, the reference's eager order);
* the cos / sin table: fp32 within 1e-6 of cos / sin of the fp32 angle; bf16
  within one bf16 ulp, 99.9% of entries identical (fp32 cos / sin round a
  value lying within an ulp of a bf16 rounding boundary either way).

Plus the serving drop-ins (``srswa.unlimited_dash_ops``) and the HF rebinding
(``srswa.patch``) on stand-ins of the reference's state objects and classes."""

import math
import types

import numpy as np
import pytest
import torch

from oracle import page_oracle as P

pytestmark = pytest.mark.gpu

IMG, PG = 128815, 128816


def _docs(rng, R, T):
    out = []
    for r in range(R):
        toks = [0]
        while len(toks) < T // 2:
            toks.append(PG if r % 3 else 5)
            toks += [IMG if r % 2 else P.MM_PAD_SHIFT + r] * int(rng.integers(20, 60))
        toks += list(rng.integers(10, 1000, size=5))
        while len(toks) < T:
            toks.append(PG)
            toks += list(rng.integers(10, 1000, size=int(rng.integers(3, 12))))
        out.append(np.array(toks[:T], np.int64))
    return out


@pytest.mark.parametrize("idx_dtype,bs", [(torch.int64, 16), (torch.int32, 64)])
def test_decode_meta_token_by_token(dev, idx_dtype, bs):
    from srswa import page_ops
    print(f"decode meta idx={idx_dtype} bs={bs}", flush=True)
    rng = np.random.default_rng(21 + bs)
    R, T, per_page, max_pages = 5, 300, 30, 16
    docs = _docs(rng, R, T)
    nblk = -(-T // bs)
    npg = R * nblk + 4
    bt = rng.permutation(npg)[:R * nblk].reshape(R, nblk)
    n_slots = npg * bs
    st, cs = P.SlotState(n_slots), P.CoordState(R + 2, max_pages)
    st.img_page[:] = 3
    rows = np.array([2, 0, 4, 1, 3])
    d = dict(s_page=torch.from_numpy(st.img_page.copy()).to(dev), s_mark=torch.zeros(n_slots, dtype=torch.int32, device=dev),
             s_run=torch.zeros(n_slots, dtype=torch.int32, device=dev),
             s_pp=torch.zeros(n_slots, dtype=torch.int32, device=dev),
             c_mark=torch.zeros(R + 2, dtype=torch.int32, device=dev), c_pp=torch.zeros(R + 2, dtype=torch.int32, device=dev),
             c_cnt=torch.zeros(R + 2, max_pages, dtype=torch.int32, device=dev))
    bt_d = torch.from_numpy(bt).to(dev, idx_dtype)
    rows_d = torch.from_numpy(rows).to(dev)
    for t in range(T):
        ids = np.array([dd[t] for dd in docs])
        seq = np.full(R, t + 1)
        slot = bt[np.arange(R), t // bs] * bs + t % bs
        q, tok, page = P.decode_meta_step(ids, bt, seq, slot, rows, st, cs, IMG, PG, per_page, bs)
        gq, gt, gp = page_ops.page_decode_meta(
            torch.from_numpy(ids).to(dev, idx_dtype), bt_d, torch.from_numpy(seq).to(dev, idx_dtype),
            torch.from_numpy(slot).to(dev, idx_dtype), rows_d, image_token_id=IMG, page_token_id=PG,
            per_page=per_page, block_size=bs, **d)
        assert gq.cpu().numpy().tolist() == q.tolist(), t
        assert gt.cpu().numpy().tolist() == tok.tolist(), t
        assert gp.cpu().numpy().tolist() == page.tolist(), t
    np.testing.assert_array_equal(d["s_page"].cpu().numpy(), st.img_page)
    np.testing.assert_array_equal(d["s_mark"].cpu().numpy(), st.marker_cum)
    np.testing.assert_array_equal(d["s_run"].cpu().numpy(), st.img_run)
    np.testing.assert_array_equal(d["s_pp"].cpu().numpy(), st.prompt_pages)
    np.testing.assert_array_equal(d["c_cnt"].cpu().numpy(), cs.cnt)
    np.testing.assert_array_equal(d["c_mark"].cpu().numpy(), cs.st_marker)
    np.testing.assert_array_equal(d["c_pp"].cpu().numpy(), cs.st_pp)


def _slot_pages(rng, num_blocks, bs, runs=True):
    n = num_blocks * bs
    if not runs:
        return np.where(rng.random(n) < 0.5, rng.integers(0, 9, n), -1).astype(np.int32)
    out, p = [], 0
    while len(out) < n:
        k = int(rng.integers(bs // 2 + 1, 3 * bs))
        out += [-1] * k if rng.random() < 0.3 else [p] * k
        p += 1
    return np.array(out[:n], np.int32)


@pytest.mark.parametrize("bs,R,nblk,runs", [(16, 6, 40, True), (64, 9, 130, True), (128, 3, 70, False),
                                            (32, 4, 3, False), (256, 2, 9, True)])
def test_decode_allow(dev, bs, R, nblk, runs):
    from srswa import page_ops
    print(f"decode allow bs={bs} R={R} nblk={nblk}", flush=True)
    rng = np.random.default_rng(bs + R)
    num_blocks = R * nblk + 5
    s_page = _slot_pages(rng, num_blocks, bs, runs)
    bt = rng.permutation(num_blocks)[:R * nblk].reshape(R, nblk)
    bt[0, -1] = num_blocks + 50            # out of range: clamped to the last page
    seq = rng.integers(1, nblk * bs + 1, size=R)
    seq[-1] = nblk * bs
    qp = rng.integers(-1, 12, size=R).astype(np.int32)
    for max_block in (nblk, nblk + 70, max(1, nblk - 2)):
        ref = P.decode_allow(bt, s_page, qp, seq, max_block, num_blocks, bs)
        out = torch.full((R + 1, max_block + 3), 7, dtype=torch.int8, device=dev)
        got = page_ops.page_decode_allow(torch.from_numpy(bt).to(dev), torch.from_numpy(s_page).to(dev),
                                         torch.from_numpy(qp).to(dev), torch.from_numpy(seq).to(dev, torch.int32),
                                         max_block=max_block, num_blocks=num_blocks, block_size=bs, out=out)
        np.testing.assert_array_equal(got.cpu().numpy(), ref)
        assert (out[R:].cpu() == 7).all() and (out[:, max_block:].cpu() == 7).all()


def test_decode_allow_serving_size(dev):
    """64 requests x 2048 pages of 64 slots (a 128k-token cache)."""
    from srswa import page_ops
    rng = np.random.default_rng(5)
    R, nblk, bs = 64, 2048, 64
    num_blocks = R * nblk
    s_page = _slot_pages(rng, num_blocks, bs)
    bt = rng.permutation(num_blocks).reshape(R, nblk)
    seq = rng.integers(4096, nblk * bs + 1, size=R)
    qp = rng.integers(-1, 400, size=R).astype(np.int32)
    ref = P.decode_allow(bt, s_page, qp, seq, nblk, num_blocks, bs)
    got = page_ops.page_decode_allow(torch.from_numpy(bt).to(dev), torch.from_numpy(s_page).to(dev),
                                     torch.from_numpy(qp).to(dev), torch.from_numpy(seq).to(dev),
                                     max_block=nblk, num_blocks=num_blocks, block_size=bs)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)


def test_local_union(dev):
    from srswa import page_ops
    rng = np.random.default_rng(8)
    R, bs = 7, 64
    seq = np.array([0, 1, 64, 65, 4000, 70000, 3])
    for lb, aw, ow, mb in ((4, 30, 40, 35), (1, 50, 20, 45), (0, 10, 64, 64), (9, 64, 64, 64)):
        allow = rng.integers(0, 2, size=(R, aw)).astype(np.int8)
        ref = np.full((R, ow), 5, np.int8)
        P.local_union(allow, seq, ref, mb, bs, lb)
        out = torch.full((R, ow), 5, dtype=torch.int8, device=dev)
        page_ops.page_local_union(torch.from_numpy(allow).to(dev), torch.from_numpy(seq).to(dev), out,
                                  max_block=mb, block_size=bs, local_blocks=lb)
        np.testing.assert_array_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_cos_sin(dev, dtype):
    from srswa import page_ops
    rng = np.random.default_rng(9)
    T, dim, pairs = 777, 128, 8
    inv_tok, inv_page = P.page2d_freqs(dim, 10000.0, 256.0, pairs)
    tok = rng.integers(0, 200000, size=T)
    page = rng.integers(-5, 3000, size=T)
    for page_mod in (0, 2):
        c, s = P.page2d_cos_sin(tok, page, inv_tok, inv_page, dim, page_mod)
        gc, gs = page_ops.page2d_cos_sin(torch.from_numpy(tok).to(dev), torch.from_numpy(page).to(dev, torch.int32),
                                         torch.from_numpy(inv_tok), torch.from_numpy(inv_page), dim=dim,
                                         page_mod=page_mod, dtype=dtype)
        for got, ref in ((gc, c), (gs, s)):
            g = got.float().cpu().numpy().astype(np.float64)
            if dtype == torch.float32:
                assert np.abs(g - ref).max() <= 1e-6
            else:
                key = "bf16" if dtype == torch.bfloat16 else "f16"
                r = P.round_to(ref.astype(np.float32), key).astype(np.float64)
                ulp = 2.0 ** -8 if key == "bf16" else 2.0 ** -11
                assert np.abs(g - r).max() <= ulp
                assert (g == r).mean() >= 0.999


@pytest.mark.parametrize("dtype,key", [(torch.bfloat16, "bf16"), (torch.float16, "f16"), (torch.float32, "f32")])
def test_rope_flat_pair(dev, dtype, key):
    from srswa import page_ops
    g = torch.Generator().manual_seed(12)
    T, hd, HX, HY = 301, 128, 10, 1
    x = (torch.randn(T, HX * hd, generator=g) * 4).to(dtype)
    y = (torch.randn(T, HY * hd, generator=g) * 4).to(dtype)
    ang = torch.rand(T, hd // 2, generator=g) * 3000
    cos = torch.cat((ang, ang), -1).cos().to(dtype)
    sin = torch.cat((ang, ang), -1).sin().to(dtype)
    ox, oy = page_ops.page2d_rope(x.to(dev), cos.to(dev), sin.to(dev), hd, y=y.to(dev))
    for src, got, H in ((x, ox, HX), (y, oy, HY)):
        ref = P.rope_apply(src.float().view(T, H, hd).numpy(), cos.float().numpy()[:, None],
                           sin.float().numpy()[:, None], key)
        np.testing.assert_array_equal(got.float().cpu().view(T, H, hd).numpy(), ref)
    single = page_ops.page2d_rope(x.to(dev), cos.to(dev), sin.to(dev), hd)
    assert torch.equal(single, ox)


@pytest.mark.parametrize("dtype,key,hd", [(torch.bfloat16, "bf16", 128), (torch.float16, "f16", 64),
                                          (torch.float32, "f32", 64)])
def test_rope_bhsd_strided(dev, dtype, key, hd):
    """HF layout: q / k as transposed views of [B, S, H, hd], cos / sin [1, S, hd]."""
    from srswa import page_ops
    g = torch.Generator().manual_seed(13)
    B, S, Hq, Hk = 2, 90, 4, 1
    q = (torch.randn(B, S, Hq, hd, generator=g) * 2).to(dtype).to(dev).transpose(1, 2)
    k = (torch.randn(B, S, Hk, hd, generator=g) * 2).to(dtype).to(dev).transpose(1, 2)
    ang = torch.rand(1, S, hd // 2, generator=g) * 100
    cos = torch.cat((ang, ang), -1).cos().to(dtype).to(dev)
    sin = torch.cat((ang, ang), -1).sin().to(dtype).to(dev)
    oq, ok = page_ops.rope_bhsd(q, k, cos, sin)
    for src, got in ((q, oq), (k, ok)):
        ref = P.rope_apply(src.float().cpu().numpy(), cos.float().cpu().numpy()[:, None],
                           sin.float().cpu().numpy()[:, None], key)
        np.testing.assert_array_equal(got.float().cpu().numpy(), ref)


@pytest.mark.parametrize("gaps", [True, False])
def test_block_bounds_and_candidates(dev, gaps):
    from srswa import page_ops
    rng = np.random.default_rng(14 + gaps)
    B, L, bs, cq = 3, 2000, 64, 300
    nblk = -(-L // bs) + 2                        # blocks past the ids count as empty
    if gaps:
        ids = np.where(rng.random((B, L)) < 0.3, rng.integers(0, 12, size=(B, L)), -1)
    else:
        ids = np.stack([_slot_pages(rng, -(-L // bs), bs)[:L] for _ in range(B)])
    qtp = rng.integers(-1, 14, size=(B, L))
    pos = rng.integers(-20, L + 20, size=(B, cq))
    ref_b = P.block_bounds(ids, nblk, bs)
    ref_c = P.candidate_mask_page_aware(ids, qtp, pos, nblk, bs)
    ids_d = torch.from_numpy(ids).to(dev)
    gb = page_ops.page_block_bounds(ids_d, nblk=nblk, block_size=bs)
    np.testing.assert_array_equal(gb.cpu().numpy(), ref_b)
    gc = page_ops.page_candidate_mask(gb, ids_d.to(torch.int32), torch.from_numpy(qtp).to(dev),
                                      torch.from_numpy(pos).to(dev, torch.int32), nblk=nblk, block_size=bs)
    np.testing.assert_array_equal(gc.cpu().numpy(), ref_c)
    if not gaps:                                  # contiguous pages: the plain range test is the same mask
        gr = page_ops.page_candidate_mask(gb, None, torch.from_numpy(qtp).to(dev),
                                          torch.from_numpy(pos).to(dev), nblk=nblk, block_size=bs, range_test=True)
        np.testing.assert_array_equal(gr.cpu().numpy(), ref_c)


# --------------------------------------------------------------- drop-ins
class _PageState:
    def __init__(self, n, dev):
        self.image_token_id, self.page_token_id, self.per_page_image_tokens = IMG, PG, 30
        self._slot_img_page = torch.full((n,), -1, dtype=torch.int32, device=dev)
        self._slot_marker_cum = torch.zeros(n, dtype=torch.int32, device=dev)
        self._slot_img_run = torch.zeros(n, dtype=torch.int32, device=dev)
        self._slot_prompt_pages = torch.zeros(n, dtype=torch.int32, device=dev)

    def _ensure(self, n, device):
        assert self._slot_img_page.numel() >= n


class _CoordState:
    def __init__(self, rows, max_pages, dev, row_of_req):
        self.max_pages = max_pages
        self.st_marker = torch.zeros(rows, dtype=torch.int32, device=dev)
        self.st_pp = torch.zeros(rows, dtype=torch.int32, device=dev)
        self.cnt = torch.zeros(rows, max_pages, dtype=torch.int32, device=dev)
        self.row_of_req = row_of_req

    def _ensure(self, device):
        pass

    def _rows(self, layout):
        assert layout.start_pos.dtype == torch.int64
        return self.row_of_req


def test_serving_dropins(dev):
    from srswa import unlimited_dash_ops as U
    rng = np.random.default_rng(15)
    R, T, bs, max_pages = 3, 200, 64, 12
    docs = _docs(rng, R, T)
    nblk = -(-T // bs)
    npg = R * nblk + 2
    bt = rng.permutation(npg)[:R * nblk].reshape(R, nblk)
    ps, st = _PageState(npg * bs, dev), P.SlotState(npg * bs)
    rows = np.array([1, 2, 0])
    cs_d, cs = _CoordState(R, max_pages, dev, torch.from_numpy(rows).to(dev)), P.CoordState(R, max_pages)
    rope = U.PageRope2D(128, 10000.0, 256.0, 8)
    qb, tb, pb = (torch.empty(8, dtype=d, device=dev) for d in (torch.int32, torch.int64, torch.int64))
    cos_buf = torch.empty(8, 128, dtype=torch.bfloat16, device=dev)
    sin_buf = torch.empty(8, 128, dtype=torch.bfloat16, device=dev)
    for t in range(T):
        ids = np.array([d[t] for d in docs])
        seq, slot = np.full(R, t + 1), bt[np.arange(R), t // bs] * bs + t % bs
        q, tok, page = P.decode_meta_step(ids, bt, seq, slot, rows, st, cs, IMG, PG, 30, bs)
        seq_d = torch.from_numpy(seq).to(dev, torch.int32)
        gq, (gt, gp) = U.decode_meta_fused(input_ids=torch.from_numpy(ids).to(dev), block_table=torch.from_numpy(bt).to(dev),
                                           seq_lens=seq_d, slot_mapping=torch.from_numpy(slot).to(dev),
                                           page_state=ps, coord_state=cs_d, num_slots=npg * bs, block_size=bs,
                                           out_q_page=qb, out_tok=tb, out_page=pb)
        assert gq.data_ptr() == qb.data_ptr() and gq.cpu().tolist() == q.tolist()
        assert gt.cpu().tolist() == tok.tolist() and gp.cpu().tolist() == page.tolist()
        if t % 37 == 0 or t == T - 1:
            ref = P.decode_allow(bt, st.img_page, q, seq, nblk + 3, npg, bs)
            got = U.decode_allow_fused(block_table=torch.from_numpy(bt).to(dev), page_state=ps, q_page=gq,
                                       seq_lens=seq_d, max_block=nblk + 3, num_blocks=npg, block_size=bs)
            np.testing.assert_array_equal(got.cpu().numpy(), ref)
            un = torch.zeros(R, nblk + 5, dtype=torch.int8, device=dev)
            U.local_union_fused(allow=got, seq_lens=seq_d, out=un, max_block=nblk + 3, block_size=bs,
                                local_blocks=2)
            ref_u = np.zeros((R, nblk + 5), np.int8)
            P.local_union(ref, seq, ref_u, nblk + 3, bs, 2)
            np.testing.assert_array_equal(un.cpu().numpy(), ref_u)
            c, s = U.cos_sin_2d_fused(rope=rope, tok_pos=gt, page_pos=gp, dtype=torch.bfloat16,
                                      out_cos=cos_buf, out_sin=sin_buf)
            assert c.data_ptr() == cos_buf.data_ptr()
            rc, rs = P.page2d_cos_sin(tok, page, rope.inv_tok.numpy(), rope.inv_page.numpy(), 128)
            assert np.abs(c.float().cpu().numpy() - rc).max() <= 2.0 ** -8
            x = torch.randn(R, 10 * 128, device=dev).to(torch.bfloat16)
            y = torch.randn(R, 128, device=dev).to(torch.bfloat16)
            ox, oy = U.apply_page2d_rope_pair(x, y, c, s, 128)
            ref_x = P.rope_apply(x.float().cpu().view(R, 10, 128).numpy(), c.float().cpu().numpy()[:, None],
                                 s.float().cpu().numpy()[:, None], "bf16")
            np.testing.assert_array_equal(ox.float().cpu().view(R, 10, 128).numpy(), ref_x)
            assert torch.equal(U.apply_page2d_rope(y, c, s, 128), oy)
    np.testing.assert_array_equal(ps._slot_img_page.cpu().numpy(), st.img_page)


def test_hf_patch_page_isolation(dev):
    """srswa.patch rebinds the indexer's candidate mask, the 2-axis rotary and
    the llama rotary of a stand-in _sparse_base_impl; results vs the oracle."""
    from srswa import patch

    calls = []

    class DeepseekV2Indexer:
        block_size = 64
        image_bucket_constraint = True

        def _build_kl_candidate_mask(self, *a, **k):
            calls.append("mask")
            return "eager-mask"

    class DeepseekV2IndexerRotary2D:
        def __init__(self):
            self.dim, self.page_mod = 128, 0
            self.inv_tok, self.inv_page = (torch.from_numpy(t) for t in P.page2d_freqs(128, 10000.0, 256.0, 8))

        def forward(self, x, tok_pos, page_pos):
            calls.append("rot")
            return "eager-rot"

    def _llama_apply_rotary_pos_emb(q, k, cos, sin, position_ids=None, unsqueeze_dim=1):
        calls.append("rope")
        return "eager-rope"

    base = types.ModuleType("_sparse_base_impl")
    base.DeepseekV2Indexer, base.DeepseekV2IndexerRotary2D = DeepseekV2Indexer, DeepseekV2IndexerRotary2D
    base._llama_apply_rotary_pos_emb = _llama_apply_rotary_pos_emb
    mod = types.SimpleNamespace(_base=base)
    names = patch.apply(mod)
    assert "DeepseekV2Indexer._build_kl_candidate_mask" in names and "DeepseekV2IndexerRotary2D.forward" in names
    rng = np.random.default_rng(16)
    B, L, cq, bs = 2, 1000, 50, 64
    nblk = -(-L // bs)
    ids = np.stack([_slot_pages(rng, nblk, bs)[:L] for _ in range(B)])
    qtp = rng.integers(-1, 20, size=(B, L))
    pos = rng.integers(0, L, size=(B, cq))
    idx = DeepseekV2Indexer()
    got = idx._build_kl_candidate_mask(torch.from_numpy(pos).to(dev), nblk, None, B, cq,
                                       torch.from_numpy(ids).to(dev), torch.from_numpy(qtp).to(dev))
    assert got.shape == (B, 1, cq, nblk)
    np.testing.assert_array_equal(got[:, 0].cpu().numpy(), P.candidate_mask_page_aware(ids, qtp, pos, nblk, bs))
    img = rng.random((B, L)) < 0.02
    got = idx._build_kl_candidate_mask(torch.from_numpy(pos).to(dev), nblk, torch.from_numpy(img).to(dev), B, cq)
    np.testing.assert_array_equal(got[:, 0].cpu().numpy(), P.candidate_mask_image(img, nblk, bs, cq))
    # host tensors still reach the original
    assert idx._build_kl_candidate_mask(torch.from_numpy(pos), nblk, None, B, cq) == "eager-mask"
    rot = DeepseekV2IndexerRotary2D()
    x = torch.zeros(B, 4, 7, 128, dtype=torch.bfloat16, device=dev)
    tok = torch.from_numpy(rng.integers(0, 5000, size=(B, 7))).to(dev)
    page = torch.from_numpy(rng.integers(0, 40, size=(B, 7))).to(dev)
    c, s = rot.forward(x, tok, page)
    assert c.shape == (B, 7, 128) and c.dtype == torch.bfloat16
    rc, _ = P.page2d_cos_sin(tok.cpu().numpy().ravel(), page.cpu().numpy().ravel(), rot.inv_tok.numpy(),
                             rot.inv_page.numpy(), 128)
    assert np.abs(c.float().cpu().numpy().reshape(-1, 128) - rc).max() <= 2.0 ** -8
    q = torch.randn(B, 4, 7, 128, device=dev).to(torch.bfloat16)
    k = torch.randn(B, 1, 7, 128, device=dev).to(torch.bfloat16)
    oq, ok = base._llama_apply_rotary_pos_emb(q, k, c, s)
    ref = P.rope_apply(q.float().cpu().numpy(), c.float().cpu().numpy()[:, None], s.float().cpu().numpy()[:, None], "bf16")
    np.testing.assert_array_equal(oq.float().cpu().numpy(), ref)
    assert calls == ["mask"]
    patch.restore(mod)
    assert base._llama_apply_rotary_pos_emb is _llama_apply_rotary_pos_emb
    assert DeepseekV2Indexer()._build_kl_candidate_mask() == "eager-mask"


def test_hf_decode_allow(dev):
    """_uocr_dash_decode_allow: prefill bounds then decode rows, vs the
    reference's own torch formulas restated on the CPU (min / max test)."""
    from srswa import page_isolation as PI

    class Cache:
        def __init__(self, n):
            self.n = n

        def get_seq_length(self):
            return self.n

    rng = np.random.default_rng(17)
    B, bs = 2, 64
    docs = _docs(rng, B, 900)
    ids = torch.from_numpy(np.stack(docs)).to(dev)
    ind = types.SimpleNamespace(image_token_id=IMG, page_token_id=PG, block_size=bs, per_page_image_tokens=30)
    cache = Cache(0)
    assert PI.uocr_dash_decode_allow(ind, ids, cache) is None
    cache.n = 900
    # CPU restatement: per-token image page, block bounds, query page of the next token
    npi = np.stack(docs)
    is_img = (npi == IMG) | (npi >= P.MM_PAD_SHIFT)
    cum = np.cumsum(npi == PG, axis=1)
    run = np.cumsum(is_img, axis=1)
    page = np.where(is_img, np.where(cum > 0, cum - 1, (run - 1) // 30), -1)
    bounds = P.block_bounds(page, -(-900 // bs), bs)
    pp = np.where(is_img, cum, 0).max(axis=1)
    for step, tokid in enumerate([PG, 77, PG, 5, PG]):
        nxt = torch.full((B, 1), tokid, device=dev)
        got = PI.uocr_dash_decode_allow(ind, nxt, cache)
        cum_last = cum[:, -1] + sum(1 for t in [PG, 77, PG, 5, PG][:step + 1] if t == PG)
        qp = cum_last - 1 - pp
        qp = np.where(qp >= 0, qp, -1)
        nblk = -(-(cache.n + 1) // bs)
        for b in range(B):
            lo, hi = bounds[b, :, 0], bounds[b, :, 1]
            same = (lo >= 0) & (lo <= qp[b]) & (hi >= qp[b]) & (qp[b] >= 0)
            exp = np.zeros(nblk, bool)
            exp[:len(same)] = same[:nblk]
            if qp[b] < 0 or not same.any():
                exp[:] = True
            np.testing.assert_array_equal(got[b].cpu().numpy(), exp)
        cache.n += 1
