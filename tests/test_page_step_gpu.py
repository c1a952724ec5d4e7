"""Multi-token page state on the device (srswa_page_step / srswa_coord_step /
srswa_page_ids / srswa_page_rope_pos + _tok) against the CPU oracle
(oracle/page_oracle.py, pinned by tests/test_page_pins.py): every output and
every state array bit-exact (integer work).

Steps mix prefill chunks of several requests, decode tokens at the front of
the flat batch (num_decode_tokens), generated tokens inside an extend
(gen_start), stale per-slot pages from an earlier request, int32 and int64
index arrays, and chunks of more than one 256-token scan block."""

import types

import numpy as np
import pytest
import torch

from oracle import page_oracle as P

pytestmark = pytest.mark.gpu
IMG, PG = 128815, 128816


def _doc(rng, pages, img=(60, 300), mark=0.8):
    toks = [0]
    for _ in range(pages):
        if rng.random() < mark:
            toks.append(PG)
        toks += [IMG] * int(rng.integers(*img))
    toks += list(rng.integers(10, 1000, size=int(rng.integers(3, 9))))
    for _ in range(pages + 1):
        toks.append(PG)
        toks += list(rng.integers(10, 1000, size=int(rng.integers(2, 40))))
    return np.array(toks, np.int64)


def _steps(rng, docs, max_chunk=700):
    """Serving steps over the documents: each step, every unfinished request
    contributes a chunk (a finished-prompt request one generated token)."""
    pos = [0] * len(docs)
    while any(p < len(d) for p, d in zip(pos, docs)):
        lens = [min(int(rng.integers(1, max_chunk)), len(d) - p) for p, d in zip(pos, docs)]
        yield list(pos), lens
        pos = [p + n for p, n in zip(pos, lens)]


def _flat(docs, pos, lens, bt, bs):
    ids, slots, qs = [], [], [0]
    for r, d in enumerate(docs):
        for t in range(pos[r], pos[r] + lens[r]):
            ids.append(d[t])
            slots.append(bt[r, t // bs] * bs + t % bs)
        qs.append(qs[-1] + lens[r])
    return np.array(ids, np.int64), np.array(slots, np.int64), np.array(qs, np.int64)


@pytest.mark.parametrize("i64", [False, True])
def test_page_step_matches_oracle(dev, i64):
    print(f"page step i64={i64}", flush=True)
    rng = np.random.default_rng(21 + int(i64))
    bs, per_page = 16, 24
    docs = [_doc(rng, int(rng.integers(1, 5))) for _ in range(4)]
    nblk = max(-(-len(d) // bs) for d in docs) + 1
    R = len(docs)
    perm = rng.permutation(R * nblk + 3)
    bt = perm[:R * nblk].reshape(R, nblk).astype(np.int64)
    n_slots = (R * nblk + 3) * bs
    st = P.SlotState(n_slots)
    st.img_page[:] = 9                                     # stale pages of an earlier request
    dt = torch.int64 if i64 else torch.int32
    s_dev = [torch.tensor(x, dtype=torch.int32, device=dev) for x in
             (st.img_page, st.marker_cum, st.img_run, st.prompt_pages)]
    from srswa import page_ops
    for k, (pos, lens) in enumerate(_steps(rng, docs)):
        ids, slots, qs = _flat(docs, pos, lens, bt, bs)
        nd = 1 if k % 3 == 2 else 0                        # the first token counts as a decode token
        gen = np.array([len(d) - 40 for d in docs]) if k % 2 else None
        exp = P.page_step(ids, qs, np.array(pos), bt, slots, st, IMG, PG, per_page, bs, num_decode_tokens=nd,
                          gen_start=gen)
        got = page_ops.page_step(torch.tensor(ids, dtype=dt, device=dev), torch.tensor(qs, device=dev),
                                 torch.tensor(pos, device=dev), torch.tensor(bt, dtype=dt, device=dev),
                                 torch.tensor(slots, dtype=dt, device=dev), s_page=s_dev[0], s_mark=s_dev[1],
                                 s_run=s_dev[2], s_pp=s_dev[3], image_token_id=IMG, page_token_id=PG,
                                 per_page=per_page, block_size=bs, num_decode_tokens=nd,
                                 gen_start=None if gen is None else torch.tensor(gen, device=dev))
        np.testing.assert_array_equal(got.cpu().numpy(), exp, err_msg=f"step {k}")
        for name, a, b in zip(("img_page", "marker", "run", "pp"), s_dev,
                              (st.img_page, st.marker_cum, st.img_run, st.prompt_pages)):
            np.testing.assert_array_equal(a.cpu().numpy(), b, err_msg=f"step {k} {name}")


def test_coord_step_matches_oracle(dev):
    print("coord step", flush=True)
    rng = np.random.default_rng(23)
    docs = [_doc(rng, int(rng.integers(1, 5))) for _ in range(3)]
    R, pages = len(docs), 48
    cs = P.CoordState(R + 2, pages)
    rows = np.array([3, 0, 2])
    st_m = torch.zeros(R + 2, dtype=torch.int32, device=dev)
    st_p = torch.zeros(R + 2, dtype=torch.int32, device=dev)
    cnt = torch.zeros(R + 2, pages, dtype=torch.int32, device=dev)
    gen = np.array([len(d) - 30 for d in docs])
    from srswa import page_ops
    for k, (pos, lens) in enumerate(_steps(rng, docs, max_chunk=500)):
        ids, _, qs = _flat(docs, pos, lens, np.zeros((R, 1024), np.int64), 16)
        tok, page, mk, pp = P.coord_step(ids, qs, np.array(pos), rows, cs, IMG, PG, gen_start=gen)
        g = page_ops.coord_step(torch.tensor(ids, device=dev), torch.tensor(qs, device=dev),
                                torch.tensor(pos, device=dev), torch.tensor(rows, device=dev), st_marker=st_m,
                                st_pp=st_p, cnt=cnt, image_token_id=IMG, page_token_id=PG,
                                gen_start=torch.tensor(gen, device=dev), with_carry=True)
        for name, a, b in zip(("tok", "page", "marker", "pp"), g, (tok, page, mk, pp)):
            np.testing.assert_array_equal(a.cpu().numpy(), b, err_msg=f"step {k} {name}")
        np.testing.assert_array_equal(st_m.cpu().numpy(), cs.st_marker)
        np.testing.assert_array_equal(st_p.cpu().numpy(), cs.st_pp)
        np.testing.assert_array_equal(cnt.cpu().numpy(), cs.cnt)


def _prompts(rng, B, mark=0.8):
    docs = [_doc(rng, int(rng.integers(1, 6)), img=(100, 600), mark=mark) for _ in range(B)]
    L = max(len(d) for d in docs)
    return np.stack([np.concatenate([d, np.full(L - len(d), 5)]) for d in docs]), L


@pytest.mark.parametrize("scope", [True, False])
def test_page_aware_ids_matches_oracle(dev, scope):
    rng = np.random.default_rng(25)
    ids, L = _prompts(rng, 3)
    ids[2, :] = 7                                          # a row without images
    klen = L + 11                                          # padded with -1 past the ids
    from srswa import page_ops
    img, ip, qp, counts = page_ops.page_aware_ids(torch.tensor(ids, device=dev), image_token_id=IMG,
                                                  page_token_id=PG, key_length=klen, per_page=273,
                                                  page_scope_prefill=scope)
    e_img, e_ip, e_qp = P.page_aware_ids(ids, IMG, PG, klen, 273, page_scope_prefill=scope)
    np.testing.assert_array_equal(img.cpu().numpy(), e_img)
    np.testing.assert_array_equal(ip.cpu().numpy(), e_ip)
    np.testing.assert_array_equal(qp.cpu().numpy(), e_qp)
    np.testing.assert_array_equal(counts.cpu().numpy()[:, 0], (e_qp >= 0).sum(1))
    np.testing.assert_array_equal(counts.cpu().numpy()[:, 1], e_img.sum(1))


def test_page_rope_pos_matches_oracle(dev):
    rng = np.random.default_rng(27)
    ids, L = _prompts(rng, 3, mark=1.0)
    from srswa import page_ops
    page, pre, info = page_ops.page_rope_pos(torch.tensor(ids, device=dev), image_token_id=IMG, page_token_id=PG,
                                             key_length=L)
    n_pg = int(info[:, 1].max()) + 1
    tok, pf = page_ops.page_rope_tok(page, pre, n_pg)
    e_tok, e_page, e_pf = P.page_rope_pos(ids, IMG, PG, L)
    np.testing.assert_array_equal(page.cpu().numpy(), e_page)
    np.testing.assert_array_equal(tok.cpu().numpy(), e_tok)
    np.testing.assert_array_equal(pf.cpu().numpy(), e_pf)


def test_dropins_on_duck_typed_states(dev):
    """The drop-in ``step`` methods and HF builders through duck-typed owners:
    the backend's state objects (their tensors, _ensure, _rows, _rewind,
    _snapshot) and an indexer with the reference's fields."""
    from srswa import page_isolation as PI
    from srswa.unlimited_dash_ops import page_state as PS
    rng = np.random.default_rng(29)
    docs = [_doc(rng, 2) for _ in range(2)]
    bs, n_slots = 16, 4096
    nblk = max(-(-len(d) // bs) for d in docs) + 1
    bt = np.arange(2 * nblk).reshape(2, nblk)
    ids, slots, qs = _flat(docs, [0, 0], [len(d) for d in docs], bt, bs)
    T = len(ids)

    class _PS:
        block_size, image_token_id, page_token_id, per_page_image_tokens = bs, IMG, PG, 273

        def _ensure(self, n, device):
            if not hasattr(self, "_slot_img_page"):
                self._slot_img_page = torch.full((n,), -1, dtype=torch.int32, device=device)
                self._slot_marker_cum = torch.zeros(n, dtype=torch.int32, device=device)
                self._slot_img_run = torch.zeros(n, dtype=torch.int32, device=device)
                self._slot_prompt_pages = torch.zeros(n, dtype=torch.int32, device=device)

    layout = types.SimpleNamespace(num_tokens=T, num_reqs=2, q_start=torch.tensor(qs, device=dev),
                                   start_pos=torch.zeros(2, dtype=torch.int64, device=dev),
                                   block_table=torch.tensor(bt, device=dev), num_decode_tokens=0, gen_start=None,
                                   req_of_token=torch.tensor(np.repeat([0, 1], [len(d) for d in docs]), device=dev))
    ps = _PS()
    q = PS.page_isolation_step(ps, torch.tensor(ids, device=dev), layout, torch.tensor(slots, device=dev), n_slots)
    st = P.SlotState(n_slots)
    exp = P.page_step(ids, qs, np.zeros(2, np.int64), bt, slots, st, IMG, PG, 273, bs)
    np.testing.assert_array_equal(q.cpu().numpy(), exp)
    assert PS.page_isolation_step(ps, torch.tensor(ids, device=dev), layout, torch.tensor(slots, device=dev),
                                  n_slots).data_ptr() == q.data_ptr()          # a fixed-address output

    class _CS:
        image_token_id, page_token_id, max_pages = IMG, PG, 32

        def _ensure(self, device):
            if not hasattr(self, "st_marker"):
                self.st_marker = torch.zeros(3, dtype=torch.int32, device=device)
                self.st_pp = torch.zeros(3, dtype=torch.int32, device=device)
                self.cnt = torch.zeros(3, 32, dtype=torch.int32, device=device)

        def _rows(self, lay):
            return torch.tensor([1, 2], device=dev)

        def _rewind_rejected(self, lay, row):
            self.rewound = True

        def _snapshot(self, *args):
            self.snap = args

    cs = _CS()
    tok, page = PS.coord_step(cs, torch.tensor(ids, device=dev), layout)
    ocs = P.CoordState(3, 32)
    e_tok, e_page, e_mk, e_pp = P.coord_step(ids, qs, np.zeros(2, np.int64), np.array([1, 2]), ocs, IMG, PG)
    np.testing.assert_array_equal(tok.cpu().numpy(), e_tok)
    np.testing.assert_array_equal(page.cpu().numpy(), e_page)
    assert cs.rewound and len(cs.snap) == 12
    np.testing.assert_array_equal(cs.snap[6].cpu().numpy(), e_mk)              # marker_cum to the snapshot
    np.testing.assert_array_equal(cs.snap[7].cpu().numpy(), e_pp)              # pp
    np.testing.assert_array_equal(cs.snap[8].cpu().numpy(), e_page)            # the page buckets
    np.testing.assert_array_equal(cs.snap[10].cpu().numpy(), np.zeros(2))      # st_pp as before the step

    ind = types.SimpleNamespace(q_proj=types.SimpleNamespace(weight=torch.zeros(1, device=dev)),
                                per_page_image_tokens=273, image_token_id=IMG, page_token_id=PG, rope_page_span=0,
                                _page_rope_bail=lambda reason: ("bail", reason))
    pids, L = _prompts(rng, 2, mark=1.0)
    got = PI.build_page_aware_ids(ind, torch.tensor(pids), IMG, PG, L)
    want = P.page_aware_ids(pids, IMG, PG, L, 273)
    for g_, w_ in zip(got, want):
        np.testing.assert_array_equal(g_.cpu().numpy(), w_)
    tp = PI.build_page_rope_pos(ind, torch.tensor(pids), L)
    e_tok, e_page, e_pf = P.page_rope_pos(pids, IMG, PG, L)
    np.testing.assert_array_equal(tp[0].cpu().numpy(), e_tok)
    np.testing.assert_array_equal(tp[1].cpu().numpy(), e_page)
    np.testing.assert_array_equal(ind._page_rope_meta["pf_cnt"].cpu().numpy(), e_pf)
    assert PI.build_page_rope_pos(ind, torch.full((1, 30), 7), 30)[0] == "bail"
