"""Pins of the gather-KL oracle (oracle/kl_oracle.py)."""

import pytest
import torch

from oracle import kl_oracle as K


def _case(seed, B=2, HI=1, G=3, HKV=1, T=40, Sk=200, d=16, Dh=16, bs=16, topk=4, lw=24, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    HQ = HI * G
    q_idx = torch.randn(B, HI, T, d, generator=g, dtype=dtype)
    idx_k = torch.randn(B, Sk, d, generator=g, dtype=dtype)
    q_main = torch.randn(B, HQ, T, Dh, generator=g, dtype=dtype)
    k_main = torch.randn(B, HKV, Sk, Dh, generator=g, dtype=dtype)
    pos = (torch.arange(T) + (Sk - T)).expand(B, T).clone()
    nblk = -(-Sk // bs)
    sel = torch.stack([torch.stack([torch.stack([torch.randperm(nblk, generator=g)[:topk] for _ in range(T)])
                                    for _ in range(HI)]) for _ in range(B)]).to(torch.int32)
    sel[:, :, ::5, -1] = -1                       # empty slots
    sel[:, :, :2] = -1                             # rows with nothing selected
    sel[:, :, 2, :] = nblk - 1                     # a row whose only block lies past it
    return q_idx, idx_k, q_main, k_main, sel, pos


def _gather_form(q_idx, idx_k, q_main, k_main, sel, pos, bs, lw, scaling, rdt):
    """The n_idx_heads == 1 branch of select_and_kl_loss
    (HF/_sparse_base_impl.py:3413-3478) restated: gather each row's selected
    keys, softmax over them only."""
    B, HI, T, topk = sel.shape
    assert HI == 1
    Sk = idx_k.shape[1]
    HQ, HKV = q_main.shape[1], k_main.shape[1]
    rnd = (lambda x: x) if rdt is None else (lambda x: x.to(rdt).to(x.dtype))
    tok_raw = (sel.clamp_min(0).long().unsqueeze(-1) * bs + torch.arange(bs)).reshape(B, 1, T, topk * bs)
    local_start = (pos - (lw - 1)).clamp(min=0)
    keep = ((sel >= 0).unsqueeze(-1).expand(-1, -1, -1, -1, bs).reshape(B, 1, T, topk * bs)
            & (tok_raw < Sk) & (tok_raw <= pos[:, None, :, None]) & (tok_raw < local_start[:, None, :, None]))
    tok = tok_raw.clamp(max=Sk - 1)[:, 0]                                        # [B, T, S_sel]
    k_sel = torch.stack([idx_k[b][tok[b]] for b in range(B)])                   # [B, T, S_sel, d]
    s = rnd(torch.einsum("btsd,btd->bts", k_sel, q_idx[:, 0]))[:, None]
    log_q = torch.log_softmax(s.masked_fill(~keep, -1e9), -1)
    p = 0
    for h in range(HQ):
        km = torch.stack([k_main[b, h // (HQ // HKV)][tok[b]] for b in range(B)])
        sh = rnd(torch.einsum("btsd,btd->bts", km, q_main[:, h]))[:, None] * scaling
        p = p + torch.softmax(sh.masked_fill(~keep, -1e9), -1)
    p = p / HQ
    term = torch.where(keep, p * (torch.log(p.clamp_min(1e-12)) - log_q), torch.zeros_like(p))
    return term.sum(-1), keep.any(-1)


@pytest.mark.parametrize("rdt", [None, torch.bfloat16])
def test_dense_equals_gather_form(rdt):
    q_idx, idx_k, q_main, k_main, sel, pos = _case(1, G=4, HKV=2)
    kl, valid = K.gather_kl_dense(q_idx, idx_k, q_main, k_main, sel, pos, block_size=16, local_window=24,
                                  scaling=0.3, round_dtype=rdt)
    kl2, valid2 = _gather_form(q_idx, idx_k, q_main, k_main, sel, pos, 16, 24, 0.3, rdt)
    assert torch.equal(valid, valid2)
    assert (kl - kl2).abs().max().item() < 1e-10
    assert valid.any() and (~valid).any()
    assert (kl >= -1e-12).all()                          # KL(p || q) >= 0
    assert (kl[~valid] == 0).all()


def test_zero_when_student_is_the_teacher():
    q_idx, idx_k, q_main, k_main, sel, pos = _case(2, G=1, HKV=1)
    kl, valid = K.gather_kl_dense(q_main.clone(), k_main[:, 0].clone(), q_main, k_main, sel, pos, block_size=16,
                                  local_window=24, scaling=1.0, round_dtype=None)
    assert valid.any() and kl.abs().max().item() < 1e-12


def test_multi_index_heads_group_mean():
    """HI = 2 index heads, each against the mean of its own 3 query heads."""
    q_idx, idx_k, q_main, k_main, sel, pos = _case(3, HI=2, G=3, HKV=2)
    kl, _ = K.gather_kl_dense(q_idx, idx_k, q_main, k_main, sel, pos, block_size=16, local_window=24, scaling=0.5,
                              round_dtype=None)
    # index head 1 alone, with its query heads 3..5 (kv heads 1 of 2: query head h -> kv h // 3)
    kl1, _ = K.gather_kl_dense(q_idx[:, 1:], idx_k, q_main[:, 3:], k_main[:, 1:], sel[:, 1:], pos, block_size=16,
                               local_window=24, scaling=0.5, round_dtype=None)
    assert (kl[:, 1:] - kl1).abs().max().item() < 1e-12


def test_gradcheck_student_path():
    q_idx, idx_k, q_main, k_main, sel, pos = _case(4, B=1, T=12, Sk=64, d=6, Dh=5, bs=8, topk=3, lw=8)
    q_idx.requires_grad_()
    idx_k.requires_grad_()

    def f(q, k):
        kl, valid = K.gather_kl_dense(q, k, q_main, k_main, sel, pos, block_size=8, local_window=8, scaling=0.7,
                                      round_dtype=None)
        return K.kl_loss(kl, valid)

    assert torch.autograd.gradcheck(f, (q_idx, idx_k), eps=1e-6, atol=1e-6)


def test_student_gradient_closed_form():
    """d kl / d s_j = softmax(s)_j - p_j on kept keys: the backward the
    kernels implement, checked against autograd of the dense form."""
    q_idx, idx_k, q_main, k_main, sel, pos = _case(5, B=1, T=16, Sk=96, d=8, Dh=8, bs=8, topk=3, lw=8)
    q_idx.requires_grad_()
    kl, valid = K.gather_kl_dense(q_idx, idx_k, q_main, k_main, sel, pos, block_size=8, local_window=8,
                                  scaling=0.6, round_dtype=None)
    kl.sum().backward()
    keep = K.keep_mask(sel, pos, 96, 8, 8)
    s = torch.einsum("bhtd,bsd->bhts", q_idx.detach(), idx_k).masked_fill(~keep, K.NEG)
    sm = torch.softmax(s, -1)
    p = 0
    for h in range(q_main.shape[1]):
        p = p + torch.softmax((torch.einsum("btd,bsd->bts", q_main[:, h], k_main[:, 0]) * 0.6)[:, None]
                              .masked_fill(~keep, K.NEG), -1)
    p = p / q_main.shape[1]
    ds = torch.where(keep, sm - p, torch.zeros_like(p))
    dq = torch.einsum("bhts,bsd->bhtd", ds, idx_k)
    assert (dq - q_idx.grad).abs().max().item() < 1e-10
