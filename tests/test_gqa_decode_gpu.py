"""GQA decode: the heads of one kv head that read one id row are scored by one
workgroup (each K / V row loaded once for the group).

Every per-head operation keeps the per-head kernel's order, so a GQA call must
equal, bit for bit, the same call on caches (and ids) expanded to one kv head
per query head, which runs the per-head kernel; both are also checked against
the oracle (bf16 / fp16 within 2e-2).  Cases cover groups of 4 and 2 (and a
group of 6 kv-sharing heads served 2 at a time), a group that cannot be split
(3: per-head kernel), one id row shared by all heads, split-K records and the
single-workgroup path, bias / valid / repeated ids / -1 slots, two decode
queries, and the paged decode with bf16 and fp8 caches."""

import math

import pytest
import torch

from oracle import srswa_oracle as O
import srswa

pytestmark = pytest.mark.gpu
BF16_TOL = 2e-2


def _expand_heads(t, G, dim):
    return t.repeat_interleave(G, dim=dim).contiguous()


# (HQ, HKV, HI): HI index heads (ids shared by HQ / HI query heads)
GATHER_CASES = {
    "g4": (8, 2, 2),
    "g2": (4, 2, 2),
    "g6_in_pairs": (12, 2, 2),
    "g3_per_head": (6, 2, 2),
    "g4_one_id_row": (8, 2, 1),
    "ids_per_query_head": (8, 2, 8),
}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("LW", [64, 512])
@pytest.mark.parametrize("case", list(GATHER_CASES))
def test_gqa_gather_decode_equals_expanded(dev, case, LW, dtype):
    HQ, HKV, HI = GATHER_CASES[case]
    print(f"gqa gather {case} LW={LW} {dtype}", flush=True)
    g = torch.Generator().manual_seed(10 * list(GATHER_CASES).index(case) + LW)
    B, Lq, D, L, BS, K = 3, 2, 128, 4096, 64, 6 if LW == 512 else 2
    G = HQ // HKV
    q = torch.randn(B, Lq, HQ, D, generator=g).to(dtype)
    kc = torch.randn(B, L, HKV, D, generator=g).to(dtype)
    vc = torch.randn(B, L, HKV, D, generator=g).to(dtype)
    q_pos = torch.tensor([[L - 2, L - 1], [2000, 2001], [700, 701]])
    kv_len = torch.tensor([L, 2002, 702])
    nblk = L // BS
    idx = torch.randint(0, nblk, (B, HI, Lq, K), generator=g)
    idx[:, :, :, 1] = idx[:, :, :, 0]                           # a repeat
    idx[0, :, 0, K - 1] = -1                                    # an empty slot
    bias = torch.randn(B, HI, Lq, K, generator=g)
    valid = torch.rand(B, HI, Lq, K, generator=g) > 0.2
    scale = 1 / math.sqrt(D)
    kw = dict(block_size=BS, local_window=LW, scale=scale, return_lse=True)

    def run(q_, k_, v_, i_, b_, v2_):
        launch, out, lse = srswa.ops.prepare_gather_decode(
            q_.to(dev), k_.to(dev), v_.to(dev), i_.to(dev), q_pos.to(dev), bias=b_.to(dev), valid=v2_.to(dev),
            kv_len=kv_len.to(dev), **kw)
        launch()
        return out.cpu(), lse.cpu()

    out, lse = run(q, kc, vc, idx, bias, valid)
    # the same attention with one kv head (and one id row) per query head
    IG = HQ // HI
    ke, ve = _expand_heads(kc, G, 2), _expand_heads(vc, G, 2)
    ie, be, vae = (_expand_heads(t, IG, 1) for t in (idx, bias, valid))
    out_e, lse_e = run(q, ke, ve, ie, be, vae)
    assert torch.equal(out, out_e), (out.float() - out_e.float()).abs().max()
    assert torch.equal(lse, lse_e)
    ref = O.decode_attend(q.transpose(1, 2).double(), ke.transpose(1, 2).double(), ve.transpose(1, 2).double(),
                          ie, be.double(), vae, q_pos, BS, LW, scale)
    for b in range(B):                                          # kv_len clips the keys after it
        assert int(kv_len[b]) > int(q_pos[b, -1])
    err = (out.transpose(1, 2).double() - ref).abs().max().item()
    assert err <= BF16_TOL, err


@pytest.mark.parametrize("kv", [None, torch.float8_e4m3fn, torch.float8_e5m2fnuz])
def test_gqa_paged_decode_equals_expanded(dev, kv):
    print(f"gqa paged {kv}", flush=True)
    from srswa import unlimited_dash_ops as U
    g = torch.Generator().manual_seed(7)
    R, dql, HQ, HKV, D, page, nb, K, lb = 4, 2, 8, 2, 128, 64, 24, 5, 4
    G = HQ // HKV
    num_pages = R * nb + 3
    kc = torch.randn(num_pages, page, HKV, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(num_pages, page, HKV, D, generator=g).to(torch.bfloat16)
    if kv is not None:
        kc, vc = kc.to(kv), vc.to(kv)
    bt = torch.randperm(num_pages, generator=g)[:R * nb].view(R, nb).to(torch.int32)
    sl = torch.tensor([nb * page, nb * page - 37, 900, 300], dtype=torch.int32)
    q = torch.randn(R * dql, HQ, D, generator=g).to(torch.bfloat16)
    topk = torch.randint(0, nb, (HKV, R * dql, K), generator=g).to(torch.int32)
    topk[:, :, 2] = topk[:, :, 0]
    topk[1, 0, K - 1] = -1
    bias = torch.randn(HKV, R * dql, K, generator=g)
    scale = 1 / math.sqrt(D)

    def run(k_, v_, t_, b_, hkv):
        out = torch.empty(R * dql, HQ, D, dtype=torch.bfloat16, device=dev)
        U.dash_sparse_attn_decode(q.to(dev), k_.to(dev), v_.to(dev), t_.to(dev), b_.to(dev), bt.to(dev),
                                  sl.to(dev), hkv, scale, out, dql, local_blocks=lb, sparse_block_size=page)
        return out.cpu()

    out = run(kc, vc, topk, bias, HKV)
    ke = kc.view(torch.uint8).repeat_interleave(G, dim=2).view(kc.dtype) if kv is not None else _expand_heads(kc, G, 2)
    ve = vc.view(torch.uint8).repeat_interleave(G, dim=2).view(vc.dtype) if kv is not None else _expand_heads(vc, G, 2)
    out_e = run(ke, ve, _expand_heads(topk, G, 0), _expand_heads(bias, G, 0), HQ)
    assert torch.equal(out, out_e), (out.float() - out_e.float()).abs().max()
    ref = O.paged_decode_attend(q.double(), ke.float().double(), ve.float().double(), _expand_heads(topk, G, 0),
                                _expand_heads(bias, G, 0).double(), bt, sl, dql, lb, scale)
    err = (out.double() - ref).abs().max().item()
    assert err <= BF16_TOL, err
