"""Paged block-sparse prefill (srswa.unlimited_dash_ops.dash_sparse_attn, the
drop-in for the SGLang backend's K10 dash_sparse_attn) vs the CPU oracle
(``srswa_oracle.paged_prefill_attend``, K10's two passes query by query).

Bar: bf16 / fp16 outputs max-abs <= 2e-2 beyond the output format's half-ulp
(tests/tolerance.py) against fp64 on the same rounded inputs.  Inputs follow
the router's contract: per-kv-head ids packed at the front (ascending,
unique, -1 after), optional fp32 slot biases.  fp8 caches of the four torch
fp8 formats are compared against the oracle on their exact values."""

import math

import pytest
import torch

from oracle import srswa_oracle as O
from srswa import unlimited_dash_ops as U
from tolerance import assert_close_lowp

pytestmark = pytest.mark.gpu


def _case(seed, q_lens, ctx, page, Hkv, G, D, S, dtype, nb_extra=3, bias=True, kv=None):
    g = torch.Generator().manual_seed(seed)
    R = len(q_lens)
    seq = [c + q for c, q in zip(ctx, q_lens)]
    nb = max(-(-s // page) for s in seq) + nb_extra
    npages = R * nb + 4
    kc = torch.randn(npages, page, Hkv, D, generator=g).to(kv or dtype)
    vc = torch.randn(npages, page, Hkv, D, generator=g).to(kv or dtype)
    bt = torch.randperm(npages, generator=g)[:R * nb].view(R, nb).to(torch.int32)
    cu = [0]
    for ql in q_lens:
        cu.append(cu[-1] + ql)
    total = cu[-1]
    H = Hkv * G
    q = torch.randn(total, H, D, generator=g).to(dtype)
    topk = torch.full((Hkv, total, S), -1, dtype=torch.int32)
    for r in range(R):
        for n in range(cu[r], cu[r + 1]):
            qp = ctx[r] + n - cu[r]
            live = -(-seq[r] // page)
            for kh in range(Hkv):
                k = int(torch.randint(0, S + 1, (1,), generator=g))
                ids = torch.randperm(max(live, 1), generator=g)[:k].sort().values
                topk[kh, n, :len(ids)] = ids.to(torch.int32)
            _ = qp
    bsl = torch.randn(Hkv, total, S, generator=g) if bias else None
    return dict(q=q, kc=kc, vc=vc, bt=bt, cu=torch.tensor(cu, dtype=torch.int32),
                seq=torch.tensor(seq, dtype=torch.int32), ctx=torch.tensor(ctx, dtype=torch.int32),
                topk=topk, bias=bsl, max_q=max(q_lens), Hkv=Hkv, page=page)


CASES = {
    "bf16_p64_lb8": dict(q_lens=[70, 1, 130], ctx=[900, 40, 0], page=64, Hkv=2, G=2, D=128, S=8,
                         dtype=torch.bfloat16, lb=8),
    "bf16_p32_lb4_nobias": dict(q_lens=[64, 33], ctx=[500, 1200], page=32, Hkv=1, G=3, D=128, S=6,
                                dtype=torch.bfloat16, lb=4, bias=False),
    "fp16_p16_d64": dict(q_lens=[90, 17, 5], ctx=[300, 0, 77], page=16, Hkv=2, G=1, D=64, S=5,
                         dtype=torch.float16, lb=6),
    "bf16_p128_no_window": dict(q_lens=[40, 65], ctx=[600, 200], page=128, Hkv=2, G=2, D=128, S=4,
                                dtype=torch.bfloat16, lb=0),
    "fp8_e4m3fn_p64": dict(q_lens=[70, 1, 130], ctx=[900, 40, 0], page=64, Hkv=2, G=2, D=128, S=8,
                           dtype=torch.bfloat16, lb=8, kv=torch.float8_e4m3fn),
    "fp8_e5m2_p32_nobias": dict(q_lens=[64, 33], ctx=[500, 1200], page=32, Hkv=1, G=3, D=128, S=6,
                                dtype=torch.bfloat16, lb=4, bias=False, kv=torch.float8_e5m2),
    "fp8_e4m3fnuz_fp16_d64": dict(q_lens=[90, 17, 5], ctx=[300, 0, 77], page=16, Hkv=2, G=1, D=64, S=5,
                                  dtype=torch.float16, lb=6, kv=torch.float8_e4m3fnuz),
    "fp8_e5m2fnuz_p128": dict(q_lens=[40, 65], ctx=[600, 200], page=128, Hkv=2, G=2, D=128, S=4,
                              dtype=torch.bfloat16, lb=2, kv=torch.float8_e5m2fnuz),
}


@pytest.mark.parametrize("name", list(CASES))
def test_dash_sparse_attn_matches_oracle(dev, name):
    kw = dict(CASES[name])
    lb = kw.pop("lb")
    c = _case(list(CASES).index(name) + 40, **kw)
    scale = 1 / math.sqrt(kw["D"])
    out = torch.full(c["q"].shape, float("nan"), dtype=c["q"].dtype, device=dev)
    print(f"dash_sparse_attn {name}", flush=True)
    U.dash_sparse_attn(c["q"].to(dev), c["kc"].to(dev), c["vc"].to(dev), c["topk"].to(dev),
                       None if c["bias"] is None else c["bias"].to(dev), c["bt"].to(dev), c["cu"].to(dev),
                       c["seq"].to(dev), c["ctx"].to(dev), c["max_q"], c["Hkv"], scale, out, local_blocks=lb,
                       sparse_block_size=c["page"])
    ref = O.paged_prefill_attend(c["q"].double(), c["kc"].double(), c["vc"].double(), c["topk"].long(),
                                 None if c["bias"] is None else c["bias"].double(), c["bt"].long(), c["cu"].tolist(),
                                 c["seq"].tolist(), c["ctx"].tolist(), lb, scale)
    assert_close_lowp(out.cpu(), ref, kw["dtype"], 2e-2, f"dash_sparse_attn {name}")


def test_dash_sparse_attn_head_expanded_ids(dev):
    """The backend's call: one router row expanded over the kv heads with
    stride 0 (unlimited_ocr_v2_backend.py:1421-1422), read in place."""
    c = _case(77, [50, 20], [300, 64], 64, 1, 2, 128, 8, torch.bfloat16)
    Hkv = 4
    g = torch.Generator().manual_seed(5)
    kc = torch.randn(c["kc"].shape[0], 64, Hkv, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(c["vc"].shape[0], 64, Hkv, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(c["q"].shape[0], Hkv * 2, 128, generator=g).to(torch.bfloat16)
    ids = c["topk"][0].to(dev)
    bias = c["bias"][0].to(dev)
    di = ids.unsqueeze(0).expand(Hkv, -1, -1)
    db = bias.unsqueeze(0).expand(Hkv, -1, -1)
    out = torch.empty(q.shape, dtype=q.dtype, device=dev)
    U.dash_sparse_attn(q.to(dev), kc.to(dev), vc.to(dev), di, db, c["bt"].to(dev), c["cu"].to(dev), c["seq"].to(dev),
                       c["ctx"].to(dev), c["max_q"], Hkv, 0.088, out, local_blocks=8, sparse_block_size=64)
    ref = O.paged_prefill_attend(q.double(), kc.double(), vc.double(), di.cpu().long(), db.cpu().double(),
                                 c["bt"].long(), c["cu"].tolist(), c["seq"].tolist(), c["ctx"].tolist(), 8, 0.088)
    assert_close_lowp(out.cpu(), ref, torch.bfloat16, 2e-2, "dash_sparse_attn head-expanded ids")
