"""Paged decode (srswa_gather_decode_paged, the serving cache layout of
dash_sparse_attn_decode) vs the CPU oracle ``paged_decode_attend``: pages in
random order, ragged sequence lengths, 1 and 2 decode queries per request,
GQA, page sizes 16..128, no window (local_blocks 0) and the widest one (63),
-1 padding, repeated ids, bias and no bias, and fp8 caches of the four
torch fp8 formats under bf16 / fp16 queries (the oracle reads the caches'
exact fp8 values); bf16 within 2e-2 (beyond output rounding), fp32 within 1e-5
relative (max-abs error / max-abs reference)."""

import math

import pytest
import torch

from oracle import srswa_oracle as O
from tolerance import assert_close_lowp

pytestmark = pytest.mark.gpu


def _case(seed, R, dql, H, Hkv, D, page, nb, K, lb, dtype, with_bias, kv=None):
    g = torch.Generator().manual_seed(seed)
    npages = R * nb + 5
    q = torch.randn(R * dql, H, D, generator=g).to(dtype)
    kc = torch.randn(npages, page, Hkv, D, generator=g).to(kv or dtype)
    vc = torch.randn(npages, page, Hkv, D, generator=g).to(kv or dtype)
    bt = torch.randperm(npages, generator=g)[:R * nb].view(R, nb).to(torch.int32)
    sl = torch.randint(max(dql, page), nb * page + 1, (R,), generator=g).to(torch.int32)
    sl[0] = nb * page                                     # a full table
    topk = torch.randint(-1, nb, (Hkv, R * dql, K), generator=g).to(torch.int32)
    topk[:, 0, 1] = topk[:, 0, 0]                        # a repeated id
    if K > 64:
        topk[:, :, 70] = topk[:, :, 2]                   # a wide slot repeating an early one
        topk[:, :, K - 1] = topk[:, :, 90]               # two wide slots holding one id
    bias = torch.randn(Hkv, R * dql, K, generator=g) if with_bias else None
    return q, kc, vc, topk, bias, bt, sl


CASES = {
    "bf16_p64": dict(R=5, dql=1, H=10, Hkv=10, D=128, page=64, nb=24, K=8, lb=8, dtype=torch.bfloat16, with_bias=True),
    "bf16_p32_gqa_dql2": dict(R=3, dql=2, H=8, Hkv=2, D=128, page=32, nb=40, K=12, lb=4, dtype=torch.bfloat16,
                             with_bias=True),
    "bf16_p16_nowin": dict(R=4, dql=1, H=4, Hkv=4, D=128, page=16, nb=30, K=6, lb=0, dtype=torch.bfloat16,
                          with_bias=False),
    "bf16_d64_p128": dict(R=2, dql=1, H=4, Hkv=1, D=64, page=128, nb=10, K=4, lb=2, dtype=torch.bfloat16,
                         with_bias=True),
    "fp32_p32": dict(R=3, dql=1, H=4, Hkv=2, D=128, page=32, nb=20, K=5, lb=3, dtype=torch.float32,
                    with_bias=True),
    # the widest window (63 pages): the wrapped first unit reads its last keys
    # from the window's 64th page
    "bf16_p16_lb63": dict(R=3, dql=2, H=4, Hkv=4, D=128, page=16, nb=80, K=4, lb=63, dtype=torch.bfloat16,
                         with_bias=True),
    # fp8 caches (USE_FP8 of the reference's kernels): every format, converted exactly to q's dtype
    "fp8_e4m3fn_p64": dict(R=5, dql=1, H=10, Hkv=10, D=128, page=64, nb=24, K=8, lb=8, dtype=torch.bfloat16,
                           with_bias=True, kv=torch.float8_e4m3fn),
    "fp8_e5m2_p32_gqa_dql2": dict(R=3, dql=2, H=8, Hkv=2, D=128, page=32, nb=40, K=12, lb=4, dtype=torch.bfloat16,
                                  with_bias=True, kv=torch.float8_e5m2),
    "fp8_e4m3fnuz_p16_fp16": dict(R=4, dql=1, H=4, Hkv=4, D=128, page=16, nb=30, K=6, lb=2, dtype=torch.float16,
                                  with_bias=False, kv=torch.float8_e4m3fnuz),
    "fp8_e5m2fnuz_d64_p128": dict(R=2, dql=1, H=4, Hkv=1, D=64, page=128, nb=10, K=4, lb=2, dtype=torch.bfloat16,
                                  with_bias=True, kv=torch.float8_e5m2fnuz),
    # rows of more than 64 slots (the kernel's wide-slot branch): repeats, -1
    # slots and ids of blocks past seq_len among 96 / 200 slots
    "bf16_p16_wide96_dql2": dict(R=3, dql=2, H=8, Hkv=2, D=128, page=16, nb=300, K=96, lb=4,
                                 dtype=torch.bfloat16, with_bias=True),
    "bf16_p32_wide200": dict(R=2, dql=1, H=4, Hkv=4, D=128, page=32, nb=260, K=200, lb=8,
                             dtype=torch.bfloat16, with_bias=True),
    "fp32_p16_wide200_nobias": dict(R=2, dql=1, H=4, Hkv=2, D=128, page=16, nb=240, K=200, lb=2,
                                    dtype=torch.float32, with_bias=False),
}


@pytest.mark.parametrize("name", list(CASES))
def test_paged_decode_matches_oracle(dev, name):
    from srswa import unlimited_dash_ops as U

    c = CASES[name]
    q, kc, vc, topk, bias, bt, sl = _case(40 + list(CASES).index(name), **c)
    scale = 1 / math.sqrt(c["D"])
    out = torch.empty(q.shape, dtype=q.dtype, device=dev)
    U.dash_sparse_attn_decode(q.to(dev), kc.to(dev), vc.to(dev), topk.to(dev),
                              None if bias is None else bias.to(dev), bt.to(dev), sl.to(dev), c["Hkv"], scale,
                              out, c["dql"], local_blocks=c["lb"], sparse_block_size=c["page"])
    ref = O.paged_decode_attend(q.double(), kc.double(), vc.double(), topk, None if bias is None else bias.double(),
                                bt, sl, c["dql"], c["lb"], scale)
    if c["dtype"] == torch.float32:
        rel = ((out.cpu().double() - ref).abs().max() / ref.abs().max()).item()   # max-abs err / max-abs ref
        assert rel <= 1e-5, rel
    else:
        assert_close_lowp(out.cpu(), ref, c["dtype"], 2e-2, name)


@pytest.mark.parametrize("with_bias", [True, False])
def test_paged_decode_head_expanded_ids(dev, with_bias):
    """One id / bias row shared by every kv head, passed as a stride-0 view
    (the DASH step's topi[None].expand(H, ...)): the oracle on the expanded
    tensors, and bit-identical to the contiguous copy."""
    from srswa import unlimited_dash_ops as U

    c = dict(CASES["bf16_p64"], with_bias=with_bias)
    q, kc, vc, topk, bias, bt, sl = _case(77, **c)
    Hkv = c["Hkv"]
    ids = topk[0][None].expand(Hkv, -1, -1)
    bi = None if bias is None else bias[0][None].expand(Hkv, -1, -1)
    scale = 1 / math.sqrt(c["D"])
    outs = []
    for t, b in ((ids.to(dev), None if bi is None else bi.to(dev)),
                 (ids.contiguous().to(dev), None if bi is None else bi.contiguous().to(dev))):
        out = torch.empty(q.shape, dtype=q.dtype, device=dev)
        U.dash_sparse_attn_decode(q.to(dev), kc.to(dev), vc.to(dev), t, b, bt.to(dev), sl.to(dev), Hkv, scale, out,
                                  c["dql"], local_blocks=c["lb"], sparse_block_size=c["page"])
        outs.append(out)
    assert outs[0].is_contiguous()
    assert torch.equal(outs[0], outs[1])
    ref = O.paged_decode_attend(q.double(), kc.double(), vc.double(), ids.contiguous(),
                                None if bi is None else bi.contiguous().double(), bt, sl, c["dql"], c["lb"], scale)
    assert_close_lowp(outs[0].cpu(), ref, c["dtype"], 2e-2, "expanded ids")


@pytest.mark.parametrize("qdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fmt", ["float8_e4m3fn", "float8_e4m3fnuz", "float8_e5m2", "float8_e5m2fnuz"])
def test_fp8_cache_every_byte_exact(dev, fmt, qdt):
    """Every byte value of the fp8 format, NaN and infinity codes included,
    through both paged kernels: each request holds one key, so its output is
    its V row converted to q's dtype, which must equal torch's conversion
    exactly (the decode and the K10 prefill, bf16 and fp16 queries)."""
    from srswa import unlimited_dash_ops as U
    print(f"fp8 bytes {fmt} {qdt}", flush=True)
    dt = getattr(torch, fmt)
    R, page, D = 2, 16, 128
    kc = torch.zeros(R, page, 1, D, dtype=torch.uint8)               # K = +0 (code 0 in every format)
    vc = torch.zeros(R, page, 1, D, dtype=torch.uint8)
    vc[0, 0, 0] = torch.arange(128, dtype=torch.uint8)
    vc[1, 0, 0] = torch.arange(128, 256, dtype=torch.uint8)
    kc, vc = kc.view(dt), vc.view(dt)
    want = vc[:, 0, 0].to(torch.float32).to(qdt)                    # [R, D]
    bt = torch.arange(R, dtype=torch.int32).view(R, 1)
    sl = torch.ones(R, dtype=torch.int32)
    q = torch.randn(R, 1, D).to(qdt)
    topk = torch.full((1, R, 4), -1, dtype=torch.int32)

    def same(got, what):
        # equal values (the sign of a zero aside: 0 + 1 * (-0) is +0 in the
        # kernels' accumulators as in the reference's), NaN where NaN
        g, w = got.view(R, D).cpu().float(), want.float()
        ok = (g == w) | (torch.isnan(g) & torch.isnan(w))
        assert ok.all(), (what, fmt, int((~ok).sum()))

    out = torch.empty(R, 1, D, dtype=qdt, device=dev)
    U.dash_sparse_attn_decode(q.to(dev), kc.to(dev), vc.to(dev), topk.to(dev), None, bt.to(dev), sl.to(dev), 1,
                              0.1, out, 1, local_blocks=1, sparse_block_size=page)
    same(out, "decode")
    out2 = torch.empty(R, 1, D, dtype=qdt, device=dev)
    cu = torch.arange(R + 1, dtype=torch.int32)
    U.dash_sparse_attn(q.to(dev), kc.to(dev), vc.to(dev), topk.to(dev), None, bt.to(dev), cu.to(dev), sl.to(dev),
                       torch.zeros(R, dtype=torch.int32).to(dev), 1, 1, 0.1, out2, local_blocks=1,
                       sparse_block_size=page)
    same(out2, "prefill")
