"""The reference-signature drop-in modules (srswa.sparse_gather_triton,
srswa.sparse_gather_e2e_triton) on the GPU: same call signatures, layouts,
None-fallback gates and results as the reference wrappers."""

import math

import pytest
import torch

from oracle import srswa_oracle as O
from parity_report import compare_selection, report
import srswa
from srswa import sparse_gather_e2e_triton as E2E
from srswa import sparse_gather_triton as SG

pytestmark = pytest.mark.gpu


def test_gather_attention_reference_layout_and_gates(dev):
    g = torch.Generator().manual_seed(1)
    B, H, T, D, bs, lw = 2, 4, 200, 128, 32, 96
    q = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    bi = torch.randint(-1, T // bs, (B, 1, T, 4), generator=g)
    pos = torch.arange(T)[None].expand(B, -1)
    out = SG.triton_gather_attention(q.to(dev), k.to(dev), v.to(dev), bi.to(dev), pos.to(dev), None,
                                     bs, 1 / math.sqrt(D), local_window=lw)
    assert out.shape == (B, H, T, D)
    ref, _ = O.gather_attention(q.double(), k.double(), v.double(), bi, pos, bs, 1 / math.sqrt(D), lw)
    assert (out.cpu().double() - ref).abs().max().item() <= 2e-2
    # reference gates -> None
    m = torch.zeros(B, 1, T, T, device=dev)
    assert SG.triton_gather_attention(q.to(dev), k.to(dev), v.to(dev), bi.to(dev), pos.to(dev), m, bs, 0.1) is None
    assert SG.triton_gather_attention(q.to(dev), k.to(dev), v.to(dev), bi.to(dev), None, None, bs, 0.1) is None
    bad_hi = torch.zeros(B, 3, T, 4, dtype=torch.long, device=dev)
    assert SG.triton_gather_attention(q.to(dev), k.to(dev), v.to(dev), bad_hi, pos.to(dev), None, bs, 0.1) is None
    # fp32 operands run on the fp32 matrix-core form (the reference kernels are
    # dtype-generic): fp32 products and sums, within 1e-5 relative
    out32 = SG.triton_gather_attention(q.float().to(dev), k.float().to(dev), v.float().to(dev), bi.to(dev),
                                       pos.to(dev), None, bs, 1 / math.sqrt(D), local_window=lw)
    assert out32 is not None and out32.dtype == torch.float32
    ref32, _ = O.gather_attention(q.double(), k.double(), v.double(), bi, pos, bs, 1 / math.sqrt(D), lw)
    assert (out32.cpu().double() - ref32).abs().max().item() <= 1e-5 * ref32.abs().max().item()
    assert SG.SPARSE_BLOCK_SIZE_SENTINEL == 128


def test_gather_attention_e2e_bias_grad(dev):
    g = torch.Generator().manual_seed(2)
    B, H, T, D, bs, lw, S = 1, 2, 160, 128, 32, 64, 3
    q, k, v = (torch.randn(B, H, T, D, generator=g).to(torch.bfloat16) for _ in range(3))
    bi = torch.randint(0, T // bs, (B, 1, T, S), generator=g)
    bsl = torch.randn(B, T, S, generator=g)
    pos = torch.arange(T)[None]
    qd, kd, vd = (x.to(dev).requires_grad_() for x in (q, k, v))
    bd = bsl.to(dev).requires_grad_()
    out = E2E.triton_gather_attention_e2e(qd, kd, vd, bi.to(dev), bd, pos.to(dev), None, bs,
                                          1 / math.sqrt(D), lw)
    do = torch.randn(out.shape, generator=g).to(torch.bfloat16)
    out.backward(do.to(dev))
    qr, kr, vr = (x.double().requires_grad_() for x in (q, k, v))
    br = bsl.double().requires_grad_()
    ref = O.gather_attention_e2e(qr, kr, vr, bi, br, pos, bs, 1 / math.sqrt(D), lw)
    ref.backward(do.double())
    assert (out.detach().cpu().double() - ref.detach()).abs().max().item() <= 2e-2
    for a, b in ((qd, qr), (kd, kr), (vd, vr), (bd, br)):
        assert (a.grad.cpu().double() - b.grad).abs().max().item() <= 2e-2
    # gates
    assert E2E.triton_gather_attention_e2e(qd, kd, vd, bi.to(dev), bd, (pos + 1).to(dev), None, bs, 0.1) is None
    assert E2E.SPARSE_E2E_SENTINEL == 1


def _check_block_max(got, q, k, pos, seg, bs, nblk, lw, what):
    """got [B, C, nblk] against the fp64 oracle: the same -inf pattern, and
    |got - ref| <= 1e-5 * max over the block's scored keys of sum_i |q_i k_i|
    (a correct fp32 sum of the exact bf16 products stays within
    128 * 2^-24 = 7.6e-6 of that sum; a bf16-rounded accumulator would not)."""
    ref = O.block_max_scores(q.double(), k.double(), pos, seg, bs, nblk, lw)
    bound = O.block_max_scores(q.double().abs(), k.double().abs(), pos, seg, bs, nblk, lw)
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(got), fin), what
    err = (got.double()[fin] - ref[fin]).abs()
    rel = (err / bound[fin].clamp(min=1e-30)).max().item() if fin.any() else 0.0
    report(f"[err] {what}: max-abs {err.max().item() if fin.any() else 0.0:.3e}, "
           f"max |err| / sum|q k| {rel:.3e} (bar 1e-5)")
    assert rel <= 1e-5, (what, rel)


@pytest.mark.parametrize("bs", [16, 32, 64, 128])
def test_block_max_score(dev, bs):
    g = torch.Generator().manual_seed(bs)
    B, C, Sk, D, lw = 3, 150, 700, 128, 100
    q = torch.randn(B, C, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Sk, D, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, Sk, (B, C), generator=g)
    seg = torch.randint(0, 50, (B, C), generator=g)
    nblk = -(-Sk // bs) + 1
    got = SG.triton_block_max_score(q.to(dev), k.to(dev), pos.to(dev), seg.to(dev), bs, nblk, lw).cpu()
    _check_block_max(got, q, k, pos, seg, bs, nblk, lw, f"block max bs={bs}")


@pytest.mark.parametrize("bs", [32, 64])
def test_block_max_score_positions_past_the_keys(dev, bs):
    """Rows whose window starts past the last key (pos - LW + 1 > Sk, Sk not a
    multiple of 64): keys >= Sk are never scored (the reference's j < Sk mask,
    HF/sparse_gather_triton.py:471,478), so the partial last block's max comes
    from its real keys only and the blocks past Sk are -inf."""
    g = torch.Generator().manual_seed(300 + bs)
    B, C, Sk, D, lw = 2, 130, 700, 128, 64
    q = torch.randn(B, C, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Sk, D, generator=g).to(torch.bfloat16)
    pos = torch.randint(600, 1000, (B, C), generator=g)
    seg = torch.zeros(B, C, dtype=torch.long)
    seg[1] = torch.randint(0, 690, (C,), generator=g)
    nblk = -(-Sk // bs) + 2
    got = SG.triton_block_max_score(q.to(dev), k.to(dev), pos.to(dev), seg.to(dev), bs, nblk, lw).cpu()
    _check_block_max(got, q, k, pos, seg, bs, nblk, lw, f"block max past the keys bs={bs}")
    # the partial last block holds 700 % bs real keys, all remote for rows with pos >= Sk + lw - 1
    last = (Sk - 1) // bs
    far = pos >= Sk + lw - 1
    assert torch.isfinite(got[..., last][far & (seg <= last * bs)]).all()
    assert torch.isinf(got[..., last + 1:]).all()


def test_block_max_topk_ids_cfg4_chunk(dev):
    """Config 4's chunk through the path select_and_kl_loss takes
    (HF/_sparse_base_impl.py:3322-3403): block-max scores of B=4 x 2048 rows at
    the tail of 65536 keys (one index head, bf16) -> top-8 per row, -inf never
    selected.  Sampled rows (tile edges, first / last, random) against the fp64
    oracle: scores within 1e-5 of sum |q k|, ids bit-exact outside near-ties."""
    g = torch.Generator().manual_seed(20261204)
    B, C, Sk, D, bs, lw, K = 4, 2048, 65536, 128, 64, 512, 8
    q = torch.randn(B, C, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Sk, D, generator=g).to(torch.bfloat16)
    pos = (torch.arange(C) + (Sk - C)).expand(B, C).contiguous()
    seg = torch.zeros(B, C, dtype=torch.long)
    nblk = Sk // bs
    sc = SG.triton_block_max_score(q.to(dev), k.to(dev), pos.to(dev), seg.to(dev), bs, nblk, lw)
    ids = srswa.topk_rows(sc, K, invalid_at=float("-inf")).cpu()
    rows = sorted({0, 1, 63, 64, 1023, 1024, C - 65, C - 64, C - 1}
                  | set(torch.randint(0, C, (23,), generator=g).tolist()))
    r = torch.tensor(rows)
    got = sc.cpu()[:, r]
    _check_block_max(got, q[:, r], k, pos[:, r], seg[:, r], bs, nblk, lw, "config 4 chunk block max (sampled rows)")
    ref = O.block_max_scores(q[:, r].double(), k.double(), pos[:, r], seg[:, r], bs, nblk, lw)
    compare_selection(ids[:, r], ref, K, "config 4 chunk block max -> top-8 (sampled rows)",
                      invalid_at=float("-inf"))


@pytest.mark.parametrize("bs,d", [(16, 128), (64, 128), (192, 64)])
def test_block_max_score_key_slabs(dev, bs, d):
    """Keys long enough for several key slabs per query tile (slabs of >= 16
    64-key chunks of whole blocks, 3 chunks per block at bs=192); positions from
    0 to the end, so some tiles stop inside a slab and later slabs hold only -inf
    blocks; two blocks past the keys."""
    g = torch.Generator().manual_seed(100 + bs)
    B, C, Sk, lw = 2, 130, 5000, 256
    q = torch.randn(B, C, d, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Sk, d, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, Sk, (B, C), generator=g)
    pos[0, :64] = torch.arange(64) + 300          # a tile that ends in the first slab
    seg = torch.randint(0, 400, (B, C), generator=g)
    nblk = -(-Sk // bs) + 2
    got = SG.triton_block_max_score(q.to(dev), k.to(dev), pos.to(dev), seg.to(dev), bs, nblk, lw).cpu()
    _check_block_max(got, q, k, pos, seg, bs, nblk, lw, f"block max key slabs bs={bs} d={d}")


@pytest.mark.parametrize("sk", [50, 64, 129])
def test_block_max_score_short_keys(dev, sk):
    """Keys shorter than one or two 64-key chunks (a partial first chunk read
    past the keys): rows at and past the end, window 1, two blocks past Sk."""
    g = torch.Generator().manual_seed(900 + sk)
    B, C, D, bs, lw = 2, 300, 128, 64, 1
    q = torch.randn(B, C, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, sk, D, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, sk + 40, (B, C), generator=g)
    seg = torch.randint(0, max(1, sk // 2), (B, C), generator=g)
    nblk = -(-sk // bs) + 2
    got = SG.triton_block_max_score(q.to(dev), k.to(dev), pos.to(dev), seg.to(dev), bs, nblk, lw).cpu()
    _check_block_max(got, q, k, pos, seg, bs, nblk, lw, f"block max short keys sk={sk}")


@pytest.mark.parametrize("bs,d", [(64, 64), (128, 128)])
def test_block_max_score_fp16_row_tiles(dev, bs, d):
    """fp16 operands over several 256-row query tiles (the last one partial),
    rows at unrelated positions and segment starts, keys long enough for
    several key slabs, and the last key block partial (Sk % 64 != 0)."""
    g = torch.Generator().manual_seed(700 + bs + d)
    B, C, Sk, lw = 2, 600, 3001, 128
    q = torch.randn(B, C, d, generator=g).to(torch.float16)
    k = torch.randn(B, Sk, d, generator=g).to(torch.float16)
    pos = torch.randint(0, Sk + 300, (B, C), generator=g)
    seg = torch.randint(0, 900, (B, C), generator=g)
    nblk = -(-Sk // bs) + 1
    got = SG.triton_block_max_score(q.to(dev), k.to(dev), pos.to(dev), seg.to(dev), bs, nblk, lw).cpu()
    _check_block_max(got, q, k, pos, seg, bs, nblk, lw, f"block max fp16 row tiles bs={bs} d={d}")
