"""The reference-signature drop-in modules (srswa.sparse_gather_triton,
srswa.sparse_gather_e2e_triton) on the GPU: same call signatures, layouts,
None-fallback gates and results as the reference wrappers."""

import math

import pytest
import torch

from oracle import srswa_oracle as O
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
    # fp32 is not a matrix-core dtype: None (the caller's eager fallback), never a CPU path
    assert SG.triton_gather_attention(q.float().to(dev), k.float().to(dev), v.float().to(dev), bi.to(dev),
                                      pos.to(dev), None, bs, 0.1) is None
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
    ref = O.block_max_scores(q.double(), k.double(), pos, seg, bs, nblk, lw)
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(got), fin)
    assert (got.double()[fin] - ref[fin]).abs().max().item() <= 1e-3 * max(1.0, ref[fin].abs().max().item())


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
    ref = O.block_max_scores(q.double(), k.double(), pos, seg, bs, nblk, lw)
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(got), fin)
    assert (got.double()[fin] - ref[fin]).abs().max().item() <= 1e-3 * max(1.0, ref[fin].abs().max().item())
