"""DASH router kernel (srswa_dash_route) vs the CPU oracle's
``infer_route_select`` (HF/modeling_deepseekv2.py:338-362 restated): block ids
and valid flags bit-exact, bias within 1e-5 relative (fp32), over random rows,
page masks (one row falling back to every remote block), ties, non-finite
scores, short rows (nblk < top-M) and stride-0 (expanded) masks."""

import math

import pytest
import torch

from oracle import srswa_oracle as O

pytestmark = pytest.mark.gpu

P = dict(idx_scale=128.0 / math.sqrt(128), floor=1e-4, sigma=1.0, K=12, topm=16)


def _check(dev, sc, cand, p):
    from srswa import ops

    xi, bias, valid = ops.dash_route(sc.to(dev), None if cand is None else cand.to(dev), p)
    rx, rb, rv = O.infer_route_select(sc, cand, p["idx_scale"], p["floor"], p["sigma"], p["K"], p["topm"])
    assert xi.dtype == torch.int64 and valid.dtype == torch.bool and bias.dtype == torch.float32
    assert torch.equal(xi.cpu(), rx), (xi.cpu(), rx)
    assert torch.equal(valid.cpu(), rv)
    err = (bias.cpu() - rb).abs() / rb.abs().clamp(min=1.0)
    assert err.max().item() <= 1e-5, err.max().item()
    # attend-ready ids: int32, -1 in the invalid slots; bias and valid unchanged
    ai, ab, av = ops.dash_route(sc.to(dev), None if cand is None else cand.to(dev), p, attend_ids=True)
    assert ai.dtype == torch.int32
    assert torch.equal(ai.cpu(), torch.where(rv, rx, -1).to(torch.int32))
    assert torch.equal(ab, bias) and torch.equal(av, valid)


@pytest.mark.parametrize("nblk,K,topm", [(2048, 12, 16), (3000, 12, 16), (5000, 8, 16), (300, 8, 64),
                                        (40, 12, 16), (10, 12, 16), (5, 3, 0)])
def test_route_random(dev, nblk, K, topm):
    g = torch.Generator().manual_seed(nblk + K)
    B, Lq = 4, 3
    sc = torch.randn(B, Lq, nblk, generator=g) * 0.4
    sc[..., max(1, nblk - 8):] = O.SCORE_NEG            # the window / future blocks
    p = dict(P, K=K, topm=topm)
    _check(dev, sc, None, p)
    cand = torch.rand(B, Lq, nblk, generator=g) > 0.5
    cand[0, 1] = False                                   # empty mask -> every remote block
    _check(dev, sc, cand, p)


def test_route_ties_and_nonfinite(dev):
    g = torch.Generator().manual_seed(7)
    sc = (torch.randint(0, 4, (2, 4, 96), generator=g).float() * 0.25)   # many equal scores
    sc[0, 0, 3] = float("nan")
    sc[0, 1, 7] = float("inf")
    sc[1, 2, 11] = -float("inf")
    sc[..., 90:] = O.SCORE_NEG
    _check(dev, sc, None, P)
    _check(dev, sc, torch.rand(2, 4, 96, generator=g) > 0.3, dict(P, sigma=0.7, floor=1e-6))


@pytest.mark.parametrize("nblk", [2048, 300, 4000])
def test_route_many_keys_in_few_lanes(dev, nblk):
    """Blocks j = 0, 1 (mod 64) hold the largest scores: the threshold from the
    per-lane maxima then admits more than 64 keys and the kernel takes its
    round-by-round selection; j = 5 (mod 64) alone stays on the sorted path."""
    g = torch.Generator().manual_seed(11)
    j = torch.arange(nblk)
    sc = torch.randn(2, 2, nblk, generator=g) * 0.1
    sc[0, :, (j % 64) <= 1] += 5.0
    sc[1, :, (j % 64) == 5] += 5.0
    sc[..., -3:] = O.SCORE_NEG
    for cand in (None, torch.rand(2, 2, nblk, generator=g) > 0.2):
        _check(dev, sc, cand, dict(P, K=8, topm=16))
        _check(dev, sc, cand, dict(P, K=16, topm=64))


def test_route_expanded_mask_and_decode_shapes(dev):
    """The decode step passes allow[:, None, :].expand(B, Lq, nblk) (stride 0)."""
    g = torch.Generator().manual_seed(9)
    B, nblk = 64, 1024
    sc = torch.randn(B, 1, nblk, generator=g)
    sc[..., 1000:] = O.SCORE_NEG
    allow = torch.rand(B, nblk, generator=g) > 0.3
    cand = allow[:, None, :].expand(B, 1, nblk)
    _check(dev, sc, cand, P)


def test_route_rejects_wide_window(dev):
    from srswa import ops
    from srswa._lib import UnsupportedShape

    with pytest.raises(UnsupportedShape):
        ops.dash_route(torch.zeros(1, 1, 100, device=dev), None, dict(P, topm=0))
