"""Training DASH router (srswa.dash_train: DashAttention._route /
_select_and_bias, HF/dash_attention.py:1145-1204) vs the CPU oracle
(``srswa_oracle.dash_route_train`` / ``dash_select_and_bias``, fp64 on the
same inputs, with x = score * idx_scale rounded to the storage dtype as the
reference's tensors are):

* candidates exact; prior within 1e-5 (fp32) or the 16-bit bar of
  tests/tolerance.py;
* selection: the oracle's select on the kernel's own prior gives the same ids
  and validity bit for bit, the bias within the same bars;
* backward: the select backward and the route backward each alone on the
  kernel's own prior / ids (row norms within 1e-5 fp32, 2e-2 16-bit, the
  route's against the norm of its terms), and the gradient of
  sum(bias * w) + sum(prior * w2) w.r.t. the block scores end to end with the
  oracle held to the kernel's ids: rows within 1e-4 (fp32); 16-bit within
  2e-2 of the whole tensor's norm (every step rounds to the storage dtype, as
  the reference's own 16-bit chain does).
Also: the rebinding through srswa.patch on a stand-in DashAttention, host
tensors to the original methods."""

import types

import pytest
import torch

from oracle import srswa_oracle as O
from parity_report import report
from tolerance import assert_close_lowp

pytestmark = pytest.mark.gpu


def _case(seed, B, S, nblk, spread, dtype, mask):
    g = torch.Generator().manual_seed(seed)
    sc = (torch.randn(B, S, nblk, generator=g) * spread).to(dtype)
    # causal-like remote sets: row s sees blocks < s * nblk / S - 2
    lim = (torch.arange(S) * nblk // S - 2)[None, :, None]
    sc = torch.where(torch.arange(nblk)[None, None, :] <= lim, sc, torch.full((), O.SCORE_NEG, dtype=dtype))
    blk = img = None
    if mask == "block":
        blk = torch.rand(B, S, nblk, generator=g) < 0.3
    elif mask == "image":
        img = torch.rand(B, nblk, generator=g) < 0.4
    return sc, blk, img


CASES = {
    # B, S, nblk, score spread, idx_scale, dtype, mask, K, floor, sigma
    "fp32_image_k12": (2, 200, 48, 1.0, 2.0, torch.float32, "image", 12, 1e-4, 1.0),
    "fp32_block_k8_sigma": (2, 160, 96, 1.0, 1.5, torch.float32, "block", 8, 1e-3, 0.5),
    "bf16_flat_600_blocks": (1, 128, 600, 1.0, 0.1, torch.bfloat16, None, 16, 1e-4, 1.0),
    "bf16_shipped_scale": (2, 128, 64, 1.0, 11.3, torch.bfloat16, "image", 12, 1e-4, 1.0),
    "fp16_block": (1, 100, 40, 1.0, 3.0, torch.float16, "block", 10, 1e-2, 2.0),
    "fp32_1500_blocks_k64": (1, 96, 1500, 1.0, 0.5, torch.float32, "image", 64, 1e-4, 1.0),
}


def _close(got, ref, dtype, what, tol32=1e-5):
    if dtype == torch.float32:
        err = (got.double() - ref).abs().max().item() if got.numel() else 0.0
        report(f"[err] {what}: max-abs {err:.3e} (bar {tol32})")
        assert err <= tol32, (what, err)
    else:
        assert_close_lowp(got, ref, dtype, what=what)


@pytest.mark.parametrize("name", list(CASES))
def test_dash_train_router_matches_oracle(dev, name):
    from srswa import dash_train as DT
    B, S, nblk, spread, scale, dtype, mask, K, floor, sigma = CASES[name]
    print(f"dash train router {name}", flush=True)
    sc, blk, img = _case(list(CASES).index(name) + 60, B, S, nblk, spread, dtype, mask)
    xs = torch.where(sc.double() > -5e8, (sc.float() * scale).to(dtype).double(), sc.double())

    # forward
    sd = sc.to(dev).requires_grad_()
    prior, cand = DT.RouteTrainFn.apply(sd, None if blk is None else blk.to(dev),
                                        None if img is None else img.to(dev), scale, -1.0e4)
    topi, bias, valid = DT.SelectTrainFn.apply(prior, cand, K, floor, sigma)
    rp, rc = O.dash_route_train(xs, img, blk, 1.0)
    assert torch.equal(cand.cpu(), rc)
    _close(prior.detach().cpu(), rp, dtype, f"{name} prior")
    oi, ob, ov = O.dash_select_and_bias(prior.detach().cpu().double(), cand.cpu(), K, floor, sigma)
    assert torch.equal(topi.cpu(), oi) and torch.equal(valid.cpu(), ov)
    if dtype == torch.float32:
        _close(bias.detach().cpu(), ob, dtype, f"{name} bias", tol32=2e-5)
    else:
        # the reference computes log / mean / centring in the storage dtype
        # (an ulp of a bias near -6 is 2^-5 in bf16): the oracle's select in that
        # dtype on the CPU, within two of its ulps
        _, ob16, _ = O.dash_select_and_bias(prior.detach().cpu(), cand.cpu(), K, floor, sigma)
        ulp = torch.exp2(torch.floor(torch.log2(ob16.double().abs().clamp(min=2.0 ** -14))) -
                         (7 if dtype == torch.bfloat16 else 10))
        err = ((bias.detach().cpu().double() - ob16.double()).abs() / ulp).max().item()
        report(f"[err] {name} bias vs the {dtype} restatement: max {err:.2f} ulp (bar 2); "
               f"vs fp64: max-abs {(bias.detach().cpu().double() - ob).abs().max().item():.3e}")
        assert err <= 2.0

    # backward
    g = torch.Generator().manual_seed(7)
    w = torch.randn(B, S, K, generator=g)
    w2 = torch.randn(B, S, nblk, generator=g)
    ((bias.float() * w.to(dev)).sum() + (prior.float() * w2.to(dev)).sum()).backward()
    lowp = dtype != torch.float32
    # (1) the select backward alone, on the kernel's prior and ids
    pd = prior.detach()
    dp_k = DT.select_backward(w.to(dev).to(dtype), pd, cand, topi, floor, sigma).cpu().double()
    pl = pd.cpu().double().requires_grad_()
    bl, _ = O.dash_bias_given(pl, cand.cpu(), topi.cpu(), floor, sigma)
    (bl * w.to(dtype).double()).sum().backward()
    _rows_close(dp_k, pl.grad, 2e-2 if lowp else 1e-5, f"{name} select backward")
    # (2) the route backward alone, on the kernel's prior and a dense upstream gradient
    dy = w2.to(dtype)
    ds_k = DT.route_backward(dy.to(dev), pd, cand, scale).cpu().double()
    y, dyd = pd.cpu().double(), dy.double()
    gp = y.sqrt()
    q = (dyd * gp).sum(-1, keepdim=True) / gp.sum(-1, keepdim=True).clamp_min(1e-12)
    ds_o = torch.where(cand.cpu(), (dyd * gp - q * gp) * scale, torch.zeros_like(y))
    terms = torch.where(cand.cpu(), ((dyd * gp).abs() + (q * gp).abs()) * scale, torch.zeros_like(y))
    _rows_close(ds_k, ds_o, 2e-2 if lowp else 1e-5, f"{name} route backward", scale_rows=terms)
    # (3) end to end, the oracle held to the kernel's ids
    xr = xs.clone().requires_grad_()
    rp2, rc2 = O.dash_route_train(xr, img, blk, 1.0)
    rb, _ = O.dash_bias_given(rp2, rc2, topi.cpu(), floor, sigma)
    ((rb * w.double()).sum() + (rp2 * w2.double()).sum()).backward()
    got, ref = sd.grad.cpu().double(), xr.grad * scale
    if not lowp:
        _rows_close(got, ref, 1e-4, f"{name} d scores")
    else:
        # the chain rounds to the storage dtype at every step, as the reference's does
        rel = (got - ref).norm().item() / ref.norm().item()
        report(f"[err] {name} d scores end to end: rel-norm {rel:.3e} (bar 2e-2)")
        assert rel <= 2e-2


def _rows_close(got, ref, bar, what, scale_rows=None):
    """max over rows of ||got - ref|| / ||scale_rows (default ref)|| <= bar."""
    den = (ref if scale_rows is None else scale_rows).norm(dim=-1)
    num = (got - ref).norm(dim=-1)
    err = torch.where(den > 0, num / den.clamp(min=1e-300), torch.where(num > 0, float("inf"), 0.0))
    report(f"[err] {what}: max row rel-norm {err.max().item():.3e} (bar {bar})")
    assert err.max().item() <= bar, (what, err.max().item())


def test_dash_train_patch_rebinds_and_host_fallback(dev):
    from srswa import patch
    calls = []

    class DashAttention:
        image_only = True
        training = True
        sigma = 1.0
        index_dim = 128
        _neg = -1.0e4
        _sched_id = 0

        def _cur_idx_scale(self):
            return 2.0

        def _cur_prior_floor(self):
            return 1e-4

        def _route(self, block_scores, image_block_mask, block_cand=None):
            calls.append("route")
            return "eager-route"

        def _select_and_bias(self, prior, cand, nblk):
            calls.append("select")
            return "eager-select"

    class _Sched:
        def __init__(self):
            self.calibrated = []

        def needs_calib(self, sid, training):
            return not self.calibrated

        def calibrate(self, sid, scores, cand, neg, sqrt_d):
            self.calibrated.append((sid, tuple(cand.shape), neg))

    dash_mod = types.ModuleType("stand_in_dash_attention")
    dash_mod._SCHED = _Sched()
    dash_mod._KS = types.SimpleNamespace(k=12)
    DashAttention.__module__ = dash_mod.__name__
    import sys
    sys.modules[dash_mod.__name__] = dash_mod
    mod = types.SimpleNamespace(DashAttention=DashAttention)
    try:
        names = patch.apply(mod)
        assert "DashAttention._route" in names and "DashAttention._select_and_bias" in names
        att = DashAttention()
        sc, _, img = _case(3, 1, 64, 40, 1.0, torch.float32, "image")
        prior, cand = att._route(sc.to(dev), img.to(dev))
        assert dash_mod._SCHED.calibrated == [(0, (1, 64, 40), -1.0e4)]
        topi, bias, valid = att._select_and_bias(prior, cand, 40)
        assert topi.shape == (1, 64, 12) and calls == []
        rp, rc = O.dash_route_train(sc.double() * torch.where(sc > -5e8, 2.0, 1.0).double(), img, None, 1.0)
        assert torch.equal(cand.cpu(), rc)
        assert (prior.cpu().double() - rp).abs().max().item() <= 1e-5
        assert att._route(sc, img) == "eager-route" and att._select_and_bias(prior.cpu(), cand.cpu(), 40) == \
            "eager-select"
        assert calls == ["route", "select"]
    finally:
        patch.restore(mod)
        del sys.modules[dash_mod.__name__]
    assert DashAttention()._route(None, None) == "eager-route"
