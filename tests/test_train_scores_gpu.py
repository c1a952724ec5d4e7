"""DASH training block scorers on the GPU against the oracle
(oracle/train_score_oracle.py), forward and backward, through the C ABI.

Bars (fp32 path of the task): relative error max|got - ref| / max|ref| <=
1e-5 for the scores and for every gradient, the oracle in float64 on the same
fp32 inputs.  Upstream gradients carry NaN / inf / huge entries on masked
scores (the reference's hooks and masks must drop them)."""

import pytest
import torch

from oracle import train_score_oracle as T
from parity_report import report

pytestmark = pytest.mark.gpu
F32_REL = 1e-5


def _rel(got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    return (got - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)


def _upstream(z_ref, seed):
    """d loss / d z with non-finite and huge values on masked entries only (the
    caller's hook leaves kept entries finite and bounded)."""
    g = torch.randn(z_ref.shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    masked = z_ref <= -1e8
    junk = torch.tensor([float("nan"), float("inf"), -float("inf"), 1e30], dtype=torch.float64)
    idx = torch.arange(g.numel()).view(g.shape) % 4
    return torch.where(masked, junk[idx], g)


HC_CASES = {
    # name: B, S, d, bs, lb, head_cls scale, position offset per sequence
    "shipped_bs32_lb4": (2, 1500, 128, 32, 4, 0.5, (0, 0)),
    "cfg5_shape_bs64_lb8": (1, 4096, 128, 64, 8, 0.3, (0,)),
    "ragged_last_block_d64": (3, 1001, 64, 16, 2, 1.0, (0, 40, 7)),
    "bs128_zero_head_cls": (1, 777, 128, 128, 1, 0.0, (300,)),
    # the remaining (head dim, block size) pairs, each with a ragged last block
    "d128_bs16_lb3": (1, 509, 128, 16, 3, 0.7, (0,)),
    "d64_bs32_lb2": (2, 611, 64, 32, 2, 0.9, (0, 13)),
    "d64_bs64_lb1": (1, 700, 64, 64, 1, 1.2, (0,)),
    "d64_bs128_lb1": (1, 900, 64, 128, 1, 0.6, (50,)),
}


def _hc_case(name, dev):
    B, S, d, bs, lb, hcs, offs = HC_CASES[name]
    g = torch.Generator().manual_seed(list(HC_CASES).index(name) + 100)
    q = torch.randn(B, S, d, generator=g)
    k = torch.randn(B, S, d, generator=g)
    hc = torch.randn(d, generator=g) * hcs
    pos = torch.stack([torch.arange(S) + o for o in offs]).to(torch.int64)
    nblk = -(-S // bs)
    return q, k, hc, pos, nblk, bs, lb


@pytest.mark.parametrize("name", list(HC_CASES))
def test_head_cls_scores_fwd_bwd(dev, name):
    from srswa import train_scores as TS
    q, k, hc, pos, nblk, bs, lb = _hc_case(name, dev)
    print(f"head_cls scores {name}: B={q.shape[0]} S={q.shape[1]} d={q.shape[2]} bs={bs}", flush=True)
    qr, kr, hr = (x.double().requires_grad_() for x in (q, k, hc))
    zr = T.headcls_scores(qr, kr, hr, pos, nblk, bs, lb)
    gz = _upstream(zr.detach(), 7)
    zr.backward(gz)
    qd, kd, hd = (x.to(dev).requires_grad_() for x in (q, k, hc))
    z = TS.head_cls_scores(qd, kd, hd, pos.to(dev), nblk, bs, lb)
    assert z.dtype == torch.float32 and z.shape == zr.shape
    masked = zr.detach() <= -1e8
    assert torch.equal((z.cpu() <= -1e8), masked)
    ez = _rel(z.masked_fill(masked.to(dev), 0), zr.detach().masked_fill(masked, 0))
    z.backward(gz.float().to(dev))
    eq, ek, eh = _rel(qd.grad, qr.grad), _rel(kd.grad, kr.grad), _rel(hd.grad, hr.grad)
    report(f"[err] head_cls scores {name}: z max rel {ez:.3e}, dq {eq:.3e}, dk {ek:.3e}, "
           f"d head_cls {eh:.3e} (bar {F32_REL})")
    for e in (ez, eq, ek, eh):
        assert e <= F32_REL, (ez, eq, ek, eh)


@pytest.mark.parametrize("name", ["random_positions", "fewer_blocks_than_keys"])
def test_head_cls_scores_general_layouts(dev, name):
    """Arbitrary (non-monotonic) positions, so the rows of one 64-row tile reach
    different blocks and some reach past the keys; and a block grid shorter
    than the keys (nblk * bs < S: the later keys take no part and their dk rows
    stay zero)."""
    from srswa import train_scores as TS
    g = torch.Generator().manual_seed(71 if name == "random_positions" else 72)
    if name == "random_positions":
        B, S, d, bs, lb = 2, 1300, 128, 32, 2
        nblk = -(-S // bs)
        pos = torch.randint(0, 1600, (B, S), generator=g)
    else:
        B, S, d, bs, lb = 1, 1000, 64, 16, 3
        nblk = S // bs - 5
        pos = torch.arange(S)[None] + 100
    q = torch.randn(B, S, d, generator=g)
    k = torch.randn(B, S, d, generator=g)
    hc = torch.randn(d, generator=g) * 0.5
    print(f"head_cls scores {name}: B={B} S={S} d={d} bs={bs} nblk={nblk}", flush=True)
    qr, kr, hr = (x.double().requires_grad_() for x in (q, k, hc))
    zr = T.headcls_scores(qr, kr, hr, pos, nblk, bs, lb)
    gz = _upstream(zr.detach(), 8)
    zr.backward(gz)
    qd, kd, hd = (x.to(dev).requires_grad_() for x in (q, k, hc))
    z = TS.head_cls_scores(qd, kd, hd, pos.to(dev), nblk, bs, lb)
    masked = zr.detach() <= -1e8
    assert torch.equal((z.detach().cpu() <= -1e8), masked)
    ez = _rel(z.detach().masked_fill(masked.to(dev), 0), zr.detach().masked_fill(masked, 0))
    z.backward(gz.float().to(dev))
    eq, ek, eh = _rel(qd.grad, qr.grad), _rel(kd.grad, kr.grad), _rel(hd.grad, hr.grad)
    report(f"[err] head_cls scores {name}: z max rel {ez:.3e}, dq {eq:.3e}, dk {ek:.3e}, "
           f"d head_cls {eh:.3e} (bar {F32_REL})")
    for e in (ez, eq, ek, eh):
        assert e <= F32_REL, (ez, eq, ek, eh)
    if name == "fewer_blocks_than_keys":
        assert (kd.grad[:, nblk * bs:] == 0).all()


def test_head_cls_scores_deterministic(dev):
    from srswa import train_scores as TS
    q, k, hc, pos, nblk, bs, lb = _hc_case("shipped_bs32_lb4", dev)
    outs = []
    for _ in range(2):
        qd, kd, hd = (x.to(dev).requires_grad_() for x in (q, k, hc))
        z = TS.head_cls_scores(qd, kd, hd, pos.to(dev), nblk, bs, lb)
        z.backward(torch.ones_like(z))
        outs.append((z.detach(), qd.grad, kd.grad, hd.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_head_cls_padding_overflow_quirk(dev):
    """A partial last block whose real keys all have logits below -88.7: the
    reference's padding weight exp(0 - m) * 0 is NaN, so that block's summary
    is zeroed and head_cls's gradient is NaN (the fp32 oracle shows it)."""
    from srswa import train_scores as TS
    B, S, d, bs, lb = 1, 200, 64, 64, 1
    g = torch.Generator().manual_seed(9)
    q = torch.randn(B, S, d, generator=g)
    k = torch.randn(B, S, d, generator=g)
    hc = torch.randn(d, generator=g)
    k[0, 192:] = -hc * 40.0                         # block 3 (8 real keys): logits ~ -40 |hc|^2 / 8
    pos = torch.arange(S)[None] + 400
    nblk = 4
    qr, kr, hr = (x.clone().requires_grad_() for x in (q, k, hc))
    zr = T.headcls_scores(qr, kr, hr, pos, nblk, bs, lb)                 # fp32, like the reference
    kbar, _ = T.headcls_summary(k, hc, nblk, bs)
    assert kbar[0, 3].abs().max().item() == 0.0
    zr.backward(torch.ones_like(zr))
    assert torch.isnan(hr.grad).all()
    qd, kd, hd = (x.to(dev).requires_grad_() for x in (q, k, hc))
    z = TS.head_cls_scores(qd, kd, hd, pos.to(dev), nblk, bs, lb)
    masked = zr.detach() <= -1e8
    assert _rel(z.detach().masked_fill(masked.to(dev), 0), zr.detach().masked_fill(masked, 0)) <= F32_REL
    assert (z[0, :, 3].detach().cpu() == 0).all()
    z.backward(torch.ones_like(z))
    assert torch.isnan(hd.grad.cpu()).all()
    assert _rel(qd.grad, qr.grad) <= F32_REL


def test_head_cls_full_config5_shape(dev):
    """Config 5's training shape (B=2, T=16384, 64-key blocks, 512-token
    window: local_blocks 8): scores and every gradient against the fp64 oracle."""
    from srswa import train_scores as TS
    B, S, d, bs, lb = 2, 16384, 128, 64, 8
    g = torch.Generator().manual_seed(55)
    q = torch.randn(B, S, d, generator=g)
    k = torch.randn(B, S, d, generator=g)
    hc = torch.randn(d, generator=g) * 0.2
    pos = torch.arange(S)[None].expand(B, S)
    nblk = S // bs
    print("head_cls scores config 5 shape: oracle", flush=True)
    qr, kr, hr = (x.double().requires_grad_() for x in (q, k, hc))
    zr = T.headcls_scores(qr, kr, hr, pos, nblk, bs, lb)
    gz = torch.randn(zr.shape, generator=torch.Generator().manual_seed(56), dtype=torch.float64)
    zr.backward(gz)
    print("head_cls scores config 5 shape: gpu", flush=True)
    qd, kd, hd = (x.to(dev).requires_grad_() for x in (q, k, hc))
    z = TS.head_cls_scores(qd, kd, hd, pos.to(dev), nblk, bs, lb)
    z.backward(gz.float().to(dev))
    masked = zr.detach() <= -1e8
    assert torch.equal((z.detach().cpu() <= -1e8), masked)
    ez = _rel(z.detach().masked_fill(masked.to(dev), 0), zr.detach().masked_fill(masked, 0))
    eq, ek, eh = _rel(qd.grad, qr.grad), _rel(kd.grad, kr.grad), _rel(hd.grad, hr.grad)
    report(f"[err] head_cls scores config 5 shape: z max rel {ez:.3e}, dq {eq:.3e}, dk {ek:.3e}, "
           f"d head_cls {eh:.3e} (bar {F32_REL})")
    for e in (ez, eq, ek, eh):
        assert e <= F32_REL, (ez, eq, ek, eh)


def _tied_blocks(q, k, pos, nblk, bs, lw):
    """(row, block) pairs whose maximum is attained by more than one remote key."""
    B, S, _ = q.shape
    sc = torch.matmul(q.double(), k.double().transpose(-1, -2)).clamp(-1e4, 1e4)
    kp = torch.arange(S)
    sc = sc.masked_fill(kp[None, None, :] > (pos[:, :, None] - lw), float("-inf"))
    sc = torch.nn.functional.pad(sc, (0, nblk * bs - S), value=float("-inf")).view(B, S, nblk, bs)
    mx = sc.amax(-1, keepdim=True)
    cnt = ((sc == mx) & torch.isfinite(mx)).sum(-1)
    return int((cnt > 1).sum())


# Inputs lie on a 1/16 grid (|x| <= 4, or small integers): every product and
# every partial sum of a 128-term score is exact in fp32, so the kernel's
# maxima, ties and clamps are the oracle's exactly (real-valued draws would
# let fp32 rounding swap near-tied keys, which moves a whole gradient term).
BM_CASES = {
    # name: B, S, d, bs, lw, integer-valued inputs, q rows scaled past the clamp, position offsets
    "shipped_bs32_lw128": (2, 1200, 128, 32, 128, False, False, (0, 17)),
    "cfg5_like_bs64_lw512": (1, 2600, 128, 64, 512, False, False, (0,)),
    "ragged_bs16_d64": (2, 999, 64, 16, 48, False, False, (3, 0)),
    "integer_ties_bs32": (2, 900, 128, 32, 64, True, False, (0, 5)),
    "integer_ties_clamped_bs64": (1, 1100, 64, 64, 128, True, True, (0,)),
    "integer_ties_bs16": (1, 700, 128, 16, 32, True, False, (0,)),
}


def _bm_case(name):
    B, S, d, bs, lw, integer, clamped, offs = BM_CASES[name]
    nblk = -(-S // bs)
    pos = torch.stack([torch.arange(S) + o for o in offs]).to(torch.int64)
    g = torch.Generator().manual_seed(300 + list(BM_CASES).index(name))
    if integer:
        q = torch.randint(-3, 4, (B, S, d), generator=g).float()
        k = torch.randint(-3, 4, (B, S, d), generator=g).float()
        k[:, 1::7] = k[:, 0::7][:, :k[:, 1::7].shape[1]]     # repeated keys: exact ties
        if clamped:
            q[:, ::5] *= 100.0                              # scores up to 1e5: clamped, some exactly 1e4
    else:
        q = torch.randint(-64, 65, (B, S, d), generator=g).float() / 16
        k = torch.randint(-64, 65, (B, S, d), generator=g).float() / 16
    return q, k, pos, nblk, bs, lw


@pytest.mark.parametrize("name", list(BM_CASES))
def test_block_max_scores_fwd_bwd(dev, name):
    from srswa import train_scores as TS
    q, k, pos, nblk, bs, lw = _bm_case(name)
    print(f"block-max scores {name}: S={q.shape[1]} d={q.shape[2]} bs={bs} lw={lw}", flush=True)
    qr, kr = (x.double().requires_grad_() for x in (q, k))
    zr = T.blockmax_scores(qr, kr, pos, nblk, bs, lw)
    gz = _upstream(zr.detach(), 11)
    zr.backward(gz)
    qd, kd = (x.to(dev).requires_grad_() for x in (q, k))
    z = TS.block_max_scores(qd, kd, pos.to(dev), nblk, bs, lw)
    masked = zr.detach() <= -1e8
    assert torch.equal((z.detach().cpu() <= -1e8), masked)
    ez = _rel(z.detach().masked_fill(masked.to(dev), 0), zr.detach().masked_fill(masked, 0))
    z.backward(gz.float().to(dev))
    eq, ek = _rel(qd.grad, qr.grad), _rel(kd.grad, kr.grad)
    assert torch.equal(z.detach().cpu().double(), zr.detach())       # exact scores (grid inputs)
    ties = ""
    if BM_CASES[name][5]:
        n = _tied_blocks(q, k, pos, nblk, bs, lw)
        assert n > 0
        ties = f", {n} (row, block) maxima shared by several keys"
    report(f"[err] block-max scores {name}: z max rel {ez:.3e}, dq {eq:.3e}, dk {ek:.3e} (bar {F32_REL}){ties}")
    for e in (ez, eq, ek):
        assert e <= F32_REL, (ez, eq, ek)


def test_block_max_scores_deterministic(dev):
    from srswa import train_scores as TS
    q, k, pos, nblk, bs, lw = _bm_case("integer_ties_bs32")
    outs = []
    for _ in range(2):
        qd, kd = (x.to(dev).requires_grad_() for x in (q, k))
        z = TS.block_max_scores(qd, kd, pos.to(dev), nblk, bs, lw)
        z.backward(torch.ones_like(z))
        outs.append((z.detach(), qd.grad, kd.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


class _GemmaRMS(torch.nn.Module):
    def __init__(self, d):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.zeros(d))
        self.eps = 1e-6

    def forward(self, x):
        x32 = x.to(torch.promote_types(x.dtype, torch.float32))
        x32 = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + self.eps)
        return (x32 * (1.0 + self.weight)).to(x.dtype)


def _stand_in_router(hidden, d, bs, lb, seed):
    """A router carrying the reference's stage-0 attributes (q_proj, k_proj,
    q_norm, k_norm, head_cls, block_size, local_blocks, local_window)."""
    g = torch.Generator().manual_seed(seed)
    r = torch.nn.Module()
    r.index_dim, r.block_size, r.local_blocks, r.local_window = d, bs, lb, lb * bs
    r.q_proj = torch.nn.Linear(hidden, d, bias=False)
    r.k_proj = torch.nn.Linear(hidden, d, bias=False)
    r.q_norm, r.k_norm = _GemmaRMS(d), _GemmaRMS(d)
    r.head_cls = torch.nn.Parameter(torch.randn(d, generator=g) * 0.3)
    with torch.no_grad():
        for p in (r.q_proj.weight, r.k_proj.weight):
            p.copy_(torch.randn(p.shape, generator=g) / hidden ** 0.5)
        for p in (r.q_norm.weight, r.k_norm.weight):
            p.copy_(torch.randn(p.shape, generator=g) * 0.1)
    return r


def _rope_tables(pos, d):
    inv = 1.0 / (10000.0 ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    fr = pos.double()[..., None] * inv
    emb = torch.cat([fr, fr], -1)
    return emb.cos(), emb.sin()


@pytest.mark.parametrize("stage0", ["head_cls", "indexer"])
def test_patched_dash_attention_stage0(dev, stage0):
    """srswa.patch rebinds DashAttention._block_scores_headcls / _block_scores
    of a stand-in class: on device tensors the rebound method (the model's own
    projections, RMSNorms and RoPE, then the kernels) matches the oracle's
    restatement of the whole method in float64 -- scores and the gradients of
    every router weight and of the hidden states; host tensors reach the
    original method, and restore puts it back."""
    import copy
    import sys
    import types
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    from srswa import patch

    calls = []

    class DashAttention:
        def _block_scores_headcls(self, *a):
            calls.append("headcls")
            return "eager"

        def _block_scores(self, *a):
            calls.append("blockmax")
            return "eager"

    dash_mod = types.ModuleType("stand_in_dash_attention_stage0")
    dash_mod._rope_fn = apply_rotary_pos_emb
    dash_mod._sanitize_grad = T.sanitize_grad
    DashAttention.__module__ = dash_mod.__name__
    sys.modules[dash_mod.__name__] = dash_mod
    mod = types.SimpleNamespace(DashAttention=DashAttention)
    B, S, hidden, d, bs, lb = 2, 300, 96, 64, 16, 2
    g = torch.Generator().manual_seed(77)
    hs = torch.randn(B, S, hidden, generator=g)
    pid = torch.stack([torch.arange(S), torch.arange(S) + 9])
    nblk = -(-S // bs)
    cos, sin = _rope_tables(pid, d)
    try:
        names = patch.apply(mod)
        assert "DashAttention._block_scores_headcls" in names and "DashAttention._block_scores" in names
        att = DashAttention()
        router = _stand_in_router(hidden, d, bs, lb, 78)
        ref_router = copy.deepcopy(router).double()
        router = router.to(dev)
        for name in ("index_dim", "block_size", "local_blocks", "local_window", "q_proj", "k_proj", "q_norm",
                     "k_norm", "head_cls"):
            setattr(att, name, getattr(router, name))
        meth = att._block_scores_headcls if stage0 == "head_cls" else att._block_scores
        hsd = hs.to(dev).requires_grad_()
        z = meth(hsd, (cos.float().to(dev), sin.float().to(dev)), pid.to(dev), nblk)
        assert calls == []
        hr = hs.double().requires_grad_()
        oracle = T.headcls_method if stage0 == "head_cls" else T.blockmax_method
        zr = oracle(ref_router, hr, (cos, sin), pid, nblk, rope_fn=apply_rotary_pos_emb)
        masked = zr.detach() <= -1e8
        assert torch.equal(z.detach().cpu() <= -1e8, masked)
        ez = _rel(z.detach().masked_fill(masked.to(dev), 0), zr.detach().masked_fill(masked, 0))
        w = torch.randn(zr.shape, generator=g, dtype=torch.float64).masked_fill(masked, 0)
        (z * w.float().to(dev)).sum().backward()
        (zr * w).sum().backward()
        errs = {"z": ez, "hidden": _rel(hsd.grad, hr.grad)}
        for (n1, p1), (n2, p2) in zip(sorted(dict(att.q_proj.named_parameters(prefix="q_proj")).items()) +
                                      sorted(dict(att.k_proj.named_parameters(prefix="k_proj")).items()) +
                                      sorted(dict(att.q_norm.named_parameters(prefix="q_norm")).items()) +
                                      sorted(dict(att.k_norm.named_parameters(prefix="k_norm")).items()),
                                      sorted(dict(ref_router.q_proj.named_parameters(prefix="q_proj")).items()) +
                                      sorted(dict(ref_router.k_proj.named_parameters(prefix="k_proj")).items()) +
                                      sorted(dict(ref_router.q_norm.named_parameters(prefix="q_norm")).items()) +
                                      sorted(dict(ref_router.k_norm.named_parameters(prefix="k_norm")).items())):
            errs[n1] = _rel(p1.grad, p2.grad)
        if stage0 == "head_cls":
            errs["head_cls"] = _rel(att.head_cls.grad, ref_router.head_cls.grad)
        report(f"[err] patched DashAttention stage0 {stage0}: " +
               ", ".join(f"{k} {v:.2e}" for k, v in errs.items()) + f" (bar {F32_REL})")
        for k_, v in errs.items():
            assert v <= F32_REL, (k_, v)
        # host tensors: the original method
        assert meth(hs, None, pid, nblk) == "eager"
    finally:
        patch.restore(mod)
        del sys.modules[dash_mod.__name__]
    assert DashAttention()._block_scores_headcls() == "eager"
