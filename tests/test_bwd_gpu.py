"""Gather-attention backward on the matrix cores vs autograd of the fp64
oracle (C ABI through the drop-in autograd Function).

Bar: bf16/fp16 dQ/dK/dV max-abs <= 2e-2 (beyond the output format's own
half-ulp, tests/tolerance.py) against fp64 autograd on the same rounded
inputs; the fp32 per-slot bias gradient max-abs <= 2e-2; two runs are bitwise
identical (no floating-point atomics)."""

import math

import pytest
import torch

from oracle import srswa_oracle as O
from srswa import ops
from tolerance import assert_close_lowp

pytestmark = pytest.mark.gpu
TOL = 2e-2

CASES = {
    "self_bs64": dict(B=2, HQ=2, HKV=2, HI=1, T=300, Sk=300, D=128, bs=64, lw=128, S=4),
    "tiles_bs32_hi2": dict(B=1, HQ=2, HKV=2, HI=2, T=512, Sk=512, D=128, bs=32, lw=128, S=6, shared_tile=True),
    "prefix": dict(B=1, HQ=2, HKV=2, HI=1, T=130, Sk=700, D=128, bs=64, lw=256, S=5),
    "packed_gqa": dict(B=1, HQ=4, HKV=2, HI=1, T=257, Sk=257, D=64, bs=16, lw=40, S=3, packed=True),
    "bias": dict(B=2, HQ=2, HKV=2, HI=1, T=192, Sk=192, D=128, bs=32, lw=64, S=4, bias=True),
    "bias_bs128_fp16": dict(B=1, HQ=2, HKV=1, HI=1, T=400, Sk=400, D=128, bs=128, lw=200, S=3, bias=True,
                            dtype=torch.float16),
}


def _inputs(seed, B, HQ, HKV, HI, T, Sk, D, bs, lw, S, dtype=torch.bfloat16, packed=False, bias=False,
            shared_tile=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, HQ, D, generator=g).to(dtype)
    k = torch.randn(B, Sk, HKV, D, generator=g).to(dtype)
    v = torch.randn(B, Sk, HKV, D, generator=g).to(dtype)
    do = torch.randn(B, T, HQ, D, generator=g).to(dtype)
    nblk = -(-Sk // bs)
    bi = torch.randint(-1, nblk, (B, HI, T, S), generator=g)
    if shared_tile:
        bi = bi[:, :, ::64].repeat_interleave(64, dim=2)[:, :, :T].contiguous()
    bi[..., 1] = bi[..., 0]
    if packed:
        cut = T // 3
        pos = torch.cat([torch.arange(cut), torch.arange(T - cut)])[None].expand(B, -1).contiguous()
    else:
        pos = (Sk - T + torch.arange(T))[None].expand(B, -1).contiguous()
    bsl = torch.randn(B, T, S, generator=g) if bias else None
    return q, k, v, do, bi, pos, bsl


def _gpu(dev, q, k, v, do, bi, pos, bsl, bs, lw, scale):
    T, Sk = q.shape[1], k.shape[1]
    qd, kd, vd = (x.to(dev).requires_grad_() for x in (q, k, v))
    bd = None if bsl is None else bsl.to(dev).requires_grad_()
    seg = ops._seg_from_positions(pos.to(dev), T, Sk, dev)
    o = ops.GatherAttnFn.apply(qd, kd, vd, bi.to(dev), seg, bd, bs, scale, lw)
    o.backward(do.to(dev))
    return [x.grad.cpu().double() for x in (qd, kd, vd)] + ([bd.grad.cpu().double()] if bd is not None else [])


def _ref(q, k, v, do, bi, pos, bsl, bs, lw, scale):
    qd, kd, vd = (x.double().transpose(1, 2).requires_grad_() for x in (q, k, v))
    Sk = k.shape[1]
    bd = None
    dense = None
    if bsl is not None:
        bd = bsl.double().requires_grad_()
        dense = O.bias_slots_to_dense(bd, bi[:, 0], -(-Sk // bs))
    o, _ = O.gather_attention(qd, kd, vd, bi, pos, bs, scale, lw, blk_bias_dense=dense)
    o.backward(do.double().transpose(1, 2))
    out = [x.grad.transpose(1, 2) for x in (qd, kd, vd)]
    if bd is not None:
        out.append(bd.grad)
    return out


@pytest.mark.parametrize("name", list(CASES))
def test_bwd_matches_oracle(dev, name):
    c = dict(CASES[name])
    bs, lw = c["bs"], c["lw"]
    q, k, v, do, bi, pos, bsl = _inputs(10 + list(CASES).index(name), **c)
    scale = 1 / math.sqrt(c["D"])
    got = _gpu(dev, q, k, v, do, bi, pos, bsl, bs, lw, scale)
    ref = _ref(q, k, v, do, bi, pos, bsl, bs, lw, scale)
    dt = c.get("dtype", torch.bfloat16)
    for nm, gt, rf in zip(("dq", "dk", "dv", "dbias"), got, ref):
        assert_close_lowp(gt, rf, dt if nm != "dbias" else torch.float32, TOL, f"backward {name}: {nm}")


F32_CASES = {
    "f32_self_bs64": dict(B=1, HQ=2, HKV=2, HI=1, T=300, Sk=300, D=128, bs=64, lw=128, S=4),
    "f32_packed_gqa_d64": dict(B=1, HQ=4, HKV=2, HI=1, T=257, Sk=257, D=64, bs=16, lw=40, S=3, packed=True),
    "f32_bias_prefix": dict(B=1, HQ=2, HKV=1, HI=1, T=130, Sk=700, D=128, bs=32, lw=128, S=4, bias=True),
}


@pytest.mark.parametrize("name", list(F32_CASES))
def test_bwd_fp32_matches_oracle(dev, name):
    """fp32 operands on the fp32 MFMA form: every gradient (and the bias
    gradient) within 1e-5 relative (max-abs error / max-abs reference) of fp64
    autograd, the fp32 bar."""
    c = dict(F32_CASES[name])
    bs, lw = c["bs"], c["lw"]
    q, k, v, do, bi, pos, bsl = _inputs(60 + list(F32_CASES).index(name), dtype=torch.float32, **c)
    scale = 1 / math.sqrt(c["D"])
    got = _gpu(dev, q, k, v, do, bi, pos, bsl, bs, lw, scale)
    ref = _ref(q, k, v, do, bi, pos, bsl, bs, lw, scale)
    from parity_report import report
    for nm, gt, rf in zip(("dq", "dk", "dv", "dbias"), got, ref):
        rel = (gt - rf).abs().max().item() / max(rf.abs().max().item(), 1e-30)
        report(f"[err] backward fp32 {name}: {nm} max rel {rel:.3e} (bar 1e-5)")
        assert rel <= 1e-5, (nm, rel)


def test_bwd_is_deterministic(dev):
    c = dict(CASES["bias"])
    bs, lw = c["bs"], c["lw"]
    q, k, v, do, bi, pos, bsl = _inputs(99, **c)
    a = _gpu(dev, q, k, v, do, bi, pos, bsl, bs, lw, 0.1)
    b = _gpu(dev, q, k, v, do, bi, pos, bsl, bs, lw, 0.1)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("bias_dims", [3, 4])
def test_bias_shared_by_two_index_heads(dev, bias_dims):
    """A per-slot bias that does not name the index head ([B, T, S], or
    [B, 1, T, S]) feeds slot s of EVERY index head; its gradient is the sum over
    the index heads.  Reference: one fp64 oracle per index head (its own blocks,
    the same slot biases), the gradients accumulated by autograd."""
    g = torch.Generator().manual_seed(41 + bias_dims)
    B, HQ, HI, T, D, bs, lw, S = 1, 4, 2, 256, 128, 32, 64, 4
    q = torch.randn(B, T, HQ, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, T, HQ, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, T, HQ, D, generator=g).to(torch.bfloat16)
    do = torch.randn(B, T, HQ, D, generator=g).to(torch.bfloat16)
    nblk = T // bs
    bi = torch.randint(-1, nblk, (B, HI, T, S), generator=g)
    bsl = torch.randn(B, T, S, generator=g)
    if bias_dims == 4:
        bsl = bsl[:, None]
    pos = torch.arange(T)[None]
    scale = 1 / math.sqrt(D)
    got = _gpu(dev, q, k, v, do, bi, pos, bsl, bs, lw, scale)
    assert got[3].shape == bsl.shape
    qd, kd, vd = (x.double().transpose(1, 2).requires_grad_() for x in (q, k, v))
    bd = bsl.double().requires_grad_()
    b3 = bd if bias_dims == 3 else bd[:, 0]
    gh = HQ // HI
    for h in range(HI):
        hs = slice(h * gh, (h + 1) * gh)
        dense = O.bias_slots_to_dense(b3, bi[:, h], nblk)
        o, _ = O.gather_attention(qd[:, hs], kd[:, hs], vd[:, hs], bi[:, h:h + 1], pos, bs, scale, lw,
                                  blk_bias_dense=dense)
        (o * do.double().transpose(1, 2)[:, hs]).sum().backward()
    ref = [x.grad.transpose(1, 2) for x in (qd, kd, vd)] + [bd.grad]
    for nm, gt, rf in zip(("dq", "dk", "dv", "dbias"), got, ref):
        assert_close_lowp(gt, rf, torch.bfloat16 if nm != "dbias" else torch.float32, TOL,
                          f"{nm}, [{'B, T, S' if bias_dims == 3 else 'B, 1, T, S'}] bias over HI=2")
