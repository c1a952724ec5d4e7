"""Gather-attention forward on the matrix cores vs the CPU oracle (C ABI).

Bar: bf16/fp16 outputs max-abs <= 2e-2 (beyond the output format's own
half-ulp, tests/tolerance.py) against the fp64 oracle evaluated on the same
rounded inputs; fp32 LSE (natural log) within 2e-2."""

import math

import pytest
import torch

from oracle import srswa_oracle as O
from parity_report import report_error
from srswa import ops
from tolerance import assert_close_lowp

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _case(seed, B, HQ, HKV, HI, T, Sk, D, bs, lw, S, dtype=torch.bfloat16, packed=False,
          bias=False, shared_tile=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, HQ, D, generator=g).to(dtype)
    k = torch.randn(B, Sk, HKV, D, generator=g).to(dtype)
    v = torch.randn(B, Sk, HKV, D, generator=g).to(dtype)
    nblk = -(-Sk // bs)
    bi = torch.randint(-1, nblk, (B, HI, T, S), generator=g)
    if shared_tile:     # one selection per 64-row tile, as the indexer produces
        bi = bi[:, :, ::64].repeat_interleave(64, dim=2)[:, :, :T].contiguous()
    bi[..., 1] = bi[..., 0]
    if packed:
        cut = T // 3
        pos = torch.cat([torch.arange(cut), torch.arange(T - cut)])[None].expand(B, -1).contiguous()
        assert Sk == T
    else:
        pos = (Sk - T + torch.arange(T))[None].expand(B, -1).contiguous()
    bs_slots = torch.randn(B, T, S, generator=g) if bias else None
    return q, k, v, bi, pos, bs_slots


def _run(dev, q, k, v, bi, pos, bias, bs, lw, scale):
    B, T, HQ, D = q.shape
    Sk = k.shape[1]
    seg = ops._seg_from_positions(pos.to(dev), T, Sk, dev)
    o, lse = ops.gather_fwd(q.to(dev), k.to(dev), v.to(dev), bi.to(dev), block_size=bs,
                            local_window=lw, scale=scale, seg=seg,
                            bias=None if bias is None else bias.to(dev))
    dense = None
    if bias is not None:
        dense = O.bias_slots_to_dense(bias.double(), bi[:, 0], -(-Sk // bs))
    ro, rl = O.gather_attention(q.double().transpose(1, 2), k.double().transpose(1, 2),
                                v.double().transpose(1, 2), bi, pos, bs, scale, lw,
                                blk_bias_dense=dense)
    return o.cpu().double(), lse.cpu().double(), ro.transpose(1, 2), rl.transpose(1, 2)


CASES = {
    "self_bs64": dict(B=2, HQ=2, HKV=2, HI=1, T=300, Sk=300, D=128, bs=64, lw=128, S=4),
    "self_bs32_tiles": dict(B=1, HQ=2, HKV=2, HI=2, T=512, Sk=512, D=128, bs=32, lw=128, S=6, shared_tile=True),
    "prefix": dict(B=2, HQ=2, HKV=2, HI=1, T=130, Sk=1000, D=128, bs=64, lw=256, S=5),
    "packed": dict(B=1, HQ=2, HKV=1, HI=1, T=257, Sk=257, D=128, bs=16, lw=40, S=3, packed=True),
    "gqa_hi": dict(B=1, HQ=4, HKV=2, HI=2, T=200, Sk=200, D=64, bs=64, lw=64, S=4),
    "bias": dict(B=2, HQ=2, HKV=2, HI=1, T=192, Sk=192, D=128, bs=32, lw=64, S=4, bias=True),
    "fp16_bs128": dict(B=1, HQ=2, HKV=2, HI=1, T=400, Sk=700, D=128, bs=128, lw=200, S=3, dtype=torch.float16),
}


@pytest.mark.parametrize("name", list(CASES))
def test_fwd_matches_oracle(dev, name):
    c = dict(CASES[name])
    bs, lw = c["bs"], c["lw"]
    q, k, v, bi, pos, bias = _case(1 + list(CASES).index(name), **c)
    scale = 1 / math.sqrt(c["D"])
    o, lse, ro, rl = _run(dev, q, k, v, bi, pos, bias, bs, lw, scale)
    assert_close_lowp(o, ro, c.get("dtype", torch.bfloat16), TOL, f"forward {name}: o")
    assert (lse - rl).abs().max().item() <= TOL


F32_CASES = {
    "f32_self_bs64": dict(B=2, HQ=2, HKV=2, HI=1, T=300, Sk=300, D=128, bs=64, lw=128, S=4),
    "f32_prefix_bias": dict(B=1, HQ=2, HKV=1, HI=1, T=130, Sk=1000, D=128, bs=32, lw=256, S=5, bias=True),
    "f32_packed_d64": dict(B=1, HQ=4, HKV=2, HI=2, T=257, Sk=257, D=64, bs=16, lw=40, S=3, packed=True),
}


@pytest.mark.parametrize("name", list(F32_CASES))
def test_fwd_fp32_matches_oracle(dev, name):
    """fp32 operands on v_mfma_f32_32x32x2_f32 (fp32 products and sums): relative
    error of o and lse within 1e-5 of the fp64 oracle (the fp32 bar)."""
    c = dict(F32_CASES[name])
    bs, lw = c["bs"], c["lw"]
    q, k, v, bi, pos, bias = _case(40 + list(F32_CASES).index(name), dtype=torch.float32, **c)
    scale = 1 / math.sqrt(c["D"])
    o, lse, ro, rl = _run(dev, q, k, v, bi, pos, bias, bs, lw, scale)
    rel_o = (o - ro).abs().max().item() / ro.abs().max().item()
    fin = torch.isfinite(rl)
    assert torch.equal(torch.isfinite(lse), fin)
    rel_l = (lse[fin] - rl[fin]).abs().max().item() / rl[fin].abs().max().item()
    from parity_report import report
    report(f"[err] forward fp32 {name}: o max rel {rel_o:.3e}, lse max rel {rel_l:.3e} (bar 1e-5)")
    assert rel_o <= 1e-5 and rel_l <= 1e-5, (rel_o, rel_l)


@pytest.mark.parametrize("name", ["self_bs64", "bias", "gqa_hi"])
def test_tail_split_matches_whole_tiles(dev, name):
    """The tail split (a last round of tiles filling at most a fifth of the GPU
    runs as four workgroups per tile over quarters of their key chunks, then a
    merge) against every tile whole and the oracle: these small launches are
    one such round, so the split takes every tile."""
    import ctypes
    from srswa import _lib
    c = dict(CASES[name])
    bs, lw = c["bs"], c["lw"]
    q, k, v, bi, pos, bias = _case(40 + list(CASES).index(name), **c)
    scale = 1 / math.sqrt(c["D"])
    B, T, HQ, D = q.shape
    Sk = k.shape[1]
    seg = ops._seg_from_positions(pos.to(dev), T, Sk, dev)
    args = dict(block_size=bs, local_window=lw, scale=scale, seg=seg, bias=None if bias is None else bias.to(dev))
    qd, kd, vd, bd = q.to(dev), k.to(dev), v.to(dev), bi.to(dev)
    o_s, l_s = ops.gather_fwd(qd, kd, vd, bd, **args)
    o_w, l_w = ops.gather_fwd(qd, kd, vd, bd, tail_split=False, **args)
    dense = None
    if bias is not None:
        dense = O.bias_slots_to_dense(bias.double(), bi[:, 0], -(-Sk // bs))
    ro, rl = O.gather_attention(q.double().transpose(1, 2), k.double().transpose(1, 2),
                                v.double().transpose(1, 2), bi, pos, bs, scale, lw, blk_bias_dense=dense)
    ro, rl = ro.transpose(1, 2), rl.transpose(1, 2)
    for o, l, what in ((o_s, l_s, "split"), (o_w, l_w, "whole")):
        assert_close_lowp(o.cpu().double(), ro, c.get("dtype", torch.bfloat16), TOL, f"forward {name} {what}: o")
        assert (l.cpu().double() - rl).abs().max().item() <= TOL
    # the two forms of the same rows against each other: only their rounding differs
    d_o = (o_s.double() - o_w.double()).abs().max().item()
    d_l = (l_s.double() - l_w.double()).abs().max().item()
    report_error(f"forward {name} split vs whole: o", o_s, o_w, TOL)
    assert d_o <= TOL and d_l <= 1e-4, (d_o, d_l)
    # the split must have happened: one partial round of tiles
    a = _lib.FwdArgs()
    a.B, a.T, a.Sk, a.HQ, a.HKV, a.HI, a.D, a.S = B, T, Sk, HQ, k.shape[2], bi.shape[1], D, bi.shape[-1]
    a.q = a.k = a.v = a.out = qd.data_ptr()
    a.idx = bd.data_ptr()
    a.block_size, a.local_window, a.scale = bs, lw, scale
    a.dtype = _lib.dtype_code(q.dtype)
    ntiles = B * HQ * (-(-T // 64))
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    nws = _lib.lib().srswa_gather_fwd_workspace(ctypes.byref(a))
    assert (nws > 0) == (ntiles * 5 <= 4 * cus), (nws, ntiles, cus)
