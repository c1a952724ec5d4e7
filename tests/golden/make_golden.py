"""Write the golden fixtures of tests/golden/ from the pinned CPU oracle.

The reference ships no golden vectors for this path, so these fixtures are
produced by oracle/srswa_oracle.py (itself pinned by tests/test_oracle_pins.py)
on small seeded inputs that exercise the edge cases: duplicates, empty slots,
blocks overlapping the window, packing, prefix caches, ties in the top-k.
Run from the repo root: ``python tests/golden/make_golden.py``.
"""

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import srswa_oracle as O  # noqa: E402


def _bf16(x):
    return x.to(torch.bfloat16).float()


def _bits(x):
    """bf16-valued float tensor -> its bf16 bit pattern (uint16), stored exactly."""
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def decode_case():
    g = torch.Generator().manual_seed(101)
    B, H, Hkv, Lq, S, D, bs, lw, K = 2, 4, 2, 1, 500, 64, 32, 96, 6
    q, k, v = (_bf16(torch.randn(*s, generator=g)) for s in ((B, H, Lq, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    topi = torch.randint(0, S // bs, (B, Lq, K), generator=g)
    topi[:, :, 1] = topi[:, :, 0]
    topi[1, 0, 2] = 450 // bs
    bias = torch.randn(B, Lq, K, generator=g)
    valid = torch.rand(B, Lq, K, generator=g) > 0.25
    q_pos = torch.tensor([[499], [450]])
    out = O.decode_attend(q.double(), k.double(), v.double(), topi, bias.double(), valid, q_pos, bs, lw,
                          1 / math.sqrt(D))
    return dict(q_bf16=_bits(q), k_bf16=_bits(k), v_bf16=_bits(v), topi=topi.numpy(), bias=bias.numpy(),
                valid=valid.numpy(), q_pos=q_pos.numpy(), block_size=bs, local_window=lw,
                scale=1 / math.sqrt(D), out=out.numpy())


def gather_case():
    g = torch.Generator().manual_seed(102)
    B, H, T, Sk, D, bs, lw, S = 1, 2, 150, 214, 64, 16, 40, 4
    q = _bf16(torch.randn(B, H, T, D, generator=g))
    k = _bf16(torch.randn(B, H, Sk, D, generator=g))
    v = _bf16(torch.randn(B, H, Sk, D, generator=g))
    bi = torch.randint(-1, Sk // bs, (B, 1, T, S), generator=g)
    bi[..., 2] = bi[..., 1]
    pos = torch.cat([torch.arange(Sk - T, Sk - T + 60), torch.arange(T - 60)])[None]   # prefix + packed restart
    bias = torch.randn(B, T, S, generator=g)
    do = _bf16(torch.randn(B, H, T, D, generator=g))
    qd, kd, vd = (x.double().requires_grad_() for x in (q, k, v))
    bd = bias.double().requires_grad_()
    dense = O.bias_slots_to_dense(bd, bi[:, 0], -(-Sk // bs))
    o, lse = O.gather_attention(qd, kd, vd, bi, pos, bs, 1 / math.sqrt(D), lw, blk_bias_dense=dense)
    o.backward(do.double())
    return dict(q_bf16=_bits(q), k_bf16=_bits(k), v_bf16=_bits(v), block_indices=bi.numpy(),
                position_ids=pos.numpy(), bias=bias.numpy(), do_bf16=_bits(do), block_size=bs, local_window=lw, scale=1 / math.sqrt(D),
                o=o.detach().numpy(), lse=lse.detach().numpy(), dq=qd.grad.numpy(), dk=kd.grad.numpy(),
                dv=vd.grad.numpy(), dbias=bd.grad.numpy())


def indexer_case():
    g = torch.Generator().manual_seed(103)
    B, HI, Lq, S, d, bs, lb, K = 2, 2, 2, 600, 64, 32, 2, 5
    q = torch.randn(B, HI, Lq, d, generator=g)
    k = _bf16(torch.randn(B, HI, S, d, generator=g))
    k[:, :, 96:128] = k[:, :, 32:64]          # two blocks with identical keys -> exact score tie
    q_pos = torch.tensor([[599, 400], [500, 65]])
    hc = torch.randn(d, generator=g)
    sc = O.meanpool_block_scores(q, k, q_pos, bs, lb)
    sch = O.meanpool_block_scores(q, k, q_pos, bs, lb, head_cls=hc)
    return dict(q=q.numpy(), k_bf16=_bits(k), q_pos=q_pos.numpy(), head_cls=hc.numpy(), block_size=bs,
                local_blocks=lb, topk=K, scores=sc.numpy(), scores_hc=sch.numpy(),
                idx=O.topk_blocks(sc, K).numpy(), idx_hc=O.topk_blocks(sch, K).numpy())


def blockmax_case():
    g = torch.Generator().manual_seed(104)
    B, C, Sk, D, bs, lw = 2, 70, 300, 64, 32, 50
    q = _bf16(torch.randn(B, C, D, generator=g))
    k = _bf16(torch.randn(B, Sk, D, generator=g))
    pos = torch.randint(0, Sk, (B, C), generator=g)
    seg = torch.randint(0, 40, (B, C), generator=g)
    nblk = -(-Sk // bs)
    out = O.block_max_scores(q.double(), k.double(), pos, seg, bs, nblk, lw)
    return dict(q_bf16=_bits(q), k_bf16=_bits(k), pos=pos.numpy(), seg=seg.numpy(), block_size=bs,
                local_window=lw,
                nblk=nblk, out=out.numpy())


def router_case():
    """DASH router: shipped parameters (K 12, top-M 16, sigma 1, floor 1e-4), a
    page mask with one row whose masked set is empty (fallback to every remote
    block), equal scores (tie order), a short row (nblk < M) in its own case."""
    g = torch.Generator().manual_seed(105)
    B, Lq, nblk = 2, 5, 90
    sc = (torch.randn(B, Lq, nblk, generator=g) * 0.3).float()
    sc[..., 80:] = O.SCORE_NEG                          # local / future blocks
    sc[0, 1, 10:20] = 0.5                               # ties
    sc[1, 2, 5] = float("nan")
    cand = torch.rand(B, Lq, nblk, generator=g) > 0.4
    cand[1, 3] = False                                  # empty candidate set -> fallback
    idx_scale, floor, sigma, K, topm = 128.0 / math.sqrt(128), 1e-4, 1.0, 12, 16
    xi, bias, valid = O.infer_route_select(sc, cand, idx_scale, floor, sigma, K, topm)
    sc2 = sc[:, :, :10].clone()
    sc2[..., 7:] = O.SCORE_NEG
    xi2, bias2, valid2 = O.infer_route_select(sc2, None, idx_scale, floor, sigma, K, topm)
    return dict(scores=sc.numpy(), cand=cand.numpy(), idx_scale=idx_scale, floor=floor, sigma=sigma, K=K,
                topm=topm, topi=xi.numpy(), bias=bias.numpy(), valid=valid.numpy(),
                scores_short=sc2.numpy(), topi_short=xi2.numpy(), bias_short=bias2.numpy(),
                valid_short=valid2.numpy())


def main():
    for name, fn in (("decode", decode_case), ("gather", gather_case), ("indexer", indexer_case),
                     ("blockmax", blockmax_case), ("router", router_case)):
        d = fn()
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **{k: np.asarray(v) for k, v in d.items()})
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
