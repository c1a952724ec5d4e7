"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the pinned oracle).  CPU: the oracle still reproduces them.  GPU: the HIP
kernels, through the C ABI, match them (bars as in the other parity tests)."""

import math
import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
from load import load  # noqa: E402
from oracle import srswa_oracle as O  # noqa: E402
from tolerance import assert_close_lowp  # noqa: E402


def test_oracle_reproduces_fixtures():
    d = load("decode")
    out = O.decode_attend(d["q"].double(), d["k"].double(), d["v"].double(), d["topi"], d["bias"].double(),
                          d["valid"], d["q_pos"], d["block_size"], d["local_window"], d["scale"])
    assert (out - d["out"]).abs().max() < 1e-10
    g = load("gather")
    Sk = g["k"].shape[2]
    dense = O.bias_slots_to_dense(g["bias"].double(), g["block_indices"][:, 0], -(-Sk // g["block_size"]))
    o, lse = O.gather_attention(g["q"].double(), g["k"].double(), g["v"].double(), g["block_indices"],
                                g["position_ids"], g["block_size"], g["scale"], g["local_window"],
                                blk_bias_dense=dense)
    assert (o - g["o"]).abs().max() < 1e-10
    x = load("indexer")
    sc = O.meanpool_block_scores(x["q"], x["k"].float(), x["q_pos"], x["block_size"], x["local_blocks"])
    assert torch.equal(O.topk_blocks(sc, x["topk"]), x["idx"])
    b = load("blockmax")
    out = O.block_max_scores(b["q"].double(), b["k"].double(), b["pos"], b["seg"], b["block_size"], b["nblk"],
                             b["local_window"])
    assert torch.equal(torch.isfinite(out), torch.isfinite(b["out"]))
    r = load("router")
    xi, bias, valid = O.infer_route_select(r["scores"], r["cand"], r["idx_scale"], r["floor"], r["sigma"],
                                           r["K"], r["topm"])
    assert torch.equal(xi, r["topi"]) and torch.equal(valid, r["valid"])
    # fp32 logs of torch's vectorised CPU path differ in the last bits across
    # host CPUs, so the bias is compared to a few ulps
    assert (bias - r["bias"]).abs().max().item() <= 1e-6 * max(1.0, r["bias"].abs().max().item())


@pytest.mark.gpu
def test_kernels_match_fixtures(dev):
    import srswa
    from srswa import ops, sparse_gather_triton as SG

    d = load("decode")
    out = srswa.decode_attend(d["q"].to(dev), d["k"].to(dev), d["v"].to(dev), d["topi"].to(dev),
                              d["bias"].to(dev), d["valid"].to(dev), d["q_pos"].to(dev), d["block_size"],
                              d["local_window"], d["scale"]).cpu()
    assert (out.double() - d["out"]).abs().max().item() <= 2e-2

    g = load("gather")
    T, Sk = g["q"].shape[2], g["k"].shape[2]
    qd, kd, vd = (g[n].to(dev).transpose(1, 2).requires_grad_() for n in ("q", "k", "v"))
    bd = g["bias"].to(dev).requires_grad_()
    seg = ops._seg_from_positions(g["position_ids"].to(dev), T, Sk, dev)
    o = ops.GatherAttnFn.apply(qd, kd, vd, g["block_indices"].to(dev), seg, bd, g["block_size"], g["scale"],
                               g["local_window"])
    o.backward(g["do"].to(dev).transpose(1, 2))
    assert_close_lowp(o.detach().cpu().transpose(1, 2), g["o"], torch.bfloat16, 2e-2, "o")
    for n, t in (("dq", qd), ("dk", kd), ("dv", vd)):
        assert_close_lowp(t.grad.cpu().transpose(1, 2), g[n], torch.bfloat16, 2e-2, n)
    assert (bd.grad.cpu().double() - g["dbias"]).abs().max().item() <= 2e-2

    x = load("indexer")
    for hc_key, sc_key, id_key in ((None, "scores", "idx"), ("head_cls", "scores_hc", "idx_hc")):
        hc = None if hc_key is None else x[hc_key].to(dev)
        idx, sc = srswa.index_meanpool_topk(x["q"].to(dev), x["k"].transpose(1, 2).contiguous().to(dev),
                                            x["q_pos"].to(dev), block_size=x["block_size"],
                                            local_blocks=x["local_blocks"], topk=x["topk"], head_cls=hc,
                                            return_scores=True)
        ref = x[sc_key]
        valid = ref > O.SCORE_NEG * 0.5
        assert torch.equal(sc.cpu() > O.SCORE_NEG * 0.5, valid)
        scale = ref.abs().masked_fill(~valid, 0).amax(-1, keepdim=True).clamp(min=1.0)
        assert (((sc.cpu().double() - ref) / scale).abs() * valid).max().item() <= 1e-5
        ties = O.near_tie_rows(ref, x["topk"])
        same = (torch.sort(idx.cpu().long(), -1).values == torch.sort(x[id_key], -1).values).all(-1)
        assert (same | ties).all()

    b = load("blockmax")
    got = SG.triton_block_max_score(b["q"].to(dev), b["k"].to(dev), b["pos"].to(dev), b["seg"].to(dev),
                                    b["block_size"], b["nblk"], b["local_window"]).cpu().double()
    fin = torch.isfinite(b["out"])
    assert torch.equal(torch.isfinite(got), fin)
    assert (got[fin] - b["out"][fin]).abs().max().item() <= 1e-3 * max(1.0, b["out"][fin].abs().max().item())

    r = load("router")
    p = dict(idx_scale=r["idx_scale"], floor=r["floor"], sigma=r["sigma"], K=r["K"], topm=r["topm"])
    for sfx, cand in (("", r["cand"].to(dev)), ("_short", None)):
        xi, bias, valid = ops.dash_route(r["scores" + sfx].to(dev), cand, p)
        assert torch.equal(xi.cpu(), r["topi" + sfx]) and torch.equal(valid.cpu(), r["valid" + sfx])
        ref = r["bias" + sfx]
        assert ((bias.cpu() - ref).abs() <= 1e-5 * ref.abs().clamp(min=1.0)).all()
