"""HIP-graph capture of the serving entry points (the reference's serving
kernels run under CUDA-graph replay, WHL!layers/attention/unlimited_dash_ops/
attend_triton.py:37-73).  Each case is captured once on a non-default stream
with torch.cuda.graph, then replayed several times with new contents in its
static input buffers and eager work and synchronisations between the
replays; every replay must equal the eager result bit for bit.

* the DASH serving decode step: per-page summary tail refresh -> summary
  scores -> router -> paged decode;
* srswa_gather_decode_noalloc (split-K records in the library's static array);
* the gather-KL forward (row-sparse, tile kernels forked onto the caller's
  second stream and joined back) and its backward.

No step of these paths records a memset: the library has none, and every
buffer the captured region allocates comes from the graph's pool."""

import ctypes
import math

import pytest
import torch

pytestmark = pytest.mark.gpu
REPLAYS = 3


def _capture(fn, warm=2):
    """(graph, outputs of the captured call) with fn run eagerly on the side
    stream first (allocations of per-stream scratch, first-use set-up)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warm):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def _noise(dev):
    """eager work between replays (a reduction over many blocks, an elementwise op)"""
    x = torch.randn(1 << 20, device=dev)
    return float((x * 2.0).sum())


def test_graph_serving_decode_step(dev):
    from srswa import ops, unlimited_dash_ops as U, workloads as W
    B, H, D, K, BS, LW = 8, 10, 128, 8, 64, 512
    c = W.paged_decode_config(B=B, H=H, D=D, Lmax=8192, lo=1500, k=K, block_size=BS, local_window=LW, device=dev)
    bt, sl = c["block_table"].to(dev), c["seq_lens"].to(dev)
    cache = U.KBarCache(c["num_pages"], 128, dev)
    hc = torch.randn(128, device=dev)
    U.headcls_scores_prefill(idx_q=c["idx_q"], kv_cache=c["idx_k_cache"], block_table=bt,
                             cu_seqlens_q=torch.arange(B + 1, device=dev), seq_lens=sl, context_lens=sl - 1,
                             head_cls=hc, max_block=bt.shape[1], block_size=BS, local_blocks=LW // BS, cache=cache)
    p = dict(idx_scale=128.0 / math.sqrt(128), floor=1e-4, sigma=1.0, K=K, topm=16)
    q_static = c["q"].view(B, H, D).clone()
    iq_static = c["idx_q"].clone()
    out = torch.empty_like(q_static)

    def step():
        cache.refresh_tail(kv_cache=c["idx_k_cache"], block_table=bt, seq_lens=sl, head_cls=hc, block_size=BS,
                           tail_pages=2)
        sc = U.headcls_scores_decode(idx_q=iq_static, cache=cache, block_table=bt, seq_lens=sl,
                                     max_block=bt.shape[1], block_size=BS, local_blocks=LW // BS, decode_query_len=1)
        topi, bias, _ = ops.dash_route(sc[0][:, None, :], None, p, attend_ids=True)
        topi = topi[:, 0]
        U.dash_sparse_attn_decode(q_static, c["k_cache"], c["v_cache"], topi[None].expand(H, B, K),
                                  bias[:, 0][None].expand(H, B, K), bt, sl, H, c["scale"], out, 1,
                                  local_blocks=LW // BS, sparse_block_size=BS)
        return topi

    gen = torch.Generator(device=dev).manual_seed(5)
    inputs = [(torch.randn(q_static.shape, device=dev, generator=gen).to(q_static.dtype),
               torch.randn(iq_static.shape, device=dev, generator=gen).to(iq_static.dtype)) for _ in range(REPLAYS)]
    eager = []
    for qi, ii in inputs:
        q_static.copy_(qi)
        iq_static.copy_(ii)
        ids = step()
        eager.append((out.clone(), ids.clone()))
    g, ids_g = _capture(step)
    for (qi, ii), (o_ref, ids_ref) in zip(inputs, eager):
        q_static.copy_(qi)
        iq_static.copy_(ii)
        _noise(dev)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ids_g, ids_ref)
        assert torch.equal(out, o_ref)


def test_graph_noalloc_decode(dev):
    from srswa import _lib, ops, workloads as W
    c = W.decode_config(B=6, H=10, D=128, Lmax=12000, lo=2000, k=8)
    q = c["q"].to(dev)
    args = (q, c["k_cache"].to(dev), c["v_cache"].to(dev), c["block_idx"].to(dev), c["q_pos"].to(dev))
    launch, out, lse = ops.prepare_gather_decode(*args, block_size=c["block_size"], local_window=c["local_window"],
                                                 scale=c["scale"], return_lse=True)
    a = _lib.DecodeArgs.from_buffer_copy(launch.args)

    def call():
        _lib.check(_lib.lib().srswa_gather_decode_noalloc(ctypes.byref(a), _lib.stream_ptr(dev)),
                   "srswa_gather_decode_noalloc")

    gen = torch.Generator(device=dev).manual_seed(6)
    inputs = [torch.randn(q.shape, device=dev, generator=gen).to(q.dtype) for _ in range(REPLAYS)]
    eager = []
    for qi in inputs:
        q.copy_(qi)
        launch()                                     # the workspace entry point, eagerly
        eager.append((out.clone(), lse.clone()))
    g, _ = _capture(call)
    for qi, (o_ref, l_ref) in zip(inputs, eager):
        q.copy_(qi)
        _noise(dev)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, o_ref) and torch.equal(lse, l_ref)


def test_graph_gather_kl_fwd_bwd_with_side_stream(dev):
    from srswa import kl as KL
    g0 = torch.Generator().manual_seed(8)
    B, HI, HQ, HKV, T, Sk, D, K = 1, 1, 4, 2, 700, 1000, 128, 6
    q_idx = (torch.randn(B, HI, T, D, generator=g0) * D ** -0.5).to(torch.bfloat16).to(dev)
    idx_k = torch.randn(B, Sk, D, generator=g0).to(torch.bfloat16).to(dev)
    q_main = torch.randn(B, HQ, T, D, generator=g0).to(torch.bfloat16).to(dev)
    k_main = torch.randn(B, HKV, Sk, D, generator=g0).to(torch.bfloat16).to(dev)
    nblk = -(-Sk // 64)
    sel = torch.stack([torch.randperm(nblk, generator=g0)[:K] for _ in range(T)]).view(B, HI, T, K)
    for tau in range(0, -(-T // 64), 2):                 # tiles of both kernel families
        sel[:, :, 64 * tau:64 * tau + 64] = torch.randperm(nblk, generator=g0)[:K]
    sel = sel.to(torch.int32).to(dev)
    pos = (torch.arange(T) + (Sk - T)).expand(B, T).to(torch.int32).to(dev)
    grad = torch.randn(B, HI, T, generator=g0).to(dev)
    kw = dict(block_size=64, local_window=128, scaling=D ** -0.5)

    def call():
        kl, valid, dsel = KL.kl_forward(q_idx, idx_k, q_main, k_main, sel, pos, **kw)
        dq, dk = KL.kl_backward(grad, q_idx, idx_k, sel, dsel, block_size=64)
        return kl, valid, dq, dk

    gen = torch.Generator(device=dev).manual_seed(9)
    inputs = [(torch.randn(q_idx.shape, device=dev, generator=gen).mul(D ** -0.5).to(q_idx.dtype),
               torch.randn(grad.shape, device=dev, generator=gen)) for _ in range(REPLAYS)]
    eager = []
    for qi, gi in inputs:
        q_idx.copy_(qi)
        grad.copy_(gi)
        eager.append(tuple(t.clone() for t in call()))
    g, outs = _capture(call)
    for (qi, gi), ref in zip(inputs, eager):
        q_idx.copy_(qi)
        grad.copy_(gi)
        _noise(dev)
        g.replay()
        torch.cuda.synchronize()
        for got, r in zip(outs, ref):
            assert torch.equal(got, r)
