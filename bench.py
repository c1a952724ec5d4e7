#!/usr/bin/env python3
"""SR-SWA benchmark on one MI355X.

Default workload (BASELINE metric): decode gather-attention, config 3 --
B=64 sequences, KV lengths log-uniform in [4k, 128k] (contiguous bf16 cache
[64, 131072, 10, 128]), 10 heads, head_dim 128, block 64, 8 selected blocks
(512 reference tokens) + a 512-token window per (sequence, head).  One "step"
is one decode attention pass over the batch (64 tokens).

Prints ONE JSON line with value = tokens/s, the roofline object of the decode
kernel (HIP-event timed over the timed region) and the CPU baseline (this
repo's oracle restatement of the reference's PyTorch decode path, timed on a
bounded sample on the host cores).  ``--config`` selects the other
configurations for ad-hoc runs; the driver uses the default.
"""

from __future__ import annotations

import argparse
import json
import math
import types
import os
import re
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "unlimited-ocr_amd"))

HBM_PEAK_GBS = 8000.0
METRIC = "decode sparse-attn tokens/s + HBM GB/s (% peak), B=64 KV=64k, 512 refs"


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _pmc_traffic(name):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration), read from profiles/<name>.md if present."""
    path = os.path.join(REPO, "profiles", f"{name}.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def host_threads():
    """Threads the CPU baseline uses: the CPUs this process may run on, capped
    by OMP_NUM_THREADS when set (a one-GPU box grants its job a 16-core share
    of a larger host and sets OMP_NUM_THREADS=16; more threads than cores of
    that share would only oversubscribe it)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def host_info():
    """CPU model and core counts of the host the baseline ran on."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity_cpus": aff,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_baseline_decode(budget_s=12.0, threads=None):
    """Time the oracle's restatement of the reference decode (_decode_attend,
    dense fp32 over all cached keys) on host cores, one config-3 sequence at a
    time, until ``budget_s`` is spent.  Returns the baseline dict."""
    import torch
    sys.path.insert(0, REPO)
    from oracle import srswa_oracle as O
    from srswa import workloads as W

    n_thr = threads or host_threads()
    torch.set_num_threads(n_thr)
    lengths = W.decode_lengths(64)
    H, D, BS, LW, K = 10, 128, 64, 512, 8
    idx_all = W.decode_block_indices(lengths, H, K, BS, LW)
    g = torch.Generator().manual_seed(W.SEED0 + 3)
    t_dense = t_gather = 0.0
    n = 0
    order = list(range(64))
    for b in order:
        Lb = int(lengths[b])
        q = torch.randn(1, H, 1, D, generator=g).to(torch.bfloat16)
        kk = torch.randn(1, H, Lb, D, generator=g).to(torch.bfloat16)
        vv = torch.randn(1, H, Lb, D, generator=g).to(torch.bfloat16)
        ti = idx_all[b:b + 1, :, None, :].long()
        qp = torch.tensor([[Lb - 1]])
        t0 = time.perf_counter()
        O.decode_attend(q, kk, vv, ti, torch.zeros(ti.shape), ti >= 0, qp, BS, LW, 1 / math.sqrt(D))
        t1 = time.perf_counter()
        O.decode_attend_gather(q[:, :, 0], kk.transpose(1, 2), vv.transpose(1, 2), idx_all[b:b + 1],
                               qp[:, 0], BS, LW, 1 / math.sqrt(D))
        t2 = time.perf_counter()
        t_dense += t1 - t0
        t_gather += t2 - t1
        n += 1
        if t_dense + t_gather > budget_s:
            break
    return {
        "value": n / t_dense, "unit": "tokens/s", "cores": n_thr, "kind": "port",
        "sample": (f"{n} of 64 config-3 sequences (L_b {int(lengths[:n].min())}..{int(lengths[:n].max())}), "
                   f"oracle restatement of _decode_attend (fp32, dense over all cached keys, "
                   f"HF/modeling_deepseekv2.py:454-481); gather-form restatement "
                   f"{n / t_gather:.1f} tokens/s"),
        "gather_form_tokens_per_s": n / t_gather,
        "host": host_info(),
    }


def bench_decode(args):
    import torch
    import srswa
    from srswa import ops, workloads as W

    dev = torch.device("cuda:0")
    B, H, D, Lmax, K, BS, LW = 64, 10, 128, 131072, 8, 64, 512
    _log(f"allocating config-3 cache [{B},{Lmax},{H},{D}] bf16 x2 on {dev}")
    c = W.decode_config(B=B, H=H, D=D, Lmax=Lmax, k=K, block_size=BS, local_window=LW, device=dev)
    idx = c["block_idx"].to(dev)
    qpos = c["q_pos"].to(dev)
    launch, out, _ = ops.prepare_gather_decode(
        c["q"], c["k_cache"], c["v_cache"], idx, qpos, block_size=BS, local_window=LW,
        scale=c["scale"])
    torch.cuda.synchronize()
    _log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        launch()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream(dev)
    # (1) warm: the K steps back to back.  Every step reads the same 336 MB, and
    # MI355X's 256 MB Infinity Cache may serve part of it from the second step on.
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(st)
    for _ in range(args.steps):
        launch()
    e1.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_warm = e0.elapsed_time(e1) / args.steps
    _log(f"warm: {args.steps} steps back to back, {ms_warm * 1e3:.2f} us/step (HIP events), "
         f"wall {wall * 1e6 / args.steps:.2f} us/step")
    # (2) cold (the reported value): the same K steps back to back, alternating
    # between two copies of the config-3 instance in different memory (2 x 43 GB).
    # Each step's 336 MB read set then follows another step's 336 MB of other
    # data, so the 256 MB Infinity Cache holds none of it; one event pair brackets
    # all K steps, as in (1).  A real decode step meets its layer's cache cold the
    # same way: the other layers' caches pass through between two reads of one.
    _log("cold: cloning the cache into a second instance")
    kc2, vc2 = c["k_cache"].clone(), c["v_cache"].clone()
    launch2, _, _ = ops.prepare_gather_decode(
        c["q"], kc2, vc2, idx, qpos, block_size=BS, local_window=LW, scale=c["scale"])
    pair = (launch, launch2)
    for i in range(4):
        pair[i % 2]()
    torch.cuda.synchronize()
    e0.record(st)
    for i in range(args.steps):
        pair[i % 2]()
    e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    del launch2, pair, kc2, vc2
    _log(f"cold: {args.steps} steps back to back, alternating two cache instances: {ms * 1e3:.2f} us/step")
    nbytes = W.decode_bytes(B, H, D, K, BS, LW)
    achieved = nbytes / (ms * 1e-3) / 1e9
    res = {
        "metric": METRIC,
        "value": B / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "cache": ("cold: the K steps alternate between two copies of the instance in different memory, "
                  "so each step's 336 MB follows 336 MB of other data and misses the 256 MB Infinity Cache"),
        "warm": {"ms_per_step": ms_warm, "tokens_per_s": B / (ms_warm * 1e-3),
                 "achieved_GBs": nbytes / (ms_warm * 1e-3) / 1e9,
                 "frac": nbytes / (ms_warm * 1e-3) / 1e9 / HBM_PEAK_GBS,
                 "note": "the same K steps back to back (read set 336 MB, may hit the Infinity Cache)"},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 cache, seeded per-head block indices)",
        "config": {"workload": "config 3: decode gather-attention, B=64, KV log-uniform 4k..128k "
                               "(contiguous [64,131072,10,128] bf16 cache), 10 heads, D=128, block 64, "
                               "top-8 blocks (512 refs) + 512-token window",
                   "B": B, "heads": H, "head_dim": D, "kv_max": Lmax, "block_size": BS,
                   "topk_blocks": K, "local_window": LW, "mean_kv_len": float(c["seq_lens"].float().mean()),
                   "parallelism": "single GPU"},
        "hbm_gbs": achieved,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": _pmc_traffic("decode_cfg3_traffic"),
                     "algorithmic_bytes_per_launch": nbytes,
                     "kernel": "srswa::decode_kernel<bf16,bf16,128,8> + decode_merge_kernel (one step, "
                               "cold cache)"},
    }
    # parity spot check of the timed output against the oracle on 2 sequences
    if not args.no_check:
        sys.path.insert(0, REPO)
        from oracle import srswa_oracle as O
        err = 0.0
        for b in (0, B - 1):
            Lb = int(c["seq_lens"][b])
            kk = c["k_cache"][b:b + 1, :Lb].cpu()
            vv = c["v_cache"][b:b + 1, :Lb].cpu()
            ref = O.decode_attend_gather(c["q"][b:b + 1].cpu(), kk, vv, c["block_idx"][b:b + 1],
                                         c["q_pos"][b:b + 1], BS, LW, c["scale"])
            err = max(err, (out[b:b + 1].cpu().double() - ref.double()).abs().max().item())
        res["spot_check_max_abs_err"] = err
        _log(f"spot check vs oracle: max-abs {err:.3e}")
    del c, out, launch
    torch.cuda.empty_cache()
    if not args.no_cpu:
        _log("cpu baseline (bounded sample)")
        res["cpu_baseline"] = cpu_baseline_decode(args.cpu_budget)
    else:
        res["cpu_baseline"] = None
    return res


def _time_launches(fn, steps, warmup, dev):
    """Average ms per call of ``fn`` (HIP events on torch's current stream, which
    is the stream the library launches on)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        fn()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def bench_indexer(args):
    """Config 2: head_cls/mean-pool indexer, B=32 decode queries, 10 heads,
    L=32768, top-8 per head (HBM-bound streaming of the eligible keys)."""
    import torch
    from srswa import ops, workloads as W
    dev = torch.device("cuda:0")
    B, H, D, L, BS, LW, K = 32, 10, 128, 32768, 64, 512, 8
    c = W.indexer_config(B=B, H=H, D=D, L=L, device=dev)
    launch, idx, _, _ = ops.prepare_index_meanpool_topk(c["q"], c["k"], c["q_pos"].to(dev), block_size=BS,
                                                         local_blocks=LW // BS, topk=K)
    ms = _time_launches(launch, args.steps, args.warmup, dev)
    nbytes = W.indexer_bytes(B, H, D, L, BS, LW)
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {"metric": "indexer queries/s + HBM GB/s (config 2)", "value": B / (ms * 1e-3), "unit": "queries/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16 keys, fp32 scores",
           "data": "synthetic (seeded; 5% hot blocks shifted +3 along the query direction)",
           "config": {"workload": "config 2: mean-pool indexer, B=32, 10 heads, L=32768, block 64, top-8",
                      "B": B, "heads": H, "kv_len": L, "block_size": BS, "topk_blocks": K},
           "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": gbs / HBM_PEAK_GBS, "traffic": _pmc_traffic("indexer_cfg2_traffic"),
                        "algorithmic_bytes_per_launch": nbytes,
                        "kernel": "srswa::index_summary_kernel<bf16,128,false> + topk_rows_kernel"}}
    if not args.no_check:
        res["selection_check"] = indexer_selection_check(c, idx, BS, LW, K)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline_indexer(args.cpu_budget)
    return res


def indexer_selection_check(c, idx, BS, LW, K, seqs=(0, 15, 31)):
    """Selected ids of the timed launch against the oracle on three whole
    sequences (10 heads each): rows compared, rows whose set matches exactly,
    near-tie rows (k-th and (k+1)-th oracle scores closer than
    1e-4 * max(1, |s_k|)), near-tie rows that differ, and rows that differ
    outside near ties."""
    import torch
    sys.path.insert(0, REPO)
    from oracle import srswa_oracle as O
    tot = {"rows": 0, "exact": 0, "near_tie": 0, "near_tie_differ": 0, "mismatched": 0}
    for b in seqs:
        q = c["q"][b:b + 1].cpu()
        k = c["k"][b:b + 1].cpu().float()
        ref = O.meanpool_block_scores(q[:, :, None, :], k.permute(0, 2, 1, 3), c["q_pos"][b:b + 1].cpu()[:, None],
                                      BS, LW // BS)[:, :, 0]
        want = O.topk_blocks(ref, K)
        ties = O.near_tie_rows(ref, K)
        got = idx[b:b + 1].cpu().long()
        same = (torch.sort(got, -1).values == torch.sort(want, -1).values).all(-1)
        tot["rows"] += same.numel()
        tot["exact"] += int(same.sum())
        tot["near_tie"] += int(ties.sum())
        tot["near_tie_differ"] += int(((~same) & ties).sum())
        tot["mismatched"] += int(((~same) & (~ties)).sum())
    tot["sequences"] = list(seqs)
    _log(f"selection check: {tot}")
    return tot


def cpu_baseline_indexer(budget_s):
    import torch
    sys.path.insert(0, REPO)
    from oracle import srswa_oracle as O
    from srswa import workloads as W
    n_thr = host_threads()
    torch.set_num_threads(n_thr)
    g = torch.Generator().manual_seed(1)
    H, D, L, BS, LW = 10, 128, 32768, 64, 512
    t = 0.0
    n = 0
    while t < budget_s and n < 32:
        q = torch.randn(1, H, 1, D, generator=g)
        k = torch.randn(1, H, L, D, generator=g).to(torch.bfloat16)
        t0 = time.perf_counter()
        sc = O.meanpool_block_scores(q, k.float(), torch.tensor([[L - 1]]), BS, LW // BS)
        O.topk_blocks(sc, 8)
        t += time.perf_counter() - t0
        n += 1
    return {"value": n / t, "unit": "queries/s", "cores": n_thr, "kind": "port",
            "sample": f"{n} config-2 queries (10 heads x 32768 keys each), oracle restatement of "
                      f"_block_scores_infer head_cls + top-k (fp32)", "host": host_info()}


def _attn_dtype(args, c, names):
    """--dtype fp32: the legs' operands as fp32 (in place in ``c``); returns
    (dtype label, MFMA peak TFLOP/s, kernel type label)."""
    import torch
    if getattr(args, "dtype", "bf16") != "fp32":
        return "bf16", 2500.0, "bf16"
    for n in names:
        c[n] = c[n].to(torch.float32)
    return "fp32", 157.3, "float"


def bench_prefill(args):
    """Config 4: chunked prefill, B=4 x 2048 query rows at the tail of 65536 keys."""
    import torch
    from srswa import ops, workloads as W
    dev = torch.device("cuda:0")
    B, T, Sk, H, D, BS, LW, K = 4, 2048, 65536, 10, 128, 64, 512, 8
    c = W.prefill_config(B=B, T=T, Sk=Sk, H=H, D=D, device=dev)
    dtl, peak, kt = _attn_dtype(args, c, ("q", "k", "v"))
    idx = c["block_idx"].to(dev)
    fn = lambda: ops.gather_fwd(c["q"], c["k"], c["v"], idx, block_size=BS, local_window=LW, scale=c["scale"])
    ms = _time_launches(fn, args.steps, args.warmup, dev)
    wp, rp = W.attended_pairs(c["block_idx"], Sk, BS, LW)
    flops = (wp + rp) * H * 4 * D
    tfs = flops / (ms * 1e-3) / 1e12
    cpu = None if args.no_cpu else cpu_baseline_rows(c, Sk, T, BS, LW, args.cpu_budget, backward=False)
    return {"metric": "chunked-prefill tokens/s + MFMA TFLOP/s (config 4)", "value": B * T / (ms * 1e-3),
            "cpu_baseline": cpu,
            "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtl,
            "data": "synthetic (seeded N(0,1); top-8 per 64-query tile from the prefix)",
            "config": {"workload": "config 4: chunked prefill B=4, 2048 of 65536, 10 heads, block 64, "
                                   "top-8 + 512 window", "flops_per_step": flops},
            "roofline": {"bound": "mfma", "achieved": tfs, "peak": peak, "unit": "TFLOP/s",
                         "frac": tfs / peak, "traffic": None,
                         "kernel": f"srswa::fwd_kernel<{kt},128>"}}


def cpu_baseline_rows(c, Sk, T, BS, LW, budget_s, backward):
    """The dense masked attention the reference runs on the CPU for prefill /
    training (HF/_sparse_base_impl.py:1803-1836, restated by the oracle's
    ``gather_attention``), in fp32, on 64-row query tiles of sequence 0 spread
    evenly over the chunk (each tile against every key up to its last row, all
    10 heads), with autograd's backward when ``backward``.  Tiles until
    ``budget_s`` is spent; tokens/s = rows / time."""
    import torch
    sys.path.insert(0, REPO)
    from oracle import srswa_oracle as O
    n_thr = host_threads()
    torch.set_num_threads(n_thr)
    ntile = T // 64
    order = [int(i) for i in torch.linspace(0, ntile - 1, steps=min(ntile, 16)).round().tolist()]
    off = Sk - T
    t = 0.0
    rows = 0
    for m in order:
        t0r, t1r = m * 64, m * 64 + 64
        kend = off + t1r
        q = c["q"][0:1, t0r:t1r].cpu().float().transpose(1, 2)
        kk = c["k"][0:1, :kend].cpu().float().transpose(1, 2)
        vv = c["v"][0:1, :kend].cpu().float().transpose(1, 2)
        bi = c["block_idx"][0:1, :, t0r:t1r].long()
        pos = torch.arange(off + t0r, off + t1r)[None]
        if backward:
            q.requires_grad_()
            kk.requires_grad_()
            vv.requires_grad_()
            do = c["do"][0:1, t0r:t1r].cpu().float().transpose(1, 2)
        ts = time.perf_counter()
        o, _ = O.gather_attention(q, kk, vv, bi, pos, BS, c["scale"], LW)
        if backward:
            o.backward(do)
        t += time.perf_counter() - ts
        rows += t1r - t0r
        if t > budget_s:
            break
    return {"value": rows / t, "unit": "tokens/s", "cores": n_thr, "kind": "port",
            "sample": (f"{rows // 64} 64-row tiles of sequence 0 spread over the chunk, 10 heads, dense fp32 "
                       f"masked attention{' forward + backward' if backward else ''} against every key up to "
                       f"the tile (oracle restatement of the reference's eager path)"),
            "host": host_info()}


def bench_paged_prefill(args):
    """Config 4's chunked prefill over the serving (paged) cache: the drop-in
    for the backend's K10 ``dash_sparse_attn``.  B=4 requests, each 2048 query
    rows at the tail of 65536 keys in randomly ordered 64-key pages; config 4's
    per-tile top-8 blocks, one router row per query expanded over the 10 kv
    heads (stride 0, as the backend passes them); window 8 blocks."""
    import torch
    from srswa import unlimited_dash_ops as U, workloads as W
    dev = torch.device("cuda:0")
    B, T, Sk, H, D, BS, LW, K = 4, 2048, 65536, 10, 128, 64, 512, 8
    c = W.prefill_config(B=B, T=T, Sk=Sk, H=H, D=D, device=dev)
    nb = Sk // BS
    g = torch.Generator().manual_seed(W.SEED0 + 44)
    perm = torch.randperm(B * nb, generator=g)
    bt = perm.view(B, nb).to(torch.int32).to(dev)
    kvd = _kv_dtype(args)
    kc = torch.empty(B * nb, BS, H, D, dtype=kvd or torch.bfloat16, device=dev)
    vc = torch.empty_like(kc)
    for b in range(B):                       # scatter each sequence's blocks into its pages
        kc[bt[b].long()] = c["k"][b].view(nb, BS, H, D).to(kc.dtype)
        vc[bt[b].long()] = c["v"][b].view(nb, BS, H, D).to(kc.dtype)
    q = c["q"].reshape(B * T, H, D)
    ids = c["block_idx"][:, 0].reshape(B * T, K).to(torch.int32).to(dev)       # [total_q, K]
    di = ids.unsqueeze(0).expand(H, -1, -1)
    cu = (torch.arange(B + 1, dtype=torch.int32) * T).to(dev)
    seq = torch.full((B,), Sk, dtype=torch.int32, device=dev)
    pre = torch.full((B,), Sk - T, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    fn = lambda: U.dash_sparse_attn(q, kc, vc, di, None, bt, cu, seq, pre, T, H, c["scale"], out,
                                    local_blocks=LW // BS, sparse_block_size=BS)
    ms = _time_launches(fn, args.steps, args.warmup, dev)
    wp, rp = W.attended_pairs(c["block_idx"], Sk, BS, LW)
    flops = (wp + rp) * H * 4 * D
    tfs = flops / (ms * 1e-3) / 1e12
    return {"metric": "paged chunked-prefill tokens/s + MFMA TFLOP/s (config 4 over KV pages)",
            "value": B * T / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded), pages in seeded random order",
            "config": {"workload": "config 4 (B=4, 2048 of 65536 keys, 10 heads, block 64, top-8 + 512 window) "
                                   f"through dash_sparse_attn over a [16384, 64, 10, 128] paged {args.kv} cache",
                       "flops_per_step": flops, "kv_cache": args.kv},
            "roofline": {"bound": "mfma", "achieved": tfs, "peak": 2500.0, "unit": "TFLOP/s",
                         "frac": tfs / 2500.0, "traffic": None,
                         "kernel": "srswa::fwd_kernel<bf16,128,paged>"}}


def bench_blockmax(args):
    """Block-max indexer scoring (the reference's K4, HF/sparse_gather_triton.py:445-524)
    on config 4's prefill chunk: one index head, B=4 sequences x 2048 query rows at the
    tail of 65536 keys; a row scores every key before its 512-token window."""
    import torch
    from srswa import ops
    dev = torch.device("cuda:0")
    B, C, Sk, D, BS, LW = 4, 2048, 65536, 128, 64, 512
    g = torch.Generator().manual_seed(20261204)
    q = (torch.randn(B, C, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    k = torch.randn(B, Sk, D, generator=g).to(torch.bfloat16).to(dev)
    pos = (torch.arange(C) + (Sk - C)).expand(B, C).contiguous()
    seg = torch.zeros(B, C, dtype=torch.long)
    nblk = Sk // BS
    posd, segd = pos.to(dev), seg.to(dev)
    fn = lambda: ops.block_max_score(q, k, posd, segd, block_size=BS, num_key_blocks=nblk, local_window=LW)
    ms = _time_launches(fn, args.steps, args.warmup, dev)
    pairs = B * int((pos[0] - LW + 1).clamp(min=0).sum())       # keys j <= pos - LW of every row
    flops = pairs * 2 * D
    tfs = flops / (ms * 1e-3) / 1e12
    return {"metric": "block-max indexer scoring rows/s + MFMA TFLOP/s (config 4 chunk)",
            "value": B * C / (ms * 1e-3), "unit": "query rows/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) keys, N(0,1/D) queries)",
            "config": {"workload": "block-max scores of B=4 x 2048 rows at positions 63488..65535 over "
                                   "65536 keys, one index head, D=128, block 64, window 512",
                       "flops_per_step": flops, "scored_pairs": pairs},
            "roofline": {"bound": "mfma", "achieved": tfs, "peak": 2500.0, "unit": "TFLOP/s",
                         "frac": tfs / 2500.0, "traffic": None, "kernel": "srswa::block_max_kernel<bf16,128>"}}


def bench_fwdbwd(args):
    """Config 5: self-attention forward + backward, B=2, T=16384."""
    import torch
    from srswa import ops, workloads as W
    dev = torch.device("cuda:0")
    B, T, H, D, BS, LW, K = 2, 16384, 10, 128, 64, 512, 8
    c = W.fwdbwd_config(B=B, T=T, H=H, D=D, device=dev)
    dtl, peak, kt = _attn_dtype(args, c, ("q", "k", "v", "do"))
    idx = c["block_idx"].to(dev)
    q, k, v, do = c["q"], c["k"], c["v"], c["do"]

    def step():
        o, lse = ops.gather_fwd(q, k, v, idx, block_size=BS, local_window=LW, scale=c["scale"])
        ops.gather_bwd(q, k, v, o, lse, do, idx, block_size=BS, local_window=LW, scale=c["scale"])

    ms = _time_launches(step, args.steps, args.warmup, dev)
    fwd = lambda: ops.gather_fwd(q, k, v, idx, block_size=BS, local_window=LW, scale=c["scale"])
    ms_f = _time_launches(fwd, args.steps, args.warmup, dev)
    o, lse = fwd()
    bwd = lambda: ops.gather_bwd(q, k, v, o, lse, do, idx, block_size=BS, local_window=LW, scale=c["scale"])
    ms_b = _time_launches(bwd, args.steps, args.warmup, dev)
    wp, rp = W.attended_pairs(c["block_idx"], T, BS, LW)
    pairs = (wp + rp) * H
    flops = pairs * (4 + 10) * D
    tfs = flops / (ms * 1e-3) / 1e12
    del o, lse
    cpu = None if args.no_cpu else cpu_baseline_rows(c, T, T, BS, LW, args.cpu_budget, backward=True)
    return {"metric": "fwd+bwd tokens/s + MFMA TFLOP/s (config 5)", "value": B * T / (ms * 1e-3),
            "cpu_baseline": cpu,
            "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtl,
            "data": "synthetic (seeded N(0,1); tile m selects min(8, m-8) blocks below m-8)",
            "config": {"workload": "config 5: fwd+bwd B=2, T=16384, 10 heads, block 64, top-8 + 512 window",
                       "flops_per_step": flops, "fwd_ms": ms_f, "bwd_ms": ms_b,
                       "fwd_tflops": pairs * 4 * D / (ms_f * 1e-3) / 1e12,
                       "bwd_tflops": pairs * 10 * D / (ms_b * 1e-3) / 1e12},
            "roofline": {"bound": "mfma", "achieved": tfs, "peak": peak, "unit": "TFLOP/s",
                         "frac": tfs / peak, "traffic": None,
                         "kernel": f"fwd_kernel<{kt}> + delta/touch/dq/dkv kernels"}}


def _kv_dtype(args):
    """The --kv cache dtype of the paged legs: None (bf16) or a torch fp8 dtype."""
    import torch
    return None if args.kv == "bf16" else getattr(torch, "float8_" + args.kv)


def bench_paged(args):
    """Config 3 over the serving (paged) cache: the same selections and bytes as
    the default leg, each sequence's blocks in randomly ordered pages.  With
    ``--kv e4m3fn`` (or another fp8 format) the K / V pages hold fp8 values
    (half the bytes), converted to bf16 as they are read."""
    import torch
    from srswa import ops, workloads as W
    dev = torch.device("cuda:0")
    B, H, D, K, BS, LW = 64, 10, 128, 8, 64, 512
    c = W.paged_decode_config(B=B, H=H, D=D, k=K, block_size=BS, local_window=LW, device=dev)
    q = c["q"].view(B, H, D)
    kvd = _kv_dtype(args)
    if kvd is not None:
        c["k_cache"], c["v_cache"] = c["k_cache"].to(kvd), c["v_cache"].to(kvd)
    launch, out = ops.prepare_gather_decode_paged(q, c["k_cache"], c["v_cache"], c["topk"].to(dev), None,
                                                  c["block_table"].to(dev), c["seq_lens"].to(dev),
                                                  decode_query_len=1, local_blocks=c["local_blocks"],
                                                  scale=c["scale"])
    ms = _time_launches(launch, args.steps, args.warmup, dev)
    nbytes = W.decode_bytes(B, H, D, K, BS, LW)
    if kvd is not None:          # K / V bytes halve; q, o and the indices do not
        kv_bytes = 2 * B * H * (LW + K * BS) * D * 2
        nbytes -= kv_bytes // 2
    achieved = nbytes / (ms * 1e-3) / 1e9
    return {"metric": "paged decode sparse-attn tokens/s (config 3 over randomly ordered KV pages)",
            "value": B / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded), pages in seeded random order",
            "config": {"workload": f"config 3, paged [num_pages, 64, 10, 128] {args.kv} cache", "B": B,
                       "num_pages": c["num_pages"], "kv_cache": args.kv},
            "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": achieved / HBM_PEAK_GBS, "traffic": _pmc_traffic(f"paged_cfg3_{args.kv}_traffic"),
                         "algorithmic_bytes_per_launch": nbytes,
                         "kernel": "srswa::decode_kernel<bf16,bf16,128,8,paged>"
                                   + (" (fp8 cache, no merge)" if kvd is not None else " + decode_merge_kernel")}}


def bench_dash(args):
    """One serving DASH decode step on config 3's paged cache: head_cls scores off
    the per-page summary cache (one router head) -> router (entmax-1.5 top-16
    window, 8 blocks, centred log-prior bias) -> paged decode with those blocks
    and biases for all 10 kv heads."""
    import torch
    from srswa import ops, unlimited_dash_ops as U, workloads as W
    dev = torch.device("cuda:0")
    B, H, D, K, BS, LW = 64, 10, 128, 8, 64, 512
    c = W.paged_decode_config(B=B, H=H, D=D, k=K, block_size=BS, local_window=LW, device=dev)
    bt, sl = c["block_table"].to(dev), c["seq_lens"].to(dev)
    cache = U.KBarCache(c["num_pages"], 128, dev)
    hc = torch.randn(128, device=dev)
    U.headcls_scores_prefill(idx_q=c["idx_q"], kv_cache=c["idx_k_cache"], block_table=bt,
                             cu_seqlens_q=torch.arange(B + 1, device=dev), seq_lens=sl, context_lens=sl - 1,
                             head_cls=hc, max_block=bt.shape[1], block_size=BS, local_blocks=LW // BS, cache=cache)
    p = dict(idx_scale=128.0 / math.sqrt(128), floor=1e-4, sigma=1.0, K=K, topm=16)
    q = c["q"].view(B, H, D)
    out = torch.empty_like(q)

    def step():
        cache.refresh_tail(kv_cache=c["idx_k_cache"], block_table=bt, seq_lens=sl, head_cls=hc, block_size=BS,
                           tail_pages=2)
        sc = U.headcls_scores_decode(idx_q=c["idx_q"], cache=cache, block_table=bt, seq_lens=sl,
                                     max_block=bt.shape[1], block_size=BS, local_blocks=LW // BS, decode_query_len=1)
        topi, bias, _ = ops.dash_route(sc[0][:, None, :], None, p, attend_ids=True)   # [B, 1, K], -1 = invalid
        topi = topi[:, 0]                                                              # [B, K]
        U.dash_sparse_attn_decode(q, c["k_cache"], c["v_cache"], topi[None].expand(H, B, K),
                                  bias[:, 0][None].expand(H, B, K), bt, sl, H, c["scale"], out, 1,
                                  local_blocks=LW // BS, sparse_block_size=BS)

    ms = _time_launches(step, args.steps, args.warmup, dev)
    return {"metric": "DASH serving decode step tokens/s (summary-cache scores -> router -> paged decode)",
            "value": B / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded)",
            "config": {"workload": "config 3 paged cache, one router head (d 128), top-16 window, 8 blocks + "
                                   "512-token window, 10 kv heads", "B": B, "max_blocks": int(bt.shape[1])}}


def bench_page(args):
    """Page isolation + Page2D RoPE.  Headline: the rotary applied to the main
    branch's q and k of a 16k-token prefill ([16384, 10*128] bf16 each, one
    launch), HBM-bound.  Beside it: the decode allow mask over config 3's paged
    cache (64 requests, per-slot image pages of every live page read once) and
    the whole one-token decode metadata step (page state + allow mask + local
    union + cos/sin table + rotary of q, k, idx_q, idx_k)."""
    import torch
    from srswa import page_ops, unlimited_dash_ops as U, workloads as W
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)
    # --- rotary at prefill size
    T, H, hd = 16384, 10, 128
    x = torch.randn(T, H * hd, device=dev, generator=g).to(torch.bfloat16)
    y = torch.randn(T, H * hd, device=dev, generator=g).to(torch.bfloat16)
    rope = U.PageRope2D(hd, 10000.0, 256.0, 8)
    tok = torch.randint(0, 4000, (T,), device=dev, generator=g)
    page = torch.randint(0, 40, (T,), device=dev, generator=g)
    cos, sin = rope.cos_sin(tok, page, torch.bfloat16)
    ms_rope = _time_launches(lambda: page_ops.page2d_rope(x, cos, sin, hd, y=y), args.steps, args.warmup, dev)
    rope_bytes = 2 * (2 * T * H * hd * 2) + 2 * T * hd * 2
    rope_gbs = rope_bytes / (ms_rope * 1e-3) / 1e9
    ms_cs = _time_launches(lambda: rope.cos_sin(tok, page, torch.bfloat16), args.steps, args.warmup, dev)
    # --- decode allow mask over config 3's paged cache
    B, BS = 64, 64
    c = W.paged_decode_config(B=B, H=H, D=hd, k=8, block_size=BS, local_window=512, device=dev)
    bt, sl = c["block_table"].to(dev), c["seq_lens"].to(dev)
    npg, maxb = c["num_pages"], bt.shape[1]
    s_page = torch.full((npg * BS,), -1, dtype=torch.int32, device=dev)
    pos = torch.arange(maxb * BS, device=dev)
    for r in range(B):                            # image pages of ~1135 tokens, text between them
        L = int(sl[r])
        p = pos[:L]
        img = torch.where(p % 1200 < 1135, p // 1200, torch.full_like(p, -1)).to(torch.int32)
        s_page[bt[r, p // BS].long() * BS + p % BS] = img
    q_page = ((sl // 1200) // 2).to(torch.int32)
    q_page[::5] = -1
    out = torch.empty(B, maxb, dtype=torch.int8, device=dev)
    allow = lambda: page_ops.page_decode_allow(bt, s_page, q_page, sl, max_block=maxb, num_blocks=npg,
                                               block_size=BS, out=out)
    ms_allow = _time_launches(allow, args.steps, args.warmup, dev)
    live = int(((sl + BS - 1) // BS).sum())
    allow_bytes = live * BS * 4 + live * 4 + B * maxb
    allow_gbs = allow_bytes / (ms_allow * 1e-3) / 1e9
    # --- one decode metadata step (page state, mask, union, cos/sin, rotary of both branches)
    ps = types.SimpleNamespace(image_token_id=128815, page_token_id=128816, per_page_image_tokens=273,
                               _slot_img_page=s_page, _slot_marker_cum=torch.zeros_like(s_page),
                               _slot_img_run=torch.zeros_like(s_page), _slot_prompt_pages=torch.zeros_like(s_page),
                               _ensure=lambda n, d: None)
    rows = torch.arange(B, device=dev)
    cs = types.SimpleNamespace(st_marker=torch.zeros(B, dtype=torch.int32, device=dev),
                               st_pp=torch.zeros(B, dtype=torch.int32, device=dev),
                               cnt=torch.zeros(B, 64, dtype=torch.int32, device=dev), max_pages=64,
                               _ensure=lambda d: None, _rows=lambda layout: rows)
    ids = torch.randint(10, 1000, (B,), device=dev, generator=g)
    slot = bt[torch.arange(B, device=dev), ((sl - 1) // BS).long()].long() * BS + (sl - 1) % BS
    qd = torch.randn(B, H * hd, device=dev, generator=g).to(torch.bfloat16)
    kd = torch.randn(B, H * hd, device=dev, generator=g).to(torch.bfloat16)
    iq = torch.randn(B, hd, device=dev, generator=g).to(torch.bfloat16)
    ik = torch.randn(B, hd, device=dev, generator=g).to(torch.bfloat16)
    cbuf = torch.empty(B, hd, dtype=torch.bfloat16, device=dev)
    sbuf = torch.empty(B, hd, dtype=torch.bfloat16, device=dev)
    union = torch.empty(B, maxb, dtype=torch.int8, device=dev)

    def meta_step():
        qp, (tk, pg) = U.decode_meta_fused(input_ids=ids, block_table=bt, seq_lens=sl, slot_mapping=slot,
                                           page_state=ps, coord_state=cs, num_slots=npg * BS, block_size=BS)
        al = U.decode_allow_fused(block_table=bt, page_state=ps, q_page=qp, seq_lens=sl, max_block=maxb,
                                  num_blocks=npg, block_size=BS, out=out)
        U.local_union_fused(allow=al, seq_lens=sl, out=union, max_block=maxb, block_size=BS, local_blocks=8)
        cc, ss = U.cos_sin_2d_fused(rope=rope, tok_pos=tk, page_pos=pg, dtype=torch.bfloat16, out_cos=cbuf,
                                    out_sin=sbuf)
        U.apply_page2d_rope_pair(qd, kd, cc, ss, hd)
        U.apply_page2d_rope_pair(iq, ik, cc, ss, hd)

    ms_meta = _time_launches(meta_step, args.steps, args.warmup, dev)
    return {"metric": "Page2D rotary of a 16k-token prefill's q and k (tokens/s)", "value": T / (ms_rope * 1e-3),
            "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_rope,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded)",
            "config": {"workload": "apply_page2d_rope_pair, q and k [16384, 10*128] bf16, cos/sin [16384, 128]",
                       "T": T, "heads": H, "head_dim": hd},
            "roofline": {"bound": "hbm", "achieved": rope_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": rope_gbs / HBM_PEAK_GBS, "traffic": _pmc_traffic("rope_page2d_16k_traffic"),
                         "algorithmic_bytes_per_launch": rope_bytes,
                         "kernel": "srswa::rope_kernel<bf16>"},
            "cos_sin_table_us": ms_cs * 1e3,
            "decode_allow": {"workload": "config 3 paged cache, 64 requests, per-slot image pages of every live page",
                             "us": ms_allow * 1e3, "achieved_GBs": allow_gbs, "frac": allow_gbs / HBM_PEAK_GBS,
                             "algorithmic_bytes": allow_bytes,
                             "kernels": "page_allow_scan_kernel<64> + page_allow_open_kernel"},
            "decode_meta_step_us": ms_meta * 1e3}


def bench_kl(args):
    """Indexer distillation KL (training, DASH / "sparse" stage) on config 5's
    shape: B=2, T=16384 rows of one index head against the mean of 10 main
    heads over each row's selected remote keys (config 5's per-tile top-8
    blocks), forward (KL + dsel) and backward (d idx_q, d idx_k)."""
    import torch
    from srswa import kl as KL, workloads as W
    dev = torch.device("cuda:0")
    B, T, H, D, BS, LW, K = 2, 16384, 10, 128, 64, 512, 8
    g = torch.Generator(device=dev).manual_seed(11)
    sel = W.tile_block_indices(B, T, T, BS, LW, K, cfg=5, mode="selfattn").to(dev)        # [B, 1, T, K]
    q_idx = (torch.randn(B, 1, T, D, device=dev, generator=g) * D ** -0.5).to(torch.bfloat16).requires_grad_()
    idx_k = torch.randn(B, T, D, device=dev, generator=g).to(torch.bfloat16).requires_grad_()
    q_main = torch.randn(B, H, T, D, device=dev, generator=g).to(torch.bfloat16)
    k_main = torch.randn(B, H, T, D, device=dev, generator=g).to(torch.bfloat16)
    pos = torch.arange(T, device=dev, dtype=torch.int32).expand(B, T).contiguous()
    scaling = D ** -0.5

    def fwd():
        return KL.kl_forward(q_idx.detach(), idx_k.detach(), q_main, k_main, sel, pos, block_size=BS,
                             local_window=LW, scaling=scaling)

    def step():
        kl, valid = KL.gather_kl(q_idx, idx_k, q_main, k_main, sel, pos, block_size=BS, local_window=LW,
                                 scaling=scaling)
        (kl * valid).sum().backward()

    ms = _time_launches(step, args.steps, args.warmup, dev)
    ms_f = _time_launches(fwd, args.steps, args.warmup, dev)
    _, rp = W.attended_pairs(sel.cpu(), T, BS, LW)              # kept (row, remote key) pairs of all B
    fwd_flops = rp * (H + 1) * 2 * D                            # one pass of the 10 teacher heads + student
    bwd_flops = rp * 2 * 2 * D                                  # d idx_q and d idx_k
    tf_f = fwd_flops / (ms_f * 1e-3) / 1e12
    return {"metric": "indexer distillation KL fwd+bwd tokens/s (config 5 shape)", "value": B * T / (ms * 1e-3),
            "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded), config 5's per-tile top-8 selections",
            "config": {"workload": "gather-KL, B=2, T=16384, 1 index head vs 10 main heads, D=128, top-8 64-key "
                                   "blocks, 512-token window excluded", "fwd_ms": ms_f, "kept_pairs": rp,
                       "fwd_flops": fwd_flops, "bwd_flops": bwd_flops},
            "roofline": {"bound": "mfma", "achieved": tf_f, "peak": 2500.0, "unit": "TFLOP/s", "frac": tf_f / 2500.0,
                         "traffic": None, "kernel": "srswa::kl_fwd_kernel<bf16,128> (one pass of algorithmic flops; "
                                                     "the kernel runs two)"}}


def bench_route(args):
    """Serving DASH router (srswa.unlimited_dash_ops.route_triton) on config 3's
    paged cache: one decode step's routing for 64 requests (summary-cache
    scores over every page, 1.5-entmax, top-8 budget, 16 packed slots), and a
    2048-row prefill chunk against the same cache.  HBM-light, launch-bound:
    the figure is the routed rows per second."""
    import torch
    from srswa import ops, unlimited_dash_ops as U, workloads as W
    dev = torch.device("cuda:0")
    B, BS, LW, K, M = 64, 64, 512, 8, 16
    c = W.paged_decode_config(B=B, device=dev)
    bt, sl = c["block_table"].to(dev), c["seq_lens"].to(dev)
    Wd = int(bt.shape[1])
    kbar = torch.zeros(c["num_pages"], 128, dtype=torch.float32, device=dev)
    hc = torch.randn(128, device=dev)
    ops.kbar_pages(c["idx_k_cache"], hc, bt, sl, kbar)
    iq = c["idx_q"].to(dev)
    out_idx = torch.empty(B, M, dtype=torch.int32, device=dev)
    out_bias = torch.empty(B, M, dtype=torch.float32, device=dev)
    score_buf = torch.empty(B, Wd, dtype=torch.float32, device=dev)
    p = dict(idx_scale=128.0 / math.sqrt(128), prior_floor=1e-4, sigma=1.0)

    def dec():
        U.route_decode_triton(idx_q=iq, k_bar=kbar, block_table=bt, seq_lens=sl, image_allow=None, out_idx=out_idx,
                              out_bias=out_bias, max_block=Wd, block_size=BS, local_blocks=LW // BS,
                              decode_query_len=1, topm=M, score_buf=score_buf, budget=K, out_slots=M, **p)

    ms_d = _time_launches(dec, args.steps, args.warmup, dev)
    R, QL = 1, 2048                                      # one request's 2048-row chunk at the end of the longest
    r = int(torch.argmax(sl))
    L = int(sl[r])
    btp, slp = bt[r:r + 1], sl[r:r + 1]
    cu = torch.tensor([0, QL], dtype=torch.int32, device=dev)
    ctx = slp - QL
    row2req = torch.zeros(QL, dtype=torch.int32, device=dev)
    iqp = torch.randn(QL, 128, device=dev)
    pi = torch.empty(QL, M, dtype=torch.int32, device=dev)
    pb = torch.empty(QL, M, dtype=torch.float32, device=dev)
    sbp = torch.empty(QL, Wd, dtype=torch.float32, device=dev)

    def pre():
        U.route_prefill_triton(idx_q=iqp, k_bar=kbar, block_table=btp, seq_lens=slp, cu_seqlens_q=cu,
                               context_lens=ctx, row2req=row2req, image_allow=None, out_idx=pi, out_bias=pb,
                               max_block=Wd, block_size=BS, local_blocks=LW // BS, topm=M, budget=K,
                               q_chunk=QL, score_buf=sbp, **p)

    ms_p = _time_launches(pre, args.steps, args.warmup, dev)
    return {"metric": "serving DASH router rows/s (decode step, config 3 cache)", "value": B / (ms_d * 1e-3),
            "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_d,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
            "data": "synthetic (seeded)",
            "config": {"workload": "route_decode_triton: 64 requests x up to 2048 pages, top-8 budget, 16 slots; "
                                   "route_prefill_triton: 2048 rows of one request", "max_blocks": Wd,
                       "prefill_rows": QL, "prefill_seq": L, "prefill_ms": ms_p,
                       "prefill_rows_per_s": QL / (ms_p * 1e-3)}}


def bench_dash_train(args):
    """Training DASH router (srswa.dash_train) on config 5's shape: B=2 x 16384
    query rows over 256 64-key blocks, bf16 block scores with the causal remote
    pattern (8 local blocks) and an image-block mask, top-12 budget: forward
    (candidates, 1.5-entmax prior, top-K, bias) + backward (bias -> prior ->
    scores).  HBM-bound row passes."""
    import torch
    from srswa import dash_train as DT
    dev = torch.device("cuda:0")
    B, S, nblk, BS, LB, K = 2, 16384, 256, 64, 8, 12
    g = torch.Generator(device=dev).manual_seed(5)
    sc = torch.randn(B, S, nblk, device=dev, generator=g).to(torch.bfloat16)
    lim = (torch.arange(S, device=dev) // BS - LB)[None, :, None]
    sc = torch.where(torch.arange(nblk, device=dev)[None, None, :] <= lim, sc,
                     torch.full((), -1.0e9, dtype=torch.bfloat16, device=dev)).requires_grad_()
    img = torch.rand(B, nblk, device=dev, generator=g) < 0.4
    gb = torch.randn(B, S, K, device=dev, generator=g).to(torch.bfloat16)
    scale = 128.0 / math.sqrt(128)

    def fwd():
        prior, cand = DT.RouteTrainFn.apply(sc, None, img, scale, -1.0e4)
        return DT.SelectTrainFn.apply(prior, cand, K, 1e-4, 1.0)

    def step():
        _, bias, _ = fwd()
        torch.autograd.backward([bias], [gb])

    ms = _time_launches(step, args.steps, args.warmup, dev)
    with torch.no_grad():
        ms_f = _time_launches(fwd, args.steps, args.warmup, dev)
    E = B * S * nblk
    traffic = 17 * E             # algorithmic bytes per step (config.bytes_per_element)
    gbs = traffic / (ms * 1e-3) / 1e9
    return {"metric": "training DASH router fwd+bwd rows/s (config 5 shape)", "value": B * S / (ms * 1e-3),
            "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded)",
            "config": {"workload": "DashAttention._route + _select_and_bias fwd+bwd, B=2, S=16384, 256 blocks, "
                                   "top-12, image-block mask", "fwd_ms": ms_f, "elements": E,
                       "bytes_per_element": "scores 2 + prior 2 + cand 1 (route) + prior 2 + cand 1 (select) + "
                                            "d prior 2 (select bwd) + d prior 2 + prior 2 + cand 1 + d scores 2 "
                                            "(route bwd) = 17"},
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": 8000.0, "unit": "GB/s", "frac": gbs / 8000.0,
                         "traffic": None, "kernel": "the four router kernels together (step time)"}}


def bench_select_kl(args):
    """The indexer's training step (srswa.indexer.select_and_kl_loss) on
    config 5's shape: B=2 x 16384 rows, one index head, chunks of 1024 rows:
    block-max scores -> top-8 -> gather-KL vs 10 main heads, + backward into
    the index q / k."""
    import torch
    from srswa import indexer as IX
    dev = torch.device("cuda:0")
    B, T, H, D, BS, LB, TK = 2, 16384, 10, 128, 64, 8, 16
    g = torch.Generator(device=dev).manual_seed(13)
    iq = (torch.randn(B, 1, T, D, device=dev, generator=g) * D ** -0.5).to(torch.bfloat16).requires_grad_()
    ik = torch.randn(B, 1, T, D, device=dev, generator=g).to(torch.bfloat16).requires_grad_()
    qm = torch.randn(B, H, T, D, device=dev, generator=g).to(torch.bfloat16)
    km = torch.randn(B, H, T, D, device=dev, generator=g).to(torch.bfloat16)
    pos = torch.arange(T, device=dev).expand(B, T).contiguous()
    hidden = torch.empty(B, T, 8, dtype=torch.bfloat16, device=dev)

    class _Indexer:
        num_heads, head_dim, block_size, local_blocks, local_window = 1, D, BS, LB, LB * BS
        topk_blocks, kl_chunk_size, image_bucket_constraint, layer_idx, kl_log_interval = TK, 1024, False, 0, 1

        def _project_index_qk(self, h, p, kv):
            return iq * 1.0, ik * 1.0

        def _remote_topk(self, nblk):
            return min(max(self.topk_blocks - self.local_blocks, 0), nblk)

        def _build_kl_candidate_mask(self, pos_chunk, nblk, img, batch, cq, image_token_page_ids=None,
                                     query_token_page_ids=None):
            return torch.ones(batch, 1, cq, nblk, dtype=torch.bool, device=pos_chunk.device)

    idx = _Indexer()

    def step():
        _, loss = IX.select_and_kl_loss(idx, hidden, qm, km, None, pos, D ** -0.5)
        loss.backward()

    ms = _time_launches(step, args.steps, args.warmup, dev)
    return {"metric": "indexer training step (select_and_kl_loss fwd+bwd) tokens/s (config 5 shape)",
            "value": B * T / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded)",
            "config": {"workload": "block-max scores + top-8 + gather-KL (1 index head vs 10 main heads) + "
                                   "backward, B=2, T=16384, D=128, chunks of 1024 rows"}}


def bench_train_scores(args):
    """The DASH training router's stage-0 scorers on config 5's shape (B=2,
    S=16384, index dim 128, fp32 index q / k): head_cls (64-key blocks, 8
    local blocks, the shipped stage) and block-max (512-token window), forward
    and forward + backward.  head_cls is HBM-bound (the [B, S, nblk] fp32
    scores dominate); block-max is an fp32 MFMA contraction over every remote
    (query, key) pair."""
    import torch
    from srswa import train_scores as TS
    dev = torch.device("cuda:0")
    B, S, D, BS, LB = 2, 16384, 128, 64, 8
    nblk = S // BS
    g = torch.Generator(device=dev).manual_seed(17)
    q = torch.randn(B, S, D, device=dev, generator=g).requires_grad_()
    k = torch.randn(B, S, D, device=dev, generator=g).requires_grad_()
    hc = (torch.randn(D, device=dev, generator=g) * 0.2).requires_grad_()
    pos = torch.arange(S, device=dev)[None].expand(B, S)
    gz = torch.randn(B, S, nblk, device=dev, generator=g)

    def hc_fwd():
        return TS.head_cls_scores(q, k, hc, pos, nblk, BS, LB)

    def hc_step():
        torch.autograd.backward([hc_fwd()], [gz])

    def bm_fwd():
        return TS.block_max_scores(q, k, pos, nblk, BS, LB * BS)

    def bm_step():
        torch.autograd.backward([bm_fwd()], [gz])

    # the head_cls kernels alone: the C ABI's forward and backward entry points
    # on prebuilt arguments (no autograd, allocation or gradient accumulation,
    # whose host time bounds the step at this size)
    import ctypes
    from srswa import _lib
    lib, sp = _lib.lib(), _lib.stream_ptr(dev)
    p32 = pos.to(torch.int32)
    kbar = torch.empty(B, nblk, D, device=dev)
    zk = torch.empty(B, S, nblk, device=dev)
    dqk, dkk, dhk = torch.empty_like(q), torch.empty_like(k), torch.empty(D, device=dev)
    common = dict(q=q.data_ptr(), q_sb=q.stride(0), q_st=q.stride(1), k=k.data_ptr(), k_sb=k.stride(0),
                  k_st=k.stride(1), head_cls=hc.data_ptr(), pos=p32.data_ptr(), pos_sb=p32.stride(0),
                  pos_st=p32.stride(1), kbar=kbar.data_ptr(), kb_sb=kbar.stride(0), z=zk.data_ptr(),
                  z_sb=zk.stride(0), z_st=zk.stride(1), B=B, S=S, D=D, nblk=nblk, block_size=BS, local_blocks=LB)
    fa = _lib.HcScoreArgs(**common)
    ba = _lib.HcScoreBwdArgs(**common, gz=gz.data_ptr(), gz_sb=gz.stride(0), gz_st=gz.stride(1),
                             dq=dqk.data_ptr(), dq_sb=dqk.stride(0), dq_st=dqk.stride(1), dk=dkk.data_ptr(),
                             dk_sb=dkk.stride(0), dk_st=dkk.stride(1), dhc=dhk.data_ptr())
    need = ctypes.c_size_t()
    _lib.check(lib.srswa_hc_score_bwd_workspace(ctypes.byref(ba), ctypes.byref(need)), "hc bwd workspace")
    scr = torch.empty(need.value, dtype=torch.uint8, device=dev)

    def hc_fwd_kernels():
        _lib.check(lib.srswa_hc_score_fwd(ctypes.byref(fa), sp), "srswa_hc_score_fwd")

    def hc_bwd_kernels():
        _lib.check(lib.srswa_hc_score_bwd(ctypes.byref(ba), ctypes.c_void_p(scr.data_ptr()), need.value, sp),
                   "srswa_hc_score_bwd")

    with torch.no_grad():
        ms_hc_fk = _time_launches(hc_fwd_kernels, args.steps, args.warmup, dev)
        ms_hc_bk = _time_launches(hc_bwd_kernels, args.steps, args.warmup, dev)
        ms_hc_f = _time_launches(hc_fwd, args.steps, args.warmup, dev)
        ms_bm_f = _time_launches(bm_fwd, max(2, args.steps // 4), 2, dev)
    ms_hc = _time_launches(hc_step, args.steps, args.warmup, dev)
    ms_bm = _time_launches(bm_step, max(2, args.steps // 4), 2, dev)
    # algorithmic work: head_cls forward moves q, k (read) and the scores (written);
    # block-max forward does 2 D flops per remote (query, key) pair
    hc_bytes = 2 * B * S * D * 4 + B * S * nblk * 4 + B * nblk * D * 4
    remote_pairs = B * sum(max(0, i - LB * BS + 1) for i in range(S))
    bm_flops = 2 * D * remote_pairs
    hc_gbs = hc_bytes / (ms_hc_fk * 1e-3) / 1e9
    bm_tfs = bm_flops / (ms_bm_f * 1e-3) / 1e12
    return {"metric": "DASH training stage-0 scorer fwd+bwd rows/s (head_cls, config 5 shape)",
            "value": B * S / (ms_hc * 1e-3), "unit": "rows/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms_hc, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded)",
            "config": {"workload": "DashAttention._block_scores_headcls / _block_scores from fp32 index q/k, "
                                   "B=2, S=16384, D=128, 64-key blocks", "head_cls_fwd_ms": ms_hc_f,
                       "head_cls_fwd_bwd_ms": ms_hc, "head_cls_fwd_kernels_ms": ms_hc_fk,
                       "head_cls_bwd_kernels_ms": ms_hc_bk, "block_max_fwd_ms": ms_bm_f, "block_max_fwd_bwd_ms": ms_bm,
                       "head_cls_fwd_bytes": hc_bytes, "block_max_fwd_flops": bm_flops},
            "roofline": {"bound": "hbm", "achieved": hc_gbs, "peak": 8000.0, "unit": "GB/s",
                         "frac": hc_gbs / 8000.0, "traffic": _pmc_traffic("train_scores_cfg5_traffic"),
                         "kernel": "head_cls forward kernels (summary + score), launched on prebuilt arguments"},
            "roofline_block_max": {"bound": "mfma", "achieved": bm_tfs, "peak": 157.3, "unit": "TFLOP/s",
                                   "frac": bm_tfs / 157.3, "kernel": "bm_fwd_kernel (fp32 MFMA)"}}


def bench_copycal(args):
    """Calibration for the HBM traffic counters: a plain device copy of a known
    size (4 GiB read + 4 GiB written per launch, far beyond the 256 MB
    Infinity Cache), so rocprofv3's FETCH_SIZE / WRITE_SIZE readings per
    dispatch can be scaled to bytes."""
    import torch
    dev = torch.device("cuda:0")
    n = 4 * 1024 * 1024 * 1024
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    ms = _time_launches(lambda: dst.copy_(src), args.steps, args.warmup, dev)
    return {"metric": "copy calibration", "value": 2 * n / (ms * 1e-3) / 1e9, "unit": "GB/s",
            "bytes_read_per_launch": n, "bytes_written_per_launch": n, "ms_per_step": ms,
            "steps": args.steps, "warmup": args.warmup, "n_gpus": 1, "higher_is_better": True}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="decode",
                    choices=["decode", "indexer", "prefill", "fwdbwd", "paged", "paged_prefill", "dash", "page", "kl",
                             "blockmax", "route", "dash_train", "select_kl", "train_scores", "copycal"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-check", action="store_true", help="skip the oracle spot check")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--dtype", default="bf16", choices=["bf16", "fp32"],
                    help="operand dtype of the prefill / fwdbwd legs (fp32: the fp32 MFMA form, 157.3 TFLOP/s peak)")
    ap.add_argument("--kv", default="bf16", choices=["bf16", "e4m3fn", "e4m3fnuz", "e5m2", "e5m2fnuz"],
                    help="K / V cache dtype of the paged legs (fp8 formats: half the bytes)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build runs on a single MI355X "
              "(no multi-GPU path); use --gpus 1", file=sys.stderr)
        sys.exit(2)
    fn = {"decode": bench_decode, "indexer": bench_indexer, "prefill": bench_prefill,
          "fwdbwd": bench_fwdbwd, "paged": bench_paged, "paged_prefill": bench_paged_prefill, "dash": bench_dash,
          "page": bench_page, "kl": bench_kl,
          "blockmax": bench_blockmax, "route": bench_route, "dash_train": bench_dash_train,
          "select_kl": bench_select_kl, "train_scores": bench_train_scores,
          "copycal": bench_copycal}[args.config]
    res = fn(args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
