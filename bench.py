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


def cpu_baseline_decode(budget_s=12.0, threads=None):
    """Time the oracle's restatement of the reference decode (_decode_attend,
    dense fp32 over all cached keys) on host cores, one config-3 sequence at a
    time, until ``budget_s`` is spent.  Returns the baseline dict."""
    import torch
    sys.path.insert(0, REPO)
    from oracle import srswa_oracle as O
    from srswa import workloads as W

    n_thr = threads or min(os.cpu_count() or 1, 16)
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
    ms = e0.elapsed_time(e1) / args.steps
    _log(f"timed {args.steps} steps: {ms * 1e3:.2f} us/step (HIP events), wall {wall * 1e6 / args.steps:.2f} us/step")
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
                     "kernel": "srswa::decode_kernel<bf16,bf16,128,8> + decode_merge_kernel (one step)"},
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


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="decode", choices=["decode"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-check", action="store_true", help="skip the oracle spot check")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build runs on a single MI355X "
              "(no multi-GPU path); use --gpus 1", file=sys.stderr)
        sys.exit(2)
    res = bench_decode(args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
