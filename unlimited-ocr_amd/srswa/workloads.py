"""Seeded synthetic inputs for the five SR-SWA benchmark configurations.

Seeds: ``torch.Generator().manual_seed(20261201 + cfg)``, per-sequence
sub-seeds ``+ 1000 * b``.  Small tensors (indices, positions, queries) are
always drawn on the CPU so every consumer sees the same bytes; the large
KV caches of the full-size decode / indexer configurations can instead be
drawn on the device (``device=`` argument) where a host copy would not fit.
"""

from __future__ import annotations

import math

import torch

SEED0 = 20261201


def _gen(cfg: int, sub: int = 0) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(SEED0 + cfg + 1000 * sub)
    return g


# ---------------------------------------------------------------- config 3
def decode_lengths(B: int, lo: int = 4096, hi: int = 131072, cfg: int = 3) -> torch.Tensor:
    """KV lengths drawn log-uniformly from [lo, hi] (floor of exp U(ln lo, ln hi))."""
    g = _gen(cfg)
    u = torch.rand(B, generator=g, dtype=torch.float64)
    L = torch.floor(torch.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))).long()
    return L.clamp(lo, hi)


def decode_block_indices(lengths: torch.Tensor, H: int, k: int, block_size: int,
                         local_window: int, cfg: int = 3) -> torch.Tensor:
    """[B, H, k] int32: per (b, h) k sorted unique blocks from
    {0 .. floor((L_b - LW) / BS) - 1} (all strictly before the window)."""
    B = lengths.shape[0]
    out = torch.full((B, H, k), -1, dtype=torch.int32)
    for b in range(B):
        g = _gen(cfg, b + 1)
        n = max(0, (int(lengths[b]) - local_window) // block_size)
        for h in range(H):
            kk = min(k, n)
            if kk > 0:
                sel = torch.randperm(n, generator=g)[:kk].sort().values
                out[b, h, :kk] = sel.to(torch.int32)
    return out


def decode_config(B=64, H=10, D=128, Lmax=131072, lo=4096, k=8, block_size=64,
                  local_window=512, dtype=torch.bfloat16, device=None, cfg=3,
                  lengths=None):
    """Config 3 (decode gather-attention).  Returns a dict with q [B,H,D],
    k_cache/v_cache [B,Lmax,H,D], block_idx [B,H,k] int32, q_pos [B] int32 (= L_b - 1),
    seq_lens [B].  With ``device`` the caches (and q) are drawn there."""
    if lengths is None:
        lengths = decode_lengths(B, lo, Lmax, cfg)
    idx = decode_block_indices(lengths, H, k, block_size, local_window, cfg)
    g = _gen(cfg, 0)
    q = torch.randn(B, H, D, generator=g, dtype=torch.float32).to(dtype)
    if device is None:
        kc = torch.randn(B, Lmax, H, D, generator=g, dtype=torch.float32).to(dtype)
        vc = torch.randn(B, Lmax, H, D, generator=g, dtype=torch.float32).to(dtype)
    else:
        gd = torch.Generator(device=device)
        gd.manual_seed(SEED0 + cfg)
        kc = torch.randn(B, Lmax, H, D, generator=gd, dtype=dtype, device=device)
        vc = torch.randn(B, Lmax, H, D, generator=gd, dtype=dtype, device=device)
        q = q.to(device)
    return dict(q=q, k_cache=kc, v_cache=vc, block_idx=idx,
                q_pos=(lengths - 1).to(torch.int32), seq_lens=lengths.to(torch.int32),
                block_size=block_size, local_window=local_window, scale=1.0 / math.sqrt(D))


def paged_decode_config(B=64, H=10, D=128, Lmax=131072, lo=4096, k=8, block_size=64, local_window=512,
                        dtype=torch.bfloat16, device=None, cfg=3, d_index=128):
    """Config 3 over the serving cache layout: each sequence's blocks live in
    pages [num_pages, block_size, H, D] dealt in a seeded random order (one page
    per block, as the serving backend asserts), block_table [B, max_blocks],
    seq_lens [B], per-kv-head selections topk [H, B, k] (config 3's indices),
    plus an index-key page cache [num_pages, block_size, d_index] and one
    router query per sequence for the stage-0 scorer."""
    lengths = decode_lengths(B, lo, Lmax, cfg)
    idx = decode_block_indices(lengths, H, k, block_size, local_window, cfg)
    nb = (lengths + block_size - 1) // block_size
    max_blocks = int(nb.max())
    npages = int(nb.sum())
    g = _gen(cfg, 0)
    perm = torch.randperm(npages, generator=g).to(torch.int32)
    bt = torch.zeros(B, max_blocks, dtype=torch.int32)
    o = 0
    for b in range(B):
        n = int(nb[b])
        bt[b, :n] = perm[o:o + n]
        o += n
    q = torch.randn(B, H, D, generator=g, dtype=torch.float32).to(dtype)
    iq = torch.randn(B, d_index, generator=g, dtype=torch.float32)
    gd = torch.Generator(device=device) if device is not None else g
    if device is not None:
        gd.manual_seed(SEED0 + cfg)
    kw = dict(generator=gd, dtype=dtype, device=device) if device is not None else dict(generator=gd)
    kc = torch.randn(npages, block_size, H, D, **kw)
    vc = torch.randn(npages, block_size, H, D, **kw)
    ikc = torch.randn(npages, block_size, d_index, **kw)
    if device is None:
        kc, vc, ikc = kc.to(dtype), vc.to(dtype), ikc.to(dtype)
    else:
        q, iq = q.to(device), iq.to(device)
    return dict(q=q, k_cache=kc, v_cache=vc, idx_k_cache=ikc, idx_q=iq, topk=idx.permute(1, 0, 2).contiguous(),
                block_table=bt, seq_lens=lengths.to(torch.int32), block_size=block_size,
                local_blocks=local_window // block_size, scale=1.0 / math.sqrt(D), num_pages=npages)


def decode_bytes(B, H, D, k, block_size, local_window, elem=2):
    """Algorithmic HBM bytes of one decode step: K and V of (k*BS + LW) keys per
    (b, h) plus q, o and the index tensor."""
    kv = B * H * (k * block_size + local_window) * D * elem * 2
    return kv + B * H * D * elem * 2 + B * H * k * 4


# ---------------------------------------------------------------- config 1
def cpu_decode_config(B=1, H=10, D=128, L=8192, block_size=64, k=8, local_window=512,
                      dtype=torch.float32, cfg=1):
    """Config 1: q, k, v iid N(0,1)/sqrt(D), one decode row at pos L-1."""
    g = _gen(cfg)
    s = 1.0 / math.sqrt(D)
    q = (torch.randn(B, H, 1, D, generator=g) * s).to(dtype)
    kk = (torch.randn(B, H, L, D, generator=g) * s).to(dtype)
    vv = (torch.randn(B, H, L, D, generator=g) * s).to(dtype)
    return dict(q=q, k=kk, v=vv, q_pos=torch.full((B, 1), L - 1, dtype=torch.int64),
                block_size=block_size, k_top=k, local_window=local_window,
                scale=1.0 / math.sqrt(D))


# ---------------------------------------------------------------- config 2
def indexer_config(B=32, H=10, D=128, L=32768, block_size=64, local_window=512,
                   frac=0.05, shift=3.0, dtype=torch.bfloat16, device=None, cfg=2):
    """Config 2: keys N(0,1); per (b, h) a unit direction u, q = sqrt(D) u + N(0,I);
    ``round(frac * nblk)`` eligible blocks get K += shift * u.  pos = L - 1.
    Returns q [B,H,D] fp32, k [B,L,H,D] in ``dtype``, q_pos [B]."""
    g = _gen(cfg)
    nblk = L // block_size
    elig = nblk - local_window // block_size            # blocks 0..elig-1 are remote
    n_hot = int(round(frac * nblk))
    u = torch.randn(B, H, D, generator=g)
    u = u / u.norm(dim=-1, keepdim=True)
    q = math.sqrt(D) * u + torch.randn(B, H, D, generator=g)
    hot = torch.stack([torch.stack([torch.randperm(elig, generator=g)[:n_hot] for _ in range(H)])
                       for _ in range(B)])                # [B,H,n_hot]
    if device is None:
        k = torch.randn(B, L, H, D, generator=g)
    else:
        gd = torch.Generator(device=device)
        gd.manual_seed(SEED0 + cfg)
        k = torch.randn(B, L, H, D, generator=gd, device=device)
    kv = k.view(B, nblk, block_size, H, D)
    for b in range(B):
        for h in range(H):
            ids = hot[b, h].to(k.device)
            kv[b, ids, :, h, :] += shift * u[b, h].to(k.device)
    k = k.to(dtype)
    return dict(q=q if device is None else q.to(device), k=k,
                q_pos=torch.full((B,), L - 1, dtype=torch.int32),
                block_size=block_size, local_window=local_window, hot=hot)


def indexer_bytes(B, H, D, L, block_size, local_window, elem=2):
    nblk = L // block_size
    elig = nblk - local_window // block_size
    return B * elig * block_size * H * D * elem + B * H * D * 4 + B * H * 8 * 4


# ---------------------------------------------------------------- configs 4 / 5
def tile_block_indices(B, T, Sk, block_size, local_window, k, tile=64, cfg=4, HI=1,
                       mode="prefix"):
    """[B, HI, T, k] int32 per-token indices broadcast from one selection per
    64-query tile.  ``mode="prefix"`` (config 4): k sorted unique blocks drawn
    from {b : BS*(b+1) <= t0_key - LW + 1} (fully before the tile's first
    window).  ``mode="selfattn"`` (config 5): tile m takes min(k, m - 8) blocks
    from {b <= m - 9}."""
    g = _gen(cfg)
    ntile = -(-T // tile)
    out = torch.full((B, HI, T, k), -1, dtype=torch.int32)
    off = Sk - T
    for b in range(B):
        for hi in range(HI):
            for m in range(ntile):
                t0 = m * tile
                if mode == "prefix":
                    n = max(0, (off + t0 - local_window + 1) // block_size)
                    kk = min(k, n)
                else:
                    n = max(0, m - 8)             # blocks 0 .. m-9
                    kk = min(k, n)
                if kk <= 0:
                    continue
                sel = torch.randperm(n, generator=g)[:kk].sort().values.to(torch.int32)
                out[b, hi, t0:t0 + tile, :kk] = sel
    return out


def prefill_config(B=4, T=2048, Sk=65536, H=10, D=128, block_size=64, local_window=512, k=8,
                   dtype=torch.bfloat16, device=None, cfg=4):
    """Config 4: chunked prefill, T query rows at the tail of an Sk-key cache."""
    idx = tile_block_indices(B, T, Sk, block_size, local_window, k, cfg=cfg, mode="prefix")
    gd = torch.Generator(device=device) if device is not None else torch.Generator()
    gd.manual_seed(SEED0 + cfg)
    kw = dict(generator=gd, dtype=dtype, device=device) if device is not None else dict(generator=gd)
    q = torch.randn(B, T, H, D, **kw)
    kc = torch.randn(B, Sk, H, D, **kw)
    vc = torch.randn(B, Sk, H, D, **kw)
    if device is None:
        q, kc, vc = q.to(dtype), kc.to(dtype), vc.to(dtype)
    return dict(q=q, k=kc, v=vc, block_idx=idx, block_size=block_size, local_window=local_window,
                scale=1.0 / math.sqrt(D))


def fwdbwd_config(B=2, T=16384, H=10, D=128, block_size=64, local_window=512, k=8,
                  dtype=torch.bfloat16, device=None, cfg=5):
    """Config 5: self-attention forward + backward, selection per 64-query tile."""
    idx = tile_block_indices(B, T, T, block_size, local_window, k, cfg=cfg, mode="selfattn")
    gd = torch.Generator(device=device) if device is not None else torch.Generator()
    gd.manual_seed(SEED0 + cfg)
    kw = dict(generator=gd, dtype=dtype, device=device) if device is not None else dict(generator=gd)
    q, kc, vc, do = (torch.randn(B, T, H, D, **kw) for _ in range(4))
    if device is None:
        q, kc, vc, do = (x.to(dtype) for x in (q, kc, vc, do))
    return dict(q=q, k=kc, v=vc, do=do, block_idx=idx, block_size=block_size,
                local_window=local_window, scale=1.0 / math.sqrt(D))


def attended_pairs(block_idx, Sk, block_size, local_window):
    """(window pairs, remote pairs) summed over rows of one head, for a tile-shared
    selection [B, HI, T, k]: the FLOP basis of configs 4 / 5."""
    B, HI, T, K = block_idx.shape
    off = Sk - T
    qi = torch.arange(T, dtype=torch.int64) + off
    win = torch.clamp(qi, max=local_window - 1) + 1                  # window length per row
    ls = qi - local_window + 1
    rem = torch.zeros(B, HI, T, dtype=torch.int64)
    for s in range(K):
        ids = block_idx[..., s].long()
        lo = ids * block_size
        hi = torch.minimum(lo + block_size, ls[None, None, :].clamp(min=0))
        hi = torch.minimum(hi, qi[None, None, :] + 1)
        rem += torch.where(ids >= 0, (hi - lo).clamp(min=0), torch.zeros_like(lo))
    return int(win.sum()) * B, int(rem[:, 0].sum())
