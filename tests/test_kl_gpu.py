"""Gather-KL kernels (srswa_gather_kl_fwd / _bwd) vs the CPU oracle
(oracle/kl_oracle.py, float64 with the reference's bf16 / fp16 rounding of the
logits): validity exact; per-row KL within 2e-3 absolute + 1e-3 relative (the
logits are rounded to 16 bits after an fp32 MFMA sum vs the oracle's exact
one, so a logit on a rounding boundary may round the other way); dsel (the
student's d kl / d logit) within 1e-4; gradients of the loss within the
16-bit tolerance of tests/tolerance.py."""

import pytest
import torch

from oracle import kl_oracle as K
from tolerance import assert_close_lowp

pytestmark = pytest.mark.gpu


def _case(seed, B, HI, G, HKV, T, Sk, D, topk, dtype, packed=False, dup=False):
    g = torch.Generator().manual_seed(seed)
    HQ = HI * G
    sc = D ** -0.5
    q_idx = (torch.randn(B, HI, T, D, generator=g) * sc).to(dtype)
    idx_k = torch.randn(B, Sk, D, generator=g).to(dtype)
    q_main = torch.randn(B, HQ, T, D, generator=g).to(dtype)
    k_main = torch.randn(B, HKV, Sk, D, generator=g).to(dtype)
    pos = (torch.arange(T) + (Sk - T)).expand(B, T).clone().to(torch.int32)
    nblk = -(-Sk // 64)
    sel = torch.stack([torch.stack([torch.stack([torch.randperm(nblk, generator=g)[:topk] for _ in range(T)])
                                    for _ in range(HI)]) for _ in range(B)]).to(torch.int32)
    sel[..., ::7, -1] = -1
    sel[..., :3, :] = -1                                  # rows with nothing selected
    if dup:
        sel[..., 5::9, 1] = sel[..., 5::9, 0]             # a repeated id counts once
    seg = None
    if packed:                                            # two samples per sequence
        seg = torch.where(torch.arange(T) + (Sk - T) >= Sk // 2, Sk // 2, 0).expand(B, T).to(torch.int32)
    return q_idx, idx_k, q_main, k_main, sel, pos, seg, D ** -0.5


CASES = [
    # seed, B, HI, G, HKV, T, Sk, D, topk, dtype, packed, dup
    (1, 2, 1, 10, 10, 200, 1500, 128, 8, torch.bfloat16, False, False),   # the shipped config's shape
    (2, 1, 2, 4, 2, 130, 900, 128, 6, torch.bfloat16, True, True),        # two index heads, GQA, packed
    (3, 2, 1, 3, 1, 97, 700, 64, 5, torch.float16, False, True),
    (4, 1, 1, 1, 1, 64, 64 * 20 - 5, 64, 16, torch.bfloat16, False, False),
]


@pytest.mark.parametrize("case", CASES)
def test_forward_and_dsel(dev, case):
    seed, B, HI, G, HKV, T, Sk, D, topk, dtype, packed, dup = case
    print(f"kl fwd seed={seed} B={B} HI={HI} G={G} T={T} Sk={Sk} D={D} K={topk}", flush=True)
    from srswa import kl as KL
    q_idx, idx_k, q_main, k_main, sel, pos, seg, scaling = _case(seed, B, HI, G, HKV, T, Sk, D, topk, dtype, packed,
                                                                  dup)
    lw = 128
    kl, valid, dsel = KL.kl_forward(q_idx.to(dev), idx_k.to(dev), q_main.to(dev), k_main.to(dev), sel.to(dev),
                                    pos.to(dev), block_size=64, local_window=lw, scaling=scaling,
                                    seg=None if seg is None else seg.to(dev))
    rk, rv = K.gather_kl_dense(q_idx.double(), idx_k.double(), q_main.double(), k_main.double(), sel, pos,
                               block_size=64, local_window=lw, scaling=scaling, seg=seg, round_dtype=dtype)
    assert torch.equal(valid.cpu(), rv)
    err = (kl.cpu().double() - rk).abs() - 1e-3 * rk.abs()
    assert err.max().item() <= 2e-3, err.max().item()
    assert rv.any() and (~rv).any()
    # dsel: softmax(student) - p on kept keys, per selected slot
    keep = K.keep_mask(sel, pos, Sk, 64, lw, seg)
    s = K._round(torch.einsum("bhtd,bsd->bhts", q_idx.double(), idx_k.double()), dtype).masked_fill(~keep, K.NEG)
    sm = torch.softmax(s, -1)
    p = torch.zeros_like(sm)
    for h in range(HI * G):
        sh = K._round(torch.einsum("btd,bsd->bts", q_main[:, h].double(), k_main[:, h // (HI * G // HKV)].double()),
                      dtype) * scaling
        p[:, h // G] += torch.softmax(sh.masked_fill(~keep[:, h // G], K.NEG), -1)
    p /= G
    ref_ds = torch.where(keep, sm - p, torch.zeros_like(p))
    got = dsel.cpu().double()
    nblk = -(-Sk // 64)
    for bb in range(B):
        for ih in range(HI):
            for t in range(T):
                seen = set()
                for slot in range(topk):
                    c = int(sel[bb, ih, t, slot])
                    if c < 0 or c in seen:
                        assert got[bb, ih, t, slot].abs().max() == 0
                        continue
                    seen.add(c)
                    n = min(64, Sk - 64 * c)
                    ref = ref_ds[bb, ih, t, 64 * c:64 * c + n]
                    assert (got[bb, ih, t, slot, :n] - ref).abs().max().item() <= 1e-4, (bb, ih, t, slot)
    del nblk


def test_row_sparse_and_tile_paths_agree(dev):
    """Tiles alternate between rows sharing one selection (the tile kernel
    takes them) and rows selecting unrelated blocks (flagged, block-major);
    T spans three 1024-row ranges.  The block-major path against the oracle,
    and against the tile kernel run on every tile (fp32 rounding apart)."""
    from srswa import kl as KL
    B, HI, G, HKV, T, Sk, D, topk, dtype = 1, 1, 4, 2, 2200, 2600, 128, 8, torch.bfloat16
    print(f"kl row-sparse vs tile B={B} T={T} Sk={Sk} K={topk}", flush=True)
    q_idx, idx_k, q_main, k_main, sel, pos, seg, scaling = _case(11, B, HI, G, HKV, T, Sk, D, topk, dtype)
    g = torch.Generator().manual_seed(12)
    nblk = -(-Sk // 64)
    for tau in range(0, -(-T // 64), 2):                  # even tiles: one selection for all their rows
        sel[:, :, 64 * tau:64 * tau + 64] = torch.randperm(nblk, generator=g)[:topk].to(torch.int32)
    lw = 256
    args = (q_idx.to(dev), idx_k.to(dev), q_main.to(dev), k_main.to(dev), sel.to(dev), pos.to(dev))
    kl, valid, dsel = KL.kl_forward(*args, block_size=64, local_window=lw, scaling=scaling)
    kl_t, valid_t, dsel_t = KL.kl_forward(*args, block_size=64, local_window=lw, scaling=scaling, row_sparse=False)
    assert torch.equal(valid, valid_t)
    assert (kl - kl_t).abs().max().item() <= 1e-5 + 1e-5 * kl_t.abs().max().item()
    assert (dsel - dsel_t).abs().max().item() <= 1e-5
    qr = q_idx.double().requires_grad_()
    kr = idx_k.double().requires_grad_()
    rk, rv = K.gather_kl_dense(qr, kr, q_main.double(), k_main.double(), sel, pos,
                               block_size=64, local_window=lw, scaling=scaling, seg=None, round_dtype=dtype)
    assert torch.equal(valid.cpu(), rv)
    err = (kl.cpu().double() - rk.detach()).abs() - 1e-3 * rk.detach().abs()
    assert err.max().item() <= 2e-3, err.max().item()
    # backward: shared tiles on the tile dQ kernel, the others block-major
    qd = q_idx.to(dev).requires_grad_()
    kd = idx_k.to(dev).requires_grad_()
    klg, vg = KL.gather_kl(qd, kd, q_main.to(dev), k_main.to(dev), sel.to(dev), pos.to(dev), block_size=64,
                           local_window=lw, scaling=scaling)
    K.kl_loss(klg, vg).backward()
    K.kl_loss(rk, rv).backward()
    assert_close_lowp(qd.grad.cpu(), qr.grad, dtype, what="d q_idx (mixed tiles)")
    assert_close_lowp(kd.grad.cpu(), kr.grad, dtype, what="d idx_k (mixed tiles)")


def test_side_stream_is_the_callers_and_optional(dev):
    """The row-sparse forward and the backward take the second stream and its
    two events from the caller (srswa_kl_args / srswa_kl_bwd_args): with them
    and without them (every kernel on the current stream) the results are the
    same bits and match the oracle; handing over only some of the three is
    rejected before anything is launched."""
    import ctypes
    from srswa import _lib, kl as KL
    B, HI, G, HKV, T, Sk, D, topk, dtype = 1, 1, 2, 2, 1100, 1500, 128, 6, torch.bfloat16
    q_idx, idx_k, q_main, k_main, sel, pos, seg, scaling = _case(31, B, HI, G, HKV, T, Sk, D, topk, dtype)
    g = torch.Generator().manual_seed(32)
    nblk = -(-Sk // 64)
    for tau in range(0, -(-T // 64), 2):                  # mixed tiles: both kernel families run
        sel[:, :, 64 * tau:64 * tau + 64] = torch.randperm(nblk, generator=g)[:topk].to(torch.int32)
    lw = 128
    args = (q_idx.to(dev), idx_k.to(dev), q_main.to(dev), k_main.to(dev), sel.to(dev), pos.to(dev))
    two = KL.kl_forward(*args, block_size=64, local_window=lw, scaling=scaling, side_stream=True)
    one = KL.kl_forward(*args, block_size=64, local_window=lw, scaling=scaling, side_stream=False)
    for x, y in zip(two, one):
        assert torch.equal(x, y)
    grad = torch.randn(B, HI, T, generator=g).to(dev)
    dq2, dk2 = KL.kl_backward(grad, args[0], args[1], args[4], two[2], block_size=64, side_stream=True)
    dq1, dk1 = KL.kl_backward(grad, args[0], args[1], args[4], one[2], block_size=64, side_stream=False)
    assert torch.equal(dq2, dq1) and torch.equal(dk2, dk1)
    rk, rv = K.gather_kl_dense(q_idx.double(), idx_k.double(), q_main.double(), k_main.double(), sel, pos,
                               block_size=64, local_window=lw, scaling=scaling, seg=None, round_dtype=dtype)
    assert torch.equal(one[1].cpu(), rv)
    assert ((one[0].cpu().double() - rk).abs() - 1e-3 * rk.abs()).max().item() <= 2e-3
    # a stream without its events is refused (nothing launched)
    s, _, _ = KL.side_channel(args[0].device)
    a = _lib.KlBwdArgs(B=B, HI=HI, T=T, Sk=Sk, D=D, K=topk, block_size=64, dtype=_lib.dtype_code(dtype),
                       q_idx=args[0].data_ptr(), idx_k=args[1].data_ptr(), sel=args[4].data_ptr(),
                       dsel=one[2].data_ptr(), grad=grad.data_ptr(), dq_idx=dq1.data_ptr(), dk_idx=dk1.data_ptr(),
                       side_stream=s.cuda_stream)
    rc = _lib.lib().srswa_gather_kl_bwd(ctypes.byref(a), None, 0, _lib.stream_ptr(args[0].device))
    assert rc == 2, rc                                    # SRSWA_INVALID


@pytest.mark.parametrize("case", CASES[:3])
def test_backward(dev, case):
    seed, B, HI, G, HKV, T, Sk, D, topk, dtype, packed, dup = case
    print(f"kl bwd seed={seed} D={D} dtype={dtype}", flush=True)
    from srswa import kl as KL
    q_idx, idx_k, q_main, k_main, sel, pos, seg, scaling = _case(seed, B, HI, G, HKV, T, Sk, D, topk, dtype, packed,
                                                                  dup)
    lw = 128
    qd = q_idx.to(dev).requires_grad_()
    kd = idx_k.to(dev).requires_grad_()
    kl, valid = KL.gather_kl(qd, kd, q_main.to(dev), k_main.to(dev), sel.to(dev), pos.to(dev), block_size=64,
                             local_window=lw, scaling=scaling, seg=None if seg is None else seg.to(dev))
    loss = K.kl_loss(kl, valid)
    loss.backward()
    qr = q_idx.double().requires_grad_()
    kr = idx_k.double().requires_grad_()
    rk, rv = K.gather_kl_dense(qr, kr, q_main.double(), k_main.double(), sel, pos, block_size=64, local_window=lw,
                               scaling=scaling, seg=seg, round_dtype=dtype)
    K.kl_loss(rk, rv).backward()
    assert_close_lowp(qd.grad.cpu(), qr.grad, dtype, what="d q_idx")
    assert_close_lowp(kd.grad.cpu(), kr.grad, dtype, what="d idx_k")
    # deterministic: a second backward gives the same bits
    qd2 = q_idx.to(dev).requires_grad_()
    kd2 = idx_k.to(dev).requires_grad_()
    kl2, valid2 = KL.gather_kl(qd2, kd2, q_main.to(dev), k_main.to(dev), sel.to(dev), pos.to(dev), block_size=64,
                               local_window=lw, scaling=scaling, seg=None if seg is None else seg.to(dev))
    K.kl_loss(kl2, valid2).backward()
    assert torch.equal(qd.grad, qd2.grad) and torch.equal(kd.grad, kd2.grad)


def test_kl_chunk_fn_dropin(dev):
    """KLChunkFn.apply with the reference's block-level keep mask and
    same-segment mask, against the dense oracle."""
    from srswa import kl as KL
    q_idx, idx_k, q_main, k_main, sel, pos, seg, scaling = _case(5, 1, 2, 3, 3, 90, 800, 128, 5, torch.bfloat16,
                                                                  packed=True)
    nblk = -(-800 // 64)
    keep_block = torch.zeros(1, 2, 90, nblk + 1, dtype=torch.bool)
    keep_block.scatter_(-1, torch.where(sel >= 0, sel.long(), nblk), True)
    keep_block = keep_block[..., :nblk]
    j = torch.arange(800)
    same_seg = (j[None, None, None, :] >= seg[:, None, :, None]) & (j[None, None, None, :] < torch.where(
        seg[:, None, :, None] == 0, 400, 800))
    qd = q_idx.to(dev).requires_grad_()
    kl = KL.KLChunkFn.apply(qd, idx_k[:, None].to(dev), q_main.to(dev), k_main.to(dev), keep_block.to(dev),
                            pos.to(dev), 64, scaling, 3, 1, 128, same_seg.to(dev))
    rk, _ = K.gather_kl_dense(q_idx.double(), idx_k.double(), q_main.double(), k_main.double(), sel, pos,
                              block_size=64, local_window=128, scaling=scaling, seg=seg, round_dtype=torch.bfloat16)
    err = (kl.detach().cpu().double() - rk).abs() - 1e-3 * rk.abs()
    assert err.max().item() <= 2e-3
    kl.sum().backward()
    assert qd.grad is not None and torch.isfinite(qd.grad.float()).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_slots_are_blocks_every_block(dev, dtype):
    """The warmup stage's KL: a row lists every KL-eligible block (far more than
    64), slot s = block s.  150 key blocks, two index heads of a GQA teacher,
    packed rows, some blocks unlisted (an image constraint) and some listed past
    the row's window start (no kept key: a zero dsel row); kl / valid / dsel
    against the dense oracle, then the gradients of the loss."""
    from srswa import kl as KL
    print(f"kl slots_are_blocks {dtype}", flush=True)
    g = torch.Generator().manual_seed(41)
    B, HI, G, HKV, T, Sk, D, lw = 1, 2, 3, 2, 300, 64 * 150 - 10, 128, 256
    HQ = HI * G
    nblk = -(-Sk // 64)
    q_idx = (torch.randn(B, HI, T, D, generator=g) * D ** -0.5).to(dtype)
    idx_k = torch.randn(B, Sk, D, generator=g).to(dtype)
    q_main = torch.randn(B, HQ, T, D, generator=g).to(dtype)
    k_main = torch.randn(B, HKV, Sk, D, generator=g).to(dtype)
    pos = (torch.arange(T) * 31 + 100).expand(B, T).clone().to(torch.int32)       # rows spread over the keys
    seg = torch.where(torch.arange(T) >= 200, 64 * 100 + 17, 0).expand(B, T).to(torch.int32)
    ar = torch.arange(nblk, dtype=torch.int32)
    listed = torch.rand(B, HI, T, nblk, generator=g) > 0.15
    sel = torch.where(listed, ar, torch.full_like(ar, -1))
    qd = q_idx.to(dev).requires_grad_()
    kd = idx_k.to(dev).requires_grad_()
    kw = dict(block_size=64, local_window=lw, scaling=D ** -0.5)
    kl, valid, dsel = KL.kl_forward(q_idx.to(dev), idx_k.to(dev), q_main.to(dev), k_main.to(dev), sel.to(dev),
                                    pos.to(dev), seg=seg.to(dev), slots_are_blocks=True, **kw)
    rk, rv = K.gather_kl_dense(q_idx.double(), idx_k.double(), q_main.double(), k_main.double(), sel, pos,
                               seg=seg, round_dtype=dtype, **kw)
    assert torch.equal(valid.cpu(), rv)
    assert rv.any() and (~rv).any()
    err = (kl.cpu().double() - rk).abs() - 1e-3 * rk.abs()
    assert err.max().item() <= 2e-3, err.max().item()
    # dsel on every listed slot: softmax(student) - p on kept keys, 0 elsewhere
    keep = K.keep_mask(sel, pos, Sk, 64, lw, seg)
    s = K._round(torch.einsum("bhtd,bsd->bhts", q_idx.double(), idx_k.double()), dtype).masked_fill(~keep, K.NEG)
    sm = torch.softmax(s, -1)
    p = torch.zeros_like(sm)
    for h in range(HQ):
        sh = K._round(torch.einsum("btd,bsd->bts", q_main[:, h].double(), k_main[:, h // (HQ // HKV)].double()),
                      dtype) * kw["scaling"]
        p[:, h // G] += torch.softmax(sh.masked_fill(~keep[:, h // G], K.NEG), -1)
    p /= G
    ref_ds = torch.where(keep, sm - p, torch.zeros_like(p))
    ref_ds = torch.nn.functional.pad(ref_ds, (0, nblk * 64 - Sk)).view(B, HI, T, nblk, 64)
    got = dsel.cpu().double()
    lst = listed[..., None].expand_as(got)
    assert (got[lst] - ref_ds[lst]).abs().max().item() <= 1e-4
    # the gradients (the backward reads the listed slots only)
    kl2, valid2 = KL.gather_kl(qd, kd, q_main.to(dev), k_main.to(dev), sel.to(dev), pos.to(dev), seg=seg.to(dev),
                               slots_are_blocks=True, **kw)
    K.kl_loss(kl2, valid2).backward()
    qr = q_idx.double().requires_grad_()
    kr = idx_k.double().requires_grad_()
    rk2, rv2 = K.gather_kl_dense(qr, kr, q_main.double(), k_main.double(), sel, pos, seg=seg, round_dtype=dtype,
                                 **kw)
    K.kl_loss(rk2, rv2).backward()
    assert_close_lowp(qd.grad.cpu(), qr.grad, dtype, what="d q_idx (every block)")
    assert_close_lowp(kd.grad.cpu(), kr.grad, dtype, what="d idx_k (every block)")


def test_kl_chunk_fn_warmup_keep_all(dev):
    """KLChunkFn.apply as the warmup stage calls it: keep_block = every
    KL-eligible block (restrict_to_selected=False), 130 blocks, against the
    dense oracle, and its gradient."""
    from srswa import kl as KL
    g = torch.Generator().manual_seed(43)
    B, HI, G, T, Sk, D, lw = 1, 1, 4, 128, 64 * 130, 128, 512
    q_idx = (torch.randn(B, HI, T, D, generator=g) * D ** -0.5).to(torch.bfloat16)
    idx_k = torch.randn(B, Sk, D, generator=g).to(torch.bfloat16)
    q_main = torch.randn(B, HI * G, T, D, generator=g).to(torch.bfloat16)
    k_main = torch.randn(B, 2, Sk, D, generator=g).to(torch.bfloat16)
    pos = (Sk - 64 * T + torch.arange(T) * 64).expand(B, T).clone().to(torch.int32)
    nblk = Sk // 64
    keep_block = torch.ones(B, 1, T, nblk, dtype=torch.bool)
    qd = q_idx.to(dev).requires_grad_()
    kl = KL.KLChunkFn.apply(qd, idx_k[:, None].to(dev), q_main.to(dev), k_main.to(dev), keep_block.to(dev),
                            pos.to(dev), 64, D ** -0.5, G, 2, lw, None)
    sel = torch.arange(nblk, dtype=torch.int32).expand(B, HI, T, nblk)
    qr = q_idx.double().requires_grad_()
    rk, _ = K.gather_kl_dense(qr, idx_k.double(), q_main.double(), k_main.double(), sel, pos, block_size=64,
                              local_window=lw, scaling=D ** -0.5, round_dtype=torch.bfloat16)
    err = (kl.detach().cpu().double() - rk.detach()).abs() - 1e-3 * rk.detach().abs()
    assert err.max().item() <= 2e-3
    kl.sum().backward()
    rk.sum().backward()
    assert_close_lowp(qd.grad.cpu(), qr.grad, torch.bfloat16, what="KLChunkFn warmup d q_idx")


def test_patch_rebinds_kl_chunk_fn(dev):
    import types
    from srswa import patch

    class _KLChunkFn:
        @staticmethod
        def apply(*args):
            return "eager-kl"

    base = types.ModuleType("_sparse_base_impl")
    base._KLChunkFn = _KLChunkFn
    mod = types.SimpleNamespace(_base=base)
    assert "_KLChunkFn" in patch.apply(mod)
    q_idx, idx_k, q_main, k_main, sel, pos, seg, scaling = _case(6, 1, 1, 2, 2, 70, 600, 64, 4, torch.bfloat16)
    nblk = -(-600 // 64)
    keep_block = torch.zeros(1, 1, 70, nblk + 1, dtype=torch.bool)
    keep_block.scatter_(-1, torch.where(sel >= 0, sel.long(), nblk), True)
    keep_block = keep_block[..., :nblk]
    args = (q_idx, idx_k[:, None], q_main, k_main, keep_block, pos, 64, scaling, 2, 1, 128, None)
    assert base._KLChunkFn.apply(*args) == "eager-kl"                      # host tensors: the original
    got = base._KLChunkFn.apply(*(a.to(dev) if torch.is_tensor(a) else a for a in args))
    rk, _ = K.gather_kl_dense(q_idx.double(), idx_k.double(), q_main.double(), k_main.double(), sel, pos,
                              block_size=64, local_window=128, scaling=scaling, round_dtype=torch.bfloat16)
    assert ((got.cpu().double() - rk).abs() - 1e-3 * rk.abs()).max().item() <= 2e-3
    patch.restore(mod)
    assert base._KLChunkFn is _KLChunkFn
