"""srswa_gather_decode_noalloc (the allocation-free decode, split-K records in
a static device array) against srswa_gather_decode with a caller-owned
workspace, through the C ABI: the same kernels and record layout, so the
outputs are bitwise equal.  Two calls in a row, the second on a smaller
input (the array keeps the first call's records; the second must not read
them).  A call whose workspace exceeds the static array is refused on the
host before any launch."""

import ctypes

import pytest
import torch

from srswa import _lib, ops
from srswa import workloads as W

pytestmark = pytest.mark.gpu


def _run_both(dev, B, Lmax, lo, k):
    c = W.decode_config(B=B, H=10, D=128, Lmax=Lmax, lo=lo, k=k)
    args = (c["q"].to(dev), c["k_cache"].to(dev), c["v_cache"].to(dev), c["block_idx"].to(dev), c["q_pos"].to(dev))
    kw = dict(block_size=c["block_size"], local_window=c["local_window"], scale=c["scale"], return_lse=True)
    launch, ref, ref_lse = ops.prepare_gather_decode(*args, **kw)
    launch()
    a = launch.args                                   # the same argument struct ...
    out = torch.empty_like(ref)
    lse = torch.empty_like(ref_lse)
    a2 = _lib.DecodeArgs.from_buffer_copy(a)          # ... writing into fresh outputs
    a2.out, a2.lse = out.data_ptr(), lse.data_ptr()
    need = _lib.lib().srswa_gather_decode_workspace(ctypes.byref(a2))
    print(f"no-alloc decode: B={B} Lmax={Lmax} k={k}, split-K scratch {need} bytes", flush=True)
    assert need > 0                                   # the static array is used
    st = _lib.lib().srswa_gather_decode_noalloc(ctypes.byref(a2), _lib.stream_ptr(dev))
    _lib.check(st, "srswa_gather_decode_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(out, ref) and torch.equal(lse, ref_lse)


def test_noalloc_matches_workspace_entry_point(dev):
    _run_both(dev, B=12, Lmax=20000, lo=4000, k=8)    # larger first
    _run_both(dev, B=3, Lmax=6000, lo=1500, k=4)      # then a smaller input on the same array


def test_noalloc_refuses_oversize_before_launch(dev):
    a = _lib.DecodeArgs()
    a.B, a.Lq, a.HQ, a.HKV, a.HI, a.D, a.S, a.L = 4096, 1, 10, 10, 10, 128, 8, 131072
    a.block_size, a.local_window, a.in_dtype, a.out_dtype = 64, 512, _lib.SRSWA_BF16, _lib.SRSWA_BF16
    need = _lib.lib().srswa_gather_decode_workspace(ctypes.byref(a))
    assert need > 8 << 20
    st = _lib.lib().srswa_gather_decode_noalloc(ctypes.byref(a), _lib.stream_ptr(dev))
    assert st == _lib.SRSWA_WORKSPACE
    assert b"static" in _lib.lib().srswa_last_error()
