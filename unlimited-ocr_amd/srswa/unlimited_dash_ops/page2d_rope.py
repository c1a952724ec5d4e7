"""Drop-in for ``sglang.srt.layers.attention.unlimited_dash_ops.page2d_rope``:
the two-axis ``(tok_pos, page_pos)`` rotary (WHL!layers/attention/unlimited_dash_ops/page2d_rope.py:18-324)
with its cos / sin table and its application on the MI355X kernels.

``PageRope2D`` keeps the reference's constructor, attributes and frequency
tables (the fp32 torch formulas of page2d_rope.py:48-63, identical to
``DeepseekV2IndexerRotary2D``, HF/_sparse_base_impl.py:2019-2036); ``cos_sin``
and ``apply_page2d_rope(_pair)`` run the HIP kernels on device tensors and
keep the reference's rounding (each product and the sum rounded to the model
dtype).  Shapes the kernels do not take fall back to the eager formula, as the
reference's own wrappers do (page2d_rope.py:200-216).
"""

from __future__ import annotations

import math

import torch

from .. import page_ops
from .._lib import UnsupportedShape

# Prompt tokens of the cheapest page (page2d_rope.py:18-20).
MIN_PAGE_TOKENS = 74


def page_capacity(context_len: int) -> int:
    """Page buckets enough for any prompt of ``context_len`` tokens (page2d_rope.py:23-29)."""
    return max(1, int(context_len)) // MIN_PAGE_TOKENS + 2


class PageRope2D:
    """Frequency tables of the two-axis rotary: ``n_tok`` token pairs then
    ``page_pairs`` page pairs, ``page_mod`` folding only the page angle."""

    def __init__(self, dim: int, base_tok: float, base_page: float, page_pairs: int,
                 tok_freq_mode: str = "resample", page_mod: int = 0) -> None:
        half = dim // 2
        page_pairs = int(page_pairs)
        if not (0 < page_pairs < half):
            raise ValueError(f"[PageRope2D] page_pairs={page_pairs} must be in (0, {half}); dim={dim}")
        n_tok = half - page_pairs
        ar = torch.arange(0, n_tok, dtype=torch.int64).float()
        if str(tok_freq_mode).lower() == "truncate":
            inv_tok = 1.0 / (base_tok ** (ar * 2 / dim))
        else:
            inv_tok = 1.0 / (base_tok ** (ar / n_tok))
        inv_page = 1.0 / (base_page ** (torch.arange(0, page_pairs, dtype=torch.int64).float() / page_pairs))
        self.dim = dim
        self.n_tok = n_tok
        self.page_pairs = page_pairs
        self.base_tok = float(base_tok)
        self.base_page = float(base_page)
        self.tok_freq_mode = str(tok_freq_mode).lower()
        self.page_mod = int(page_mod or 0)
        self.inv_tok = inv_tok
        self.inv_page = inv_page
        self._dev_cache: dict = {}

    def _freqs(self, device):
        got = self._dev_cache.get(device)
        if got is None:
            got = (self.inv_tok.to(device), self.inv_page.to(device))
            self._dev_cache[device] = got
        return got

    @property
    def signature(self) -> tuple:
        return (self.dim, self.n_tok, self.page_pairs, self.base_tok, self.base_page, self.tok_freq_mode,
                self.page_mod)

    @property
    def page_mono_range(self) -> float:
        if self.page_mod > 0:
            return float(self.page_mod)
        return self.base_page ** ((self.page_pairs - 1) / self.page_pairs) * math.pi

    @property
    def tok_mono_range(self) -> float:
        return math.pi / float(self.inv_tok[-1])

    @torch.no_grad()
    def cos_sin(self, tok_pos: torch.Tensor, page_pos: torch.Tensor, dtype: torch.dtype):
        """``tok_pos`` / ``page_pos`` [T] int -> cos / sin [T, dim] in ``dtype`` (fp32 math)."""
        inv_tok, inv_page = self._freqs(tok_pos.device)
        return page_ops.page2d_cos_sin(tok_pos, page_pos, inv_tok, inv_page, dim=self.dim, page_mod=self.page_mod,
                                       dtype=dtype)


def _rope2d_eager(x, cos, sin, head_dim):
    """The eager formula (the reference's fallback for shapes its kernel skips)."""
    t = x.shape[0]
    v = x.view(t, -1, head_dim)
    half = head_dim // 2
    rot = torch.cat((-v[..., half:], v[..., :half]), dim=-1)
    return (v * cos[:, None, :] + rot * sin[:, None, :]).view_as(x)


def apply_page2d_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, head_dim: int) -> torch.Tensor:
    """NeoX rotary of ``[T, H * head_dim]`` with per-token cos / sin ``[T, head_dim]``."""
    if x.is_cuda and x.shape[0] > 0:
        try:
            return page_ops.page2d_rope(x, cos, sin, head_dim)
        except UnsupportedShape:
            pass
    return _rope2d_eager(x, cos, sin, head_dim)


def apply_page2d_rope_pair(x: torch.Tensor, y: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                           head_dim: int):
    """``apply_page2d_rope`` of two tensors sharing cos / sin, in one launch."""
    if x.is_cuda and x.shape[0] > 0 and y.shape[0] == x.shape[0]:
        try:
            return page_ops.page2d_rope(x, cos, sin, head_dim, y=y)
        except UnsupportedShape:
            pass
    return apply_page2d_rope(x, cos, sin, head_dim), apply_page2d_rope(y, cos, sin, head_dim)
