"""srswa -- MI355X-native Sparse-Reference Sliding-Window Attention (SR-SWA).

HIP kernels for gfx950 behind a C ABI (libsrswa.so, include/srswa.h), driven
from PyTorch-ROCm.  Drop-in modules keep the reference's Python surface:

* ``srswa.sparse_gather_triton``      -- triton_gather_attention, triton_block_max_score
* ``srswa.sparse_gather_e2e_triton``  -- triton_gather_attention_e2e
* ``srswa.unlimited_dash_ops``        -- the SGLang serving operators, module for module
* ``srswa.patch``                     -- rebinding of the HF model's decode attend, router
                                         scores / selection, page isolation and Page2D RoPE
* ``srswa.ops`` / ``srswa.page_ops``  -- the raw operators over the C ABI
"""

from . import _lib  # noqa: F401
from ._lib import UnsupportedShape  # noqa: F401
from .ops import decode_attend, gather_decode, index_meanpool_topk, topk_rows  # noqa: F401

__version__ = "0.1.0"
