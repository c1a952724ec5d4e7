"""Drop-in for the reference's serving operators,
``sglang.srt.layers.attention.unlimited_dash_ops`` (WHL!layers/attention/unlimited_dash_ops/),
module for module, on the MI355X kernels:

* ``attend_triton``       -- ``dash_sparse_attn``, ``dash_sparse_attn_decode``
* ``dash_stage0``         -- ``KBarCache``, ``headcls_scores_prefill``, ``headcls_scores_decode``
* ``decode_meta_triton``  -- ``decode_meta_fused``, ``decode_allow_fused``, ``cos_sin_2d_fused``,
                             ``local_union_fused``
* ``page2d_rope``         -- ``PageRope2D``, ``apply_page2d_rope``, ``apply_page2d_rope_pair``,
                             ``page_capacity``
* ``page_state``          -- ``page_isolation_step`` / ``coord_step``: the ``step`` methods of the
                             backend's ``PageIsolationState`` / ``PageCoordState``
* ``route_triton``        -- ``route_decode_triton``, ``route_prefill_triton``,
                             ``kbar_refresh_tail_triton``, ``win_bounds_decode``,
                             ``kbar_tail_plan``, ``kbar_all_plan``, ``prefill_row2req``

Every tensor the kernels see must live on the GPU (no host path).
"""

from .attend_triton import SPARSE_BLOCK_SIZE, dash_sparse_attn, dash_sparse_attn_decode  # noqa: F401
from .dash_stage0 import KBarCache, headcls_scores_decode, headcls_scores_prefill  # noqa: F401
from .decode_meta_triton import (  # noqa: F401
    cos_sin_2d_fused, decode_allow_fused, decode_meta_fused, local_union_fused)
from .page_state import coord_step, page_isolation_step  # noqa: F401
from .page2d_rope import (  # noqa: F401
    MIN_PAGE_TOKENS, PageRope2D, apply_page2d_rope, apply_page2d_rope_pair, page_capacity)
from .route_triton import (  # noqa: F401
    SCAN_TILE, kbar_all_plan, kbar_refresh_tail_triton, kbar_tail_plan, prefill_row2req, route_decode_triton,
    route_prefill_triton, win_bounds_decode)
