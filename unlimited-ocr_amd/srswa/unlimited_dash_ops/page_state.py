"""Drop-in for the multi-token steps of the serving backend's page state:
``PageIsolationState.step`` (WHL!layers/attention/unlimited_dash_ops/page_state.py:218-313)
and ``PageCoordState.step`` (WHL!…/page2d_rope.py:534-620), on the MI355X
page-step kernels.

Both functions take the backend's state object as ``self`` (duck-typed: its
per-slot / per-row int32 state tensors and its own ``_ensure``, and for the
coordinates its ``_rows`` row allocation, ``_rewind_rejected`` speculative
rewind and ``_snapshot``, which stay the backend's torch code), so they can be
bound as the two classes' ``step`` methods.  The scans, page rules, ranks and
state writes are the kernels'; nothing runs on the host.
"""

from __future__ import annotations

import torch

from .. import page_ops


def _stable(self, name: str, t_len: int, dtype, device):
    """A fixed-address output buffer per (name, length) on the state object
    (the reference copies into the backend's named buffers for CUDA-graph
    replay)."""
    bufs = self.__dict__.setdefault("_srswa_bufs", {})
    key = (name, t_len, dtype, str(device))
    buf = bufs.get(key)
    if buf is None:
        buf = torch.empty(t_len, dtype=dtype, device=device)
        bufs[key] = buf
    return buf


@torch.no_grad()
def page_isolation_step(self, input_ids, layout, slot_mapping, num_slots):
    """``PageIsolationState.step``: q_page int32 [num_tokens] (-1 = page
    unknown); the per-slot state is updated in place."""
    self._ensure(num_slots, input_ids.device)
    T = int(layout.num_tokens)
    out = _stable(self, "q_page", T, torch.int32, input_ids.device)
    page_ops.page_step(input_ids[:T], layout.q_start, layout.start_pos, layout.block_table, slot_mapping[:T],
                       s_page=self._slot_img_page, s_mark=self._slot_marker_cum, s_run=self._slot_img_run,
                       s_pp=self._slot_prompt_pages, image_token_id=self.image_token_id,
                       page_token_id=self.page_token_id, per_page=self.per_page_image_tokens,
                       block_size=self.block_size, num_decode_tokens=int(layout.num_decode_tokens),
                       gen_start=layout.gen_start, n_slots=num_slots, out_q_page=out)
    # the backend's diagnostic of an incompatible per_page value reads this;
    # the device step leaves it unset
    self._last_img_run_max = None
    return out


@torch.no_grad()
def coord_step(self, input_ids, layout):
    """``PageCoordState.step``: (tok_pos, page_pos) [num_tokens] int64, or
    None for an empty step."""
    t = int(layout.num_tokens)
    if t <= 0:
        return None
    device = input_ids.device
    self._ensure(device)
    row = self._rows(layout)
    # undo the tokens the previous step committed but the verifier rejected
    self._rewind_rejected(layout, row)
    st_marker_in = self.st_marker[row]
    st_pp_in = self.st_pp[row]
    cnt_in = self.cnt[row]
    tok, page, marker, pp = page_ops.coord_step(
        input_ids[:t], layout.q_start, layout.start_pos, row, st_marker=self.st_marker, st_pp=self.st_pp,
        cnt=self.cnt, image_token_id=self.image_token_id, page_token_id=self.page_token_id,
        num_decode_tokens=int(layout.num_decode_tokens), gen_start=layout.gen_start, with_carry=True)
    starts = layout.q_start[:-1].to(torch.int64)
    q_len = layout.q_start[1:].to(torch.int64) - starts
    tok_idx = torch.arange(t, device=device, dtype=torch.int64)
    self._snapshot(layout, row, layout.req_of_token.to(torch.int64), starts, q_len, tok_idx, marker, pp, page,
                   st_marker_in, st_pp_in, cnt_in)
    return tok, page
