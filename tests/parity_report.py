"""Parity figures that every run shows, not only failing ones.

``report`` prints a line and keeps it; ``tests/conftest.py`` repeats the
kept lines in pytest's terminal summary (so they appear under ``-q`` too).

``compare_selection`` is the block-id bar of the task: the selected SET of
every row must equal the oracle's, except in rows whose k-th and (k+1)-th
oracle scores are closer than 1e-4 * max(1, |s_k|) ("near ties", where the
fp32 summation order may legitimately swap the two).  It reports, per case,
the rows compared, the rows whose set matches exactly, the near-tie rows (and
how many of them differ), and the rows that differ outside near ties, which
must be zero.
"""

from __future__ import annotations

import torch

from oracle import srswa_oracle as O

LINES: list[str] = []


def report(line: str) -> None:
    LINES.append(line)
    print(line, flush=True)


def compare_selection(got, ref_scores, k, what, *, invalid_at=O.SCORE_NEG * 0.5, max_near_frac=0.05,
                      tie_floor=1.0):
    """got int [..., k] selected ids (any order, -1 = empty); ref_scores [..., n]
    the oracle's scores of the same rows.  ``tie_floor``: the near-tie gap is
    1e-4 * max(tie_floor, |s_k|).  Returns the counts dict."""
    ref = O.topk_blocks(ref_scores, k, invalid_at=invalid_at)
    ties = O.near_tie_rows(ref_scores, k, invalid_at=invalid_at, floor=tie_floor)
    same = (torch.sort(got.long(), -1).values == torch.sort(ref, -1).values).all(-1)
    counts = {"rows": int(same.numel()), "exact": int(same.sum()), "near_tie": int(ties.sum()),
              "near_tie_differ": int(((~same) & ties).sum()), "mismatched": int(((~same) & (~ties)).sum())}
    report(f"[ids] {what}: rows {counts['rows']}, exact {counts['exact']}, near-tie {counts['near_tie']} "
           f"(differ {counts['near_tie_differ']}), mismatched outside near-ties {counts['mismatched']}")
    assert counts["mismatched"] == 0, f"{what}: {counts['mismatched']} rows differ outside near-ties"
    assert counts["near_tie"] <= max(1, int(max_near_frac * counts["rows"])), counts
    return counts


def report_error(what, got, ref, bar):
    """Print the plain max-abs error of ``got`` against ``ref`` beside its bar."""
    err = (got.double() - ref.double()).abs().max().item() if got.numel() else 0.0
    report(f"[err] {what}: max-abs {err:.3e} (bar {bar})")
    return err
