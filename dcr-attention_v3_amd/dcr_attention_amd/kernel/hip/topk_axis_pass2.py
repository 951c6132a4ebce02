"""Pass 2 -- exact top-K selection on MI355X.

Drop-in for ``topk_pass2_select`` (reference
dcr_attention/kernel/triton/topk_axis_pass2.py:16-43), which runs a stable
descending ``torch.argsort`` of every row, keeps the first ``k_eff`` and sorts
them ascending.  This version returns the identical index set and order from
a two-level radix select on the order-preserving 16-bit key of each bf16 score
(no sort): ties at the threshold go to the lower index, -0 equals +0, NaN
ranks above +inf, output int32 ascending.
"""
from __future__ import annotations

import torch

from dcr_attention_amd import _lib


def topk_pass2_select(
    scores: torch.Tensor,    # [B, H, N] bf16 (from Pass 1)
    k_eff: int,
) -> torch.Tensor:           # [B, H, k_eff] int32, sorted ascending
    """Indices of the k_eff largest scores per row (stable, ascending)."""
    lib = _lib.load()
    _lib.require_device(scores, what="Pass 2")

    *lead, N = scores.shape
    assert scores.dtype == torch.bfloat16, f"scores must be bf16, got {scores.dtype}"
    assert k_eff > 0, f"k_eff must be > 0, got {k_eff}"
    assert k_eff < N, f"k_eff={k_eff} must be < N={N} (caller's contract)"
    assert scores.is_contiguous(), "scores must be contiguous"

    rows = scores.numel() // N
    idx = torch.empty(*lead, k_eff, dtype=torch.int32, device=scores.device)
    ws_bytes = lib.dcr_topk_select_workspace_bytes(rows, N)
    ws = _lib.workspace(ws_bytes, scores.device)
    rc = lib.dcr_topk_select(scores.data_ptr(), idx.data_ptr(), rows, N, k_eff, ws.data_ptr(),
                             ws_bytes, _lib.stream_of(scores))
    _lib.check(rc, "topk_pass2_select")
    return idx
