"""Public rank-local attention (forward) on MI355X.

Mirrors ``rank_local_attention`` (dcr_attention/kernel/rank_local_attention.py:
142-200, forward :62-125): the same arguments, defaults and exceptions.  Keys
and queries are ordered by their projection on ``axis`` (normalised here,
:38-54), query i attends to the keys whose sorted position lies within
``k_window // 2`` of its insertion rank, and the output comes back in the
caller's query order:

  1. ``prepare_sort_indices`` (sort bookkeeping, pure torch);
  2. Q gathered into Q-sorted order; K and V are not copied: the HIP kernel
     reads their rows in place through the K-sort permutation
     (``rank_local_fwd_gather_hip``: the reference gathers both into sorted
     copies first, two passes over the cache);
  3. the HIP kernel (``kernel.hip.rank_local_fwd``), in sorted Q order;
  4. ``scatter_by_inv_perm`` back to the caller's order.

Forward only, as in the reference (its backward raises NotImplementedError).
K and V may hold H_kv heads dividing Q's H (an un-repeated GQA cache); the
result equals that of the repeated cache.
"""
from __future__ import annotations

from typing import Optional

import torch

from dcr_attention_amd.kernel.hip.rank_local_fwd import cache_layout_ok, rank_local_fwd_gather_hip
from dcr_attention_amd.kernel.sort_helpers import (gather_by_sort_idx, prepare_sort_indices,
                                                    scatter_by_inv_perm)

_EPS = 1e-12


def _normalize_axis(axis: torch.Tensor) -> torch.Tensor:
    """axis / (||axis|| + 1e-12) over the last dim; [D] or [B, H, D]."""
    if axis.dim() == 1:
        return axis / (axis.norm() + _EPS)
    if axis.dim() == 3:
        return axis / (axis.norm(dim=-1, keepdim=True) + _EPS)
    raise ValueError(f"axis must be [D] or [B, H, D], got shape {tuple(axis.shape)}")


def rank_local_attention(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, axis: torch.Tensor,
                         k_window: int = 64, scale: Optional[float] = None) -> torch.Tensor:
    """Q [B, H, N_q, D]; K, V [B, H or H_kv, N_kv, D]; axis [D] or [B, H, D].
    Returns [B, H, N_q, D] in Q's dtype and the caller's query order."""
    B, H, _, D = Q.shape
    if axis.dim() == 1:
        if axis.shape[0] != D:
            raise ValueError(f"axis shape {tuple(axis.shape)} must be [D={D}]")
    elif axis.dim() == 3:
        if axis.shape != (B, H, D):
            raise ValueError(f"axis shape {tuple(axis.shape)} must be [B={B}, H={H}, D={D}]")
    else:
        raise ValueError(f"axis must be [D] or [B, H, D], got {axis.dim()}-D shape {tuple(axis.shape)}")
    if scale is None:
        scale = 1.0 / (D ** 0.5)
    if not (cache_layout_ok(K) and K.stride() == V.stride()):
        # layouts the kernel cannot read in place (e.g. transposed rows)
        K, V = K.contiguous(), V.contiguous()
    idx = prepare_sort_indices(Q, K, _normalize_axis(axis))
    Q_sorted = gather_by_sort_idx(Q, idx.sort_idx_q)
    O_sorted, _ = rank_local_fwd_gather_hip(Q_sorted, K, V, idx.sort_idx_k, idx.r_center,
                                            k_window=k_window, scale=scale)
    return scatter_by_inv_perm(O_sorted, idx.inv_q_perm)
