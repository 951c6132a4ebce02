"""Effective top-K size per decode step.

``adaptive_k_window`` follows the reference's rule
(dcr_attention/models/llama/adaptive.py:39-105) exactly, including its
float product and truncation, because the caller's k_eff defines which
index set the kernels must reproduce:

    k = min(n_kv, max(k_window_min, int(n_kv * coverage_floor)))
    if k is odd: k = min(k + 1, n_kv)

e.g. n_kv = 32769, c = 0.15 -> int(4915.35) = 4915 -> 4916; n_kv = 4096 ->
614 (the benchmark rule ceil(c * N) gives 615 there).
"""
from __future__ import annotations

import torch


def adaptive_k_window(k_window_min: int, n_kv: int, coverage_floor: float) -> int:
    """k_eff for ``n_kv`` cached keys: at least ``k_window_min`` (when
    n_kv allows), at most ``n_kv``, even unless capped at an odd ``n_kv``."""
    if n_kv <= 0:
        raise ValueError(f"n_kv must be > 0, got {n_kv}")
    if not (0.0 <= coverage_floor <= 1.0):
        raise ValueError(f"coverage_floor must be in [0, 1], got {coverage_floor}")
    k = min(max(k_window_min, int(n_kv * coverage_floor)), n_kv)
    if k & 1:
        k = min(k + 1, n_kv)
    return k


def detect_leaky_boundary(q_proj: torch.Tensor, k_proj: torch.Tensor, sort_idx: torch.Tensor,
                          k_window_eff: int, slack: float = 0.5) -> torch.Tensor:
    """Rank-local safety check (adaptive.py:108-195): [B, H] True where some
    key outside the window lies closer to the query in projection space than
    ``slack`` times the farthest key inside it.

    q_proj [B, H, 1] (query . axis), k_proj [B, H, N_kv] (keys . axis, caller
    order), sort_idx = argsort(k_proj).  The window is the k_window_eff sorted
    positions starting at the query's insertion rank minus k_window_eff // 2,
    shifted back inside [0, N_kv)."""
    B, H, N_kv = k_proj.shape
    if k_window_eff >= N_kv:
        return torch.zeros(B, H, dtype=torch.bool, device=k_proj.device)
    k_sorted = torch.gather(k_proj, -1, sort_idx)
    dist = (k_sorted - q_proj).abs()
    rank = torch.searchsorted(k_sorted.contiguous(), q_proj.contiguous()).squeeze(-1).clamp(0, N_kv - 1)
    start = (rank - k_window_eff // 2).clamp(min=0)
    end = (start + k_window_eff).clamp(max=N_kv)
    start = (end - k_window_eff).clamp(min=0)
    pos = torch.arange(N_kv, device=k_proj.device).view(1, 1, -1)
    inside = (pos >= start.unsqueeze(-1)) & (pos < end.unsqueeze(-1))
    d_in = torch.where(inside, dist, torch.zeros_like(dist)).amax(dim=-1)
    d_out = torch.where(inside, torch.full_like(dist, torch.finfo(dist.dtype).max), dist).amin(dim=-1)
    return d_out < slack * d_in


def widen_factor(prev_k: int, n_kv: int, multiplier: float = 2.0) -> int:
    """Widened window after a leaky check (adaptive.py:198-221): int(prev_k *
    multiplier) capped at n_kv, rounded up to even, and at least prev_k + 2."""
    new_k = min(int(prev_k * multiplier), n_kv)
    if new_k & 1:
        new_k = min(new_k + 1, n_kv)
    return max(new_k, prev_k + 2)
