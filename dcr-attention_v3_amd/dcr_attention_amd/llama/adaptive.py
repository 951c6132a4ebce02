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
