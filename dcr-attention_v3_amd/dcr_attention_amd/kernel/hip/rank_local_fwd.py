"""Rank-local (sorted-window) attention forward on MI355X.

Mirrors ``rank_local_fwd_triton`` (dcr_attention/kernel/rank_local_fwd_triton.py:
216-334): the same arguments, shapes, defaults and exceptions, returning
``(O, LSE)``.  Query i of head (b, h) -- in the caller's sorted-Q order --
attends to the sorted key positions j with ``|j - r_center[b,h,i]| <= k_window // 2``
with fp32 logits ``Q·K * scale`` and fp32 softmax state; ``O`` is in Q's
dtype, ``LSE`` is the fp32 natural-log sum of exponentials of each row.
``BLOCK_Q``, ``BLOCK_K`` and ``num_stages`` are accepted for signature
compatibility (the HIP kernel picks its own tiling) and ignored.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from dcr_attention_amd import _lib

_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def rank_local_fwd_hip(
    Q: torch.Tensor,
    K_sorted: torch.Tensor,
    V_sorted: torch.Tensor,
    rank_of_k: torch.Tensor,
    r_center: torch.Tensor,
    k_window: int,
    scale: Optional[float] = None,
    BLOCK_Q: Optional[int] = None,
    BLOCK_K: Optional[int] = None,
    num_stages: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Q [B, H, N_q, D], K_sorted / V_sorted [B, H, N_kv, D], r_center [B, H, N_q]
    -> O [B, H, N_q, D] (Q's dtype), LSE [B, H, N_q] fp32.  ``rank_of_k`` is
    unused, as in the reference (kept for signature symmetry)."""
    del rank_of_k, BLOCK_Q, BLOCK_K, num_stages
    lib = _lib.load()
    if not (Q.is_cuda and K_sorted.is_cuda and V_sorted.is_cuda and r_center.is_cuda):
        raise RuntimeError("rank_local_fwd_hip requires device tensors.")
    B, H, N_q, D = Q.shape
    N_kv = K_sorted.shape[-2]
    if K_sorted.shape != V_sorted.shape:
        raise ValueError(f"K_sorted shape {tuple(K_sorted.shape)} must equal "
                         f"V_sorted shape {tuple(V_sorted.shape)}")
    if K_sorted.shape[:2] != Q.shape[:2] or K_sorted.shape[-1] != D:
        raise ValueError(f"K_sorted shape {tuple(K_sorted.shape)} incompatible with "
                         f"Q shape {tuple(Q.shape)}: B, H, D must match")
    if r_center.shape != (B, H, N_q):
        raise ValueError(f"r_center shape {tuple(r_center.shape)} must equal [B={B}, H={H}, N_q={N_q}]")
    if Q.dtype not in _DTYPES or K_sorted.dtype != Q.dtype or V_sorted.dtype != Q.dtype:
        raise ValueError(f"Q/K/V must share one of {_DTYPES}, got {Q.dtype}, {K_sorted.dtype}, "
                         f"{V_sorted.dtype}")
    if scale is None:
        scale = 1.0 / (D ** 0.5)
    BH = B * H
    Q_f = Q.reshape(BH, N_q, D).contiguous()
    K_f = K_sorted.reshape(BH, N_kv, D).contiguous()
    V_f = V_sorted.reshape(BH, N_kv, D).contiguous()
    r_f = r_center.reshape(BH, N_q).to(torch.int32).contiguous()
    O = torch.empty_like(Q_f)
    LSE = torch.empty((BH, N_q), device=Q.device, dtype=torch.float32)
    rc = lib.dcr_rank_local_fwd(Q_f.data_ptr(), K_f.data_ptr(), V_f.data_ptr(),
                                _lib.DTYPE_CODE[Q.dtype], r_f.data_ptr(), O.data_ptr(),
                                LSE.data_ptr(), BH, N_q, N_kv, D, int(k_window), float(scale),
                                _lib.stream_of(Q))
    _lib.check(rc, "rank_local_fwd_hip")
    return O.reshape(B, H, N_q, D), LSE.reshape(B, H, N_q)


def cache_layout_ok(X: torch.Tensor) -> bool:
    """Whether the kernel can read a [B, H_kv, N, D] cache view in place."""
    try:
        _cache_rows(X)
        return True
    except ValueError:
        return False


def _cache_rows(X: torch.Tensor) -> int:
    """Rows between KV heads of a [B, H_kv, N, D] cache view whose rows are
    contiguous and whose heads are evenly spaced within each batch entry."""
    B, Hkv, N, D = X.shape
    if X.stride(3) != 1 or X.stride(2) != D or X.stride(1) % D != 0 or X.stride(1) < N * D:
        raise ValueError(f"K/V must have contiguous rows and a head stride that is a multiple of D "
                         f"and at least N*D, got strides {tuple(X.stride())}")
    if B > 1 and X.stride(0) != Hkv * X.stride(1):
        raise ValueError(f"K/V heads must be evenly spaced across the batch, got strides {tuple(X.stride())}")
    return X.stride(1) // D


def rank_local_fwd_gather_hip(Q_sorted: torch.Tensor, K: torch.Tensor, V: torch.Tensor,
                              sort_idx_k: torch.Tensor, r_center: torch.Tensor, k_window: int,
                              scale: Optional[float] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """The forward of ``rank_local_fwd_hip`` on K/V read in place through the
    sort permutation: K, V [B, H or H_kv, N_kv, D] (the cache, or a strided
    view of it), sort_idx_k [B, H, N_kv].  Equal bit for bit to
    ``rank_local_fwd_hip(Q_sorted, gather(K), gather(V), ...)`` without the
    two sorted copies of the cache."""
    lib = _lib.load()
    if not (Q_sorted.is_cuda and K.is_cuda and V.is_cuda and sort_idx_k.is_cuda and r_center.is_cuda):
        raise RuntimeError("rank_local_fwd_gather_hip requires device tensors.")
    B, H, N_q, D = Q_sorted.shape
    if K.shape != V.shape or K.dim() != 4 or K.shape[0] != B or K.shape[3] != D or H % K.shape[1] != 0:
        raise ValueError(f"K {tuple(K.shape)} / V {tuple(V.shape)} incompatible with Q {tuple(Q_sorted.shape)}")
    Hkv, N_kv = K.shape[1], K.shape[2]
    if sort_idx_k.shape != (B, H, N_kv):
        raise ValueError(f"sort_idx_k shape {tuple(sort_idx_k.shape)} must be [B={B}, H={H}, N_kv={N_kv}]")
    if r_center.shape != (B, H, N_q):
        raise ValueError(f"r_center shape {tuple(r_center.shape)} must equal [B={B}, H={H}, N_q={N_q}]")
    if Q_sorted.dtype not in _DTYPES or K.dtype != Q_sorted.dtype or V.dtype != Q_sorted.dtype:
        raise ValueError(f"Q/K/V must share one of {_DTYPES}")
    if K.stride() != V.stride():
        raise ValueError("K and V must share one layout")
    ldn = _cache_rows(K)
    if scale is None:
        scale = 1.0 / (D ** 0.5)
    Q_f = Q_sorted.reshape(B * H, N_q, D).contiguous()
    perm = sort_idx_k.reshape(B * H, N_kv).to(torch.int32).contiguous()
    r_f = r_center.reshape(B * H, N_q).to(torch.int32).contiguous()
    O = torch.empty_like(Q_f)
    LSE = torch.empty((B * H, N_q), device=Q_sorted.device, dtype=torch.float32)
    rc = lib.dcr_rank_local_fwd_gather(Q_f.data_ptr(), K.data_ptr(), V.data_ptr(), _lib.DTYPE_CODE[Q_sorted.dtype],
                                       perm.data_ptr(), r_f.data_ptr(), O.data_ptr(), LSE.data_ptr(), B, H, Hkv,
                                       N_q, N_kv, ldn, D, int(k_window), float(scale), _lib.stream_of(Q_sorted))
    _lib.check(rc, "rank_local_fwd_gather_hip")
    return O.reshape(B, H, N_q, D), LSE.reshape(B, H, N_q)


# The reference module's name for its GPU forward.
rank_local_fwd_triton = rank_local_fwd_hip
