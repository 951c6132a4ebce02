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


# The reference module's name for its GPU forward.
rank_local_fwd_triton = rank_local_fwd_hip
