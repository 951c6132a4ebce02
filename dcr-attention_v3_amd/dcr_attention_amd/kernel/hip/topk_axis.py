"""Top-K Q-axis pipeline on MI355X -- the two entry points of the sparse path.

Drop-in for the reference's ``topk_qaxis_select`` and
``topk_qaxis_attention`` (dcr_attention/kernel/triton/topk_axis.py:20-90):
same signatures, same results.  Each is one call into the C ABI, which
enqueues, on torch's current stream, three launches:

  score kernel   u = Q / max(||Q||, eps) (fp32) for the GQA group, then the
                 16-bit keys of the bf16 scores of all N positions (fp16/bf16:
                 plus one residual byte per score) and level-1 histogram slabs
  select_kernel  exact top-k, ascending int32 indices (rows too few to fill
                 the device: two chunked launches)
  attn_kernel    gather + online softmax, split-k; the last workgroup of each
                 GQA group merges the partials and rounds to Q's dtype
                 (attention only)

The one score shape whose u operand does not fit in registers (8 query heads
per KV head at D = 128) computes u in a separate uq_kernel launch first.
``_lib.set_sparse_path`` selects another launch sequence for
``topk_qaxis_attention`` (the whole step in one persistent launch, or an
attention that gathers each V row of a GQA group once); the three launches
above are the default.

``compute_u_Q`` is the device counterpart of the M1 helper ``_compute_u_Q``
(qaxis_topk_reference.py:42-55) that the reference's Triton path calls on the
host side (topk_axis.py:47).
"""
from __future__ import annotations

import torch

from dcr_attention_amd import _lib

_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def compute_u_Q(Q: torch.Tensor, eps: float = 1e-12) -> torch.Tensor:
    """u_Q = Q / max(||Q||_2, eps) over the last dim, fp32 (same shape as Q)."""
    lib = _lib.load()
    _lib.require_device(Q, what="u_Q")
    assert Q.dtype in _DTYPES, f"Q must be fp32/fp16/bf16, got {Q.dtype}"
    assert Q.is_contiguous(), "Q must be contiguous"
    D = Q.shape[-1]
    u = torch.empty(Q.shape, dtype=torch.float32, device=Q.device)
    rc = lib.dcr_compute_uq(Q.data_ptr(), _lib.DTYPE_CODE[Q.dtype], u.data_ptr(), Q.numel() // D,
                            D, float(eps), _lib.stream_of(Q))
    _lib.check(rc, "compute_u_Q")
    return u


def _check_qk(Q: torch.Tensor, K_cache: torch.Tensor, k_eff: int):
    B, H, D = Q.shape
    B_k, H_kv, N, D_k = K_cache.shape
    assert Q.dtype in _DTYPES, f"Q must be fp32/fp16/bf16, got {Q.dtype}"
    assert K_cache.dtype == Q.dtype, f"K_cache dtype {K_cache.dtype} != Q dtype {Q.dtype}"
    assert B == B_k and D == D_k, "Q and K_cache batch/head-dim mismatch"
    assert H % H_kv == 0, f"H={H} must be divisible by H_kv={H_kv}"
    assert k_eff > 0 and k_eff < N, f"k_eff={k_eff} must be in (0, N={N})"
    assert Q.is_contiguous(), "Q must be contiguous"
    return B, H, H_kv, N, D


def topk_qaxis_select(
    Q: torch.Tensor,         # [B, H, D]
    K_cache: torch.Tensor,   # [B, H_kv, N, D]
    k_eff: int,
    *,
    eps: float = 1e-12,
) -> torch.Tensor:           # [B, H, k_eff] int32, sorted ascending
    """Top-k key indices by Q-axis projection (u_Q + Pass 1 + Pass 2)."""
    lib = _lib.load()
    _lib.require_device(Q, K_cache, what="topk_qaxis_select")
    B, H, H_kv, N, D = _check_qk(Q, K_cache, k_eff)
    ldn = _lib.kv_head_stride(K_cache)
    idx = torch.empty(B, H, k_eff, dtype=torch.int32, device=Q.device)
    ws_bytes = lib.dcr_qaxis_select_workspace_bytes(B, H, H_kv, N, D, _lib.DTYPE_CODE[Q.dtype])
    ws = _lib.workspace(ws_bytes, Q.device)
    rc = lib.dcr_qaxis_select(Q.data_ptr(), K_cache.data_ptr(), _lib.DTYPE_CODE[Q.dtype],
                              idx.data_ptr(), B, H, H_kv, N, ldn, D, k_eff, float(eps),
                              ws.data_ptr(),
                              ws_bytes, _lib.stream_of(Q))
    _lib.check(rc, "topk_qaxis_select")
    return idx


def topk_qaxis_attention(
    Q: torch.Tensor,            # [B, H, D]
    K_cache: torch.Tensor,      # [B, H_kv, N, D]
    V_cache: torch.Tensor,      # [B, H_kv, N, D]
    k_eff: int,
    *,
    eps: float = 1e-12,
    return_indices: bool = False,
):
    """Full sparse decode attention: Q + K_cache + V_cache -> O [B, H, D].

    ``return_indices=True`` (an addition; the reference has no such flag)
    also returns the int32 [B, H, k_eff] indices that were attended.
    """
    lib = _lib.load()
    _lib.require_device(Q, K_cache, V_cache, what="topk_qaxis_attention")
    B, H, H_kv, N, D = _check_qk(Q, K_cache, k_eff)
    assert V_cache.dtype == Q.dtype, f"V_cache dtype {V_cache.dtype} != Q dtype {Q.dtype}"
    ldn = _lib.kv_head_stride(K_cache, V_cache)
    O = torch.empty(B, H, D, dtype=Q.dtype, device=Q.device)
    idx = torch.empty(B, H, k_eff, dtype=torch.int32, device=Q.device) if return_indices else None
    ws_bytes = lib.dcr_sparse_decode_workspace_bytes(B, H, H_kv, N, D, k_eff,
                                                     _lib.DTYPE_CODE[Q.dtype])
    ws = _lib.workspace(ws_bytes, Q.device)
    rc = lib.dcr_sparse_decode(Q.data_ptr(), K_cache.data_ptr(), V_cache.data_ptr(),
                               _lib.DTYPE_CODE[Q.dtype], O.data_ptr(),
                               idx.data_ptr() if idx is not None else None,
                               B, H, H_kv, N, ldn, D, k_eff, float(eps), ws.data_ptr(), ws_bytes,
                               _lib.stream_of(Q))
    _lib.check(rc, "topk_qaxis_attention")
    return (O, idx) if return_indices else O
