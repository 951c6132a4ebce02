"""Dense GQA decode attention on MI355X (comparator and k >= N fallback).

Computes the decode case (one query token) of the reference caller's dense
branch ``_sdpa_forward`` (dcr_attention/models/llama/attention.py:673-739):
``softmax_fp32(Q K^T / sqrt(D)) V`` over all N cached rows, with the GQA
mapping h -> h // n_rep done by indexing instead of materialising
``repeat_kv`` (attention.py:425-426).  Output in Q's dtype.
"""
from __future__ import annotations

import torch

from dcr_attention_amd import _lib

_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def dense_decode_attention(
    Q: torch.Tensor,            # [B, H, D]
    K_cache: torch.Tensor,      # [B, H_kv, N, D]
    V_cache: torch.Tensor,      # [B, H_kv, N, D]
) -> torch.Tensor:              # [B, H, D]
    lib = _lib.load()
    _lib.require_device(Q, K_cache, V_cache, what="dense decode attention")
    B, H, D = Q.shape
    B_k, H_kv, N, D_k = K_cache.shape
    assert Q.dtype in _DTYPES and K_cache.dtype == Q.dtype and V_cache.dtype == Q.dtype
    assert B == B_k and D == D_k and H % H_kv == 0
    assert Q.is_contiguous()
    ldn = _lib.kv_head_stride(K_cache, V_cache)
    O = torch.empty(B, H, D, dtype=Q.dtype, device=Q.device)
    ws_bytes = lib.dcr_dense_decode_workspace_bytes(B, H, H_kv, N, D)
    ws = _lib.workspace(ws_bytes, Q.device)
    rc = lib.dcr_dense_decode(Q.data_ptr(), K_cache.data_ptr(), V_cache.data_ptr(),
                              _lib.DTYPE_CODE[Q.dtype], O.data_ptr(), B, H, H_kv, N, ldn, D,
                              ws.data_ptr(), ws_bytes, _lib.stream_of(Q))
    _lib.check(rc, "dense_decode_attention")
    return O
