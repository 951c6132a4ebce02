"""Pass 3 -- fused K/V gather + online-softmax GQA attention on MI355X.

Drop-in for ``fused_topk_attention`` (reference
dcr_attention/kernel/triton/fused_attn.py:158-211).  Same arguments; the
reference's bf16-only, ``n_per_kv == 4`` and ``D == 64`` restrictions
(:179-193) are lifted.  Logits and the softmax state (m, l, o) are fp32, the
output is rounded once to Q's dtype.  Unlike the reference's one program per
(b, h), the HIP kernel splits each head's index list across workgroups
(FlashDecoding-style (m, l, o) partials merged by a combine kernel), and keeps
the heads of one GQA group in one workgroup so shared rows are fetched once.
Indices must lie in [0, N); the kernel skips any that do not.
"""
from __future__ import annotations

import torch

from dcr_attention_amd import _lib

_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def fused_topk_attention(
    Q: torch.Tensor,            # [B, H, D]
    K_cache: torch.Tensor,      # [B, H_kv, N, D]
    V_cache: torch.Tensor,      # [B, H_kv, N, D]
    indices: torch.Tensor,      # [B, H, k_eff] int32
) -> torch.Tensor:              # [B, H, D], dtype of Q
    """Softmax attention of each query head over its selected K/V rows."""
    lib = _lib.load()
    _lib.require_device(Q, K_cache, V_cache, indices, what="Pass 3")

    B, H, D = Q.shape
    B_k, H_kv, N, D_k = K_cache.shape
    B_i, H_i, k_eff = indices.shape
    assert Q.dtype in _DTYPES, f"Q must be fp32/fp16/bf16, got {Q.dtype}"
    assert K_cache.dtype == Q.dtype, f"K_cache dtype {K_cache.dtype} != Q dtype {Q.dtype}"
    assert V_cache.dtype == Q.dtype, f"V_cache dtype {V_cache.dtype} != Q dtype {Q.dtype}"
    assert indices.dtype == torch.int32, f"indices must be int32, got {indices.dtype}"
    assert Q.is_contiguous()
    ldn = _lib.kv_head_stride(K_cache, V_cache)
    assert indices.is_contiguous()
    assert B == B_k == B_i and H == H_i and D == D_k
    assert H % H_kv == 0
    assert k_eff > 0

    O = torch.empty(B, H, D, dtype=Q.dtype, device=Q.device)
    ws_bytes = lib.dcr_gather_attn_workspace_bytes(B, H, H_kv, D, k_eff)
    ws = _lib.workspace(ws_bytes, Q.device)
    rc = lib.dcr_gather_attn(Q.data_ptr(), K_cache.data_ptr(), V_cache.data_ptr(),
                             _lib.DTYPE_CODE[Q.dtype], indices.data_ptr(), O.data_ptr(),
                             B, H, H_kv, N, ldn, D, k_eff, ws.data_ptr(), ws_bytes,
                             _lib.stream_of(Q))
    _lib.check(rc, "fused_topk_attention")
    return O
