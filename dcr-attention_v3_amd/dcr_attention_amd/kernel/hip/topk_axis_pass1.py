"""Pass 1 -- projection (score) pass on MI355X.

Drop-in for ``topk_pass1_projection`` (reference
dcr_attention/kernel/triton/topk_axis_pass1.py:104-153).  Same arguments,
same output; the reference's bf16-only and ``n_per_kv == 4`` restrictions
(:123-130) are lifted to fp32/fp16/bf16 keys, n_rep in {1, 2, 4, 8} and
D in {64, 128}, and K_cache may be a strided view whose rows are contiguous
(a slice of a preallocated cache, or ``K[:, ::n_rep]`` of a repeated cache).

Numerics: ``scores[b, h, n] = bf16_rne(sum_d fp32(K[b, h // n_rep, n, d]) * u_Q[b, h, d])``
with the sum evaluated as a sequential fp32 FMA chain over d (bit-identical to
the reference M1's CPU einsum, qaxis_topk_reference.py:85).
"""
from __future__ import annotations

import torch

from dcr_attention_amd import _lib

_KEY_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def topk_pass1_projection(
    K_cache: torch.Tensor,   # [B, H_kv, N, D]
    u_Q: torch.Tensor,       # [B, H, D] fp32
) -> torch.Tensor:           # [B, H, N] bf16
    """Project every cached key onto the unit query of each head of its GQA group."""
    lib = _lib.load()
    _lib.require_device(K_cache, u_Q, what="Pass 1")

    B, H_kv, N, D = K_cache.shape
    H = u_Q.shape[1]
    assert K_cache.dtype in _KEY_DTYPES, f"K_cache must be fp32/fp16/bf16, got {K_cache.dtype}"
    assert u_Q.dtype == torch.float32, f"u_Q must be fp32, got {u_Q.dtype}"
    ldn = _lib.kv_head_stride(K_cache)
    assert u_Q.is_contiguous(), "u_Q must be contiguous"
    assert u_Q.shape == (B, H, D), f"u_Q shape {tuple(u_Q.shape)} != {(B, H, D)}"
    assert H % H_kv == 0, f"H={H} must be divisible by H_kv={H_kv}"

    scores = torch.empty(B, H, N, dtype=torch.bfloat16, device=K_cache.device)
    rc = lib.dcr_score_pass(K_cache.data_ptr(), _lib.DTYPE_CODE[K_cache.dtype], u_Q.data_ptr(),
                            scores.data_ptr(), B, H_kv, H // H_kv, N, ldn, D,
                            _lib.stream_of(K_cache))
    _lib.check(rc, "topk_pass1_projection")
    return scores
