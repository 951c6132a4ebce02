"""HIP (gfx950) implementation of the reference's Triton top-K Q-axis path.

Module names mirror ``dcr_attention/kernel/triton/`` so that a caller swaps
``dcr_attention.kernel.triton`` for ``dcr_attention_amd.kernel.hip``.
"""
from dcr_attention_amd.kernel.hip.dense import dense_decode_attention
from dcr_attention_amd.kernel.hip.fused_attn import fused_topk_attention
from dcr_attention_amd.kernel.hip.topk_axis import (compute_u_Q, topk_qaxis_attention,
                                                     topk_qaxis_select)
from dcr_attention_amd.kernel.hip.topk_axis_pass1 import topk_pass1_projection
from dcr_attention_amd.kernel.hip.topk_axis_pass2 import topk_pass2_select

__all__ = [
    "compute_u_Q",
    "dense_decode_attention",
    "fused_topk_attention",
    "topk_pass1_projection",
    "topk_pass2_select",
    "topk_qaxis_attention",
    "topk_qaxis_select",
]
