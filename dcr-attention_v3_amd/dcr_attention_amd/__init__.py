"""dcr_attention_amd -- MI355X-native DCR-Attention sparse decode path.

Host side of the drop-in for the reference's Triton path
(Seqev/dcr-attention_v3, ``dcr_attention/kernel/triton/``): the same function
names and argument meaning, backed by hand-written gfx950 HIP kernels in
``libdcr_sparse_decode.so`` (C ABI: ``include/dcr_sparse_decode.h``).

    from dcr_attention_amd.kernel.hip.topk_axis import topk_qaxis_attention
    O = topk_qaxis_attention(Q, K_cache, V_cache, k_eff)

Sub-packages
------------
``kernel.hip``  topk_qaxis_select / topk_qaxis_attention / topk_pass1_projection /
                topk_pass2_select / fused_topk_attention / compute_u_Q /
                dense_decode_attention
``llama``       the caller side: config, routing, k_eff policy, DCR attention
                wrapper and a Llama-3.2-1B-shaped decoder for the decode loop
``synthetic``   seeded inputs for the benchmark configurations
"""

__version__ = "0.1.0"
