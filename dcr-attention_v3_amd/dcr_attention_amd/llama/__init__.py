"""Llama decode caller of the sparse decode path: configuration, k_eff policy,
routing and the attention-branch glue (reference dcr_attention/models/llama/)."""
from dcr_attention_amd.llama.adaptive import adaptive_k_window
from dcr_attention_amd.llama.config import DCRLlamaConfig, DEFAULT_DCR_LLAMA_CONFIG
from dcr_attention_amd.llama.routing import Branch, explain_route, route

__all__ = ["adaptive_k_window", "DCRLlamaConfig", "DEFAULT_DCR_LLAMA_CONFIG", "Branch",
           "explain_route", "route"]
