"""HuggingFace Llama attention with the reference's routing onto the HIP path.

``DCRLlamaAttention`` stands in for a ``transformers`` ``LlamaAttention`` module
(the reference's wrapper: dcr_attention/models/llama/attention.py:54-462).  It
is built around an existing HF attention module and keeps that module's
q/k/v/o projection modules by reference, so patching a loaded model copies no
parameter.  Per call:

  1. q/k/v projections, RoPE from the ``position_embeddings`` HF's model
     computes (HF's own ``apply_rotary_pos_emb``), and the HF cache update
     (``past_key_values.update``), which returns the layer's whole cache of
     un-repeated heads, ``[B, H_kv, N_kv, D]``;
  2. ``route`` (the reference's decision order, routing.py:28-69) picks the
     branch from (N_q, N_kv, layer, config); class-level counters record it
     (attention.py:93-119);
  3. the DCR branch runs ``dcr_forward`` -- k_eff from ``adaptive_k_window``,
     then ``topk_qaxis_attention`` (the HIP score / select / attention
     sequence) -- and the dense branch ``sdpa_forward`` (decode: the HIP dense
     decode kernel; prefill: fp32-softmax eager attention with the causal
     mask, as the reference's _sdpa_forward);
  4. the o projection; returns ``(attn_output, None)`` (HF 5.x unpacks two
     values; 4.x three, the third being the cache).

Where this differs from the reference, on purpose: the reference expands K/V
with ``repeat_kv`` before routing and its top-K branch undoes it with
``K[:, ::n_rep].contiguous()`` plus a cast to bf16 -- up to four full-cache
copies per layer-step (attention.py:425-426, 808-811).  Here both branches
take the cache as HF keeps it (un-repeated heads, its own dtype): the HIP
kernels read GQA groups and strided or preallocated caches in place.

A cache whose ``update`` returns a preallocated buffer longer than the valid
length (HF's ``StaticCache``) is cut to ``cache_position[-1] + 1`` rows (a
view; the kernels take the buffer's row stride).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from dcr_attention_amd.llama.attention import dcr_forward, sdpa_forward
from dcr_attention_amd.llama.config import DCRLlamaConfig
from dcr_attention_amd.llama.routing import Branch, route

try:
    import transformers as _hf
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb as _hf_rope
    _HF_MAJOR = int(_hf.__version__.split(".")[0])
except ImportError:  # transformers absent: the wrapper is unusable, the rest of the package is not
    _hf_rope = None
    _HF_MAJOR = 5


def _rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    if _hf_rope is None:
        raise RuntimeError("DCRLlamaAttention needs transformers for its rotary embedding")
    return _hf_rope(q, k, cos, sin)


def _shape_attr(base: nn.Module, names, config_names, default=None):
    """An int shape parameter of an HF attention module: an attribute of the
    module (transformers 4.x keeps num_heads there), else of its config
    (5.x keeps only head_dim on the module)."""
    for n in names:
        v = getattr(base, n, None)
        if v is not None:
            return int(v)
    cfg = getattr(base, "config", None)
    for n in config_names:
        v = getattr(cfg, n, None) if cfg is not None else None
        if v is not None:
            return int(v)
    return default


class DCRLlamaAttention(nn.Module):
    """Routing wrapper around one HF Llama attention module (see the module
    docstring).  ``cfg`` may be replaced at any time (``reconfigure_dcr``)."""

    _dcr_invocations: int = 0
    _sdpa_invocations: int = 0

    @classmethod
    def reset_counters(cls) -> None:
        cls._dcr_invocations = 0
        cls._sdpa_invocations = 0

    @classmethod
    def get_counters(cls) -> dict:
        return {"dcr": cls._dcr_invocations, "sdpa": cls._sdpa_invocations}

    def __init__(self, base_layer: nn.Module, cfg: Optional[DCRLlamaConfig] = None) -> None:
        super().__init__()
        self.cfg = cfg if cfg is not None else DCRLlamaConfig()
        # The original module is kept (unpatch restores it) but not registered
        # as a submodule, so the patched model's parameters are not listed twice.
        object.__setattr__(self, "_base_layer", base_layer)
        self.q_proj = base_layer.q_proj
        self.k_proj = base_layer.k_proj
        self.v_proj = base_layer.v_proj
        self.o_proj = base_layer.o_proj
        self.num_heads = _shape_attr(base_layer, ("num_heads", "num_attention_heads"),
                                     ("num_attention_heads", "num_heads"))
        self.head_dim = _shape_attr(base_layer, ("head_dim",), ("head_dim",))
        if self.head_dim is None and self.num_heads:
            hidden = _shape_attr(base_layer, ("hidden_size",), ("hidden_size",))
            self.head_dim = hidden // self.num_heads if hidden else None
        self.num_key_value_heads = _shape_attr(base_layer, ("num_key_value_heads",),
                                               ("num_key_value_heads",), default=self.num_heads)
        if self.num_heads is None or self.head_dim is None:
            raise ValueError(
                f"DCRLlamaAttention: {type(base_layer).__name__} exposes no head count or head_dim "
                "(looked for num_heads / num_attention_heads and head_dim on the module and on its "
                "config)")
        if self.num_key_value_heads <= 0 or self.num_heads % self.num_key_value_heads != 0:
            raise ValueError(f"num_heads ({self.num_heads}) must be divisible by "
                             f"num_key_value_heads ({self.num_key_value_heads})")
        self.n_rep = self.num_heads // self.num_key_value_heads
        idx = getattr(base_layer, "layer_idx", None)
        self.layer_idx = 0 if idx is None else int(idx)

    @property
    def base_layer(self) -> nn.Module:
        return self._base_layer

    def extra_repr(self) -> str:
        return (f"layer_idx={self.layer_idx}, heads={self.num_heads}/{self.num_key_value_heads}, "
                f"head_dim={self.head_dim}, axis_source={self.cfg.axis_source!r}, "
                f"enable_dcr={self.cfg.enable_dcr}, T_dispatch={self.cfg.T_dispatch}, "
                f"coverage_floor={self.cfg.coverage_floor}")

    def forward(self, hidden_states: torch.Tensor,
                position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                attention_mask: Optional[torch.Tensor] = None,
                past_key_values=None, output_attentions: bool = False,
                cache_position: Optional[torch.Tensor] = None, **kwargs):
        if output_attentions:
            raise NotImplementedError("DCRLlamaAttention does not return attention weights "
                                      "(output_attentions=True); unpatch the layer to get them")
        if past_key_values is None:                       # transformers 4.x spelling
            past_key_values = kwargs.pop("past_key_value", None)
        B, T, _ = hidden_states.shape
        q = self.q_proj(hidden_states).view(B, T, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(hidden_states).view(B, T, self.num_key_value_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(B, T, self.num_key_value_heads, self.head_dim).transpose(1, 2)
        if position_embeddings is None:
            raise ValueError("DCRLlamaAttention needs position_embeddings (cos, sin) from the model")
        cos, sin = position_embeddings
        q, k = _rope(q, k, cos, sin)
        if past_key_values is not None:
            extra = {"cache_position": cache_position} if cache_position is not None else {}
            k, v = past_key_values.update(k, v, self.layer_idx, extra) if _HF_MAJOR < 5 else \
                past_key_values.update(k, v, self.layer_idx, **extra)
            if cache_position is not None and k.shape[-2] > T:
                n_valid = int(cache_position[-1]) + 1
                if n_valid < k.shape[-2]:                 # preallocated (static) cache
                    k, v = k[:, :, :n_valid], v[:, :, :n_valid]
        n_kv = k.shape[-2]

        branch = route(N_q=T, N_kv=n_kv, layer_idx=self.layer_idx, cfg=self.cfg)
        if branch is Branch.DCR:
            type(self)._dcr_invocations += 1
            out = self._dcr_branch(q, k, v)
        else:
            type(self)._sdpa_invocations += 1
            out = self._dense_branch(q, k, v, attention_mask, T, n_kv)
        out = self.o_proj(out.transpose(1, 2).reshape(B, T, self.num_heads * self.head_dim))
        if _HF_MAJOR < 5:
            return out, None, past_key_values
        return out, None

    # The two branches (separate methods so that a checker can replace one).
    def _dcr_branch(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        return dcr_forward(q, k, v, self.cfg, n_rep=self.n_rep, kv_repeated=False)

    def _dense_branch(self, q, k, v, attention_mask, n_q: int, n_kv: int) -> torch.Tensor:
        if attention_mask is not None and attention_mask.dtype == torch.bool:
            # HF's sdpa-style boolean masks (True = attend) as the additive form
            # the eager branch takes
            attention_mask = torch.zeros(attention_mask.shape, dtype=q.dtype, device=q.device) \
                .masked_fill(~attention_mask, torch.finfo(q.dtype).min)
        return sdpa_forward(q, k, v, attention_mask, n_q, n_kv, n_rep=self.n_rep, kv_repeated=False)
