"""Patch a HuggingFace Llama model so that its attention runs the DCR routing.

The reference's plugin API (dcr_attention/models/llama/monkey_patch.py:80-206),
same names, arguments, return values and errors:

    model = transformers.LlamaForCausalLM(config)          # or from_pretrained
    patch_llama_with_dcr(model, DCRLlamaConfig())          # -> layers replaced
    model.generate(...)        # decode steps route to the HIP sparse path
    reconfigure_dcr(model, DCRLlamaConfig(enable_dcr=False))
    unpatch_llama(model)                                   # -> layers restored

* Each ``layer.self_attn`` (HF ``LlamaAttention`` or a subclass) of
  ``model.model.layers`` (causal LM) or ``model.layers`` (bare model) becomes a
  ``DCRLlamaAttention`` holding the original's projection modules by
  reference: no parameter is copied and the model's parameter count is
  unchanged.
* The originals are kept in a dict on the model (attribute
  ``_dcr_patch_registry``, layer index -> module) for ``unpatch_llama``.
* Patching twice replaces nothing the second time and warns; layers outside
  ``cfg.layer_filter`` are left as they are.
"""
from __future__ import annotations

import warnings
from typing import Iterator, List, Optional, Tuple

import torch.nn as nn

from dcr_attention_amd.llama.config import DCRLlamaConfig
from dcr_attention_amd.llama.hf_attention import DCRLlamaAttention

_REGISTRY = "_dcr_patch_registry"


def _decoder_layers(model: nn.Module) -> Iterator[Tuple[int, nn.Module]]:
    """(index, decoder layer) of a Llama-family model; ValueError if the model
    has no ``model.layers`` / ``layers`` list or a layer has no ``self_attn``."""
    inner = getattr(model, "model", None)
    if inner is not None and hasattr(inner, "layers"):
        layers = inner.layers
    elif hasattr(model, "layers"):
        layers = model.layers
    else:
        raise ValueError(f"Cannot find transformer layers on {type(model).__name__}: expected "
                         "`model.model.layers` (causal LM) or `model.layers` (bare model)")
    for i, layer in enumerate(layers):
        if not hasattr(layer, "self_attn"):
            raise ValueError(f"layer {i} ({type(layer).__name__}) has no `self_attn` attribute; "
                             "not a Llama-family decoder layer")
        yield i, layer


def patch_llama_with_dcr(model: nn.Module, cfg: Optional[DCRLlamaConfig] = None) -> int:
    """Wrap every attention module of ``model`` (in place) in a
    ``DCRLlamaAttention`` sharing ``cfg``; returns the number of layers newly
    replaced (layers skipped by ``cfg.layer_filter`` or already wrapped are
    not counted)."""
    cfg = cfg if cfg is not None else DCRLlamaConfig()
    layers = list(_decoder_layers(model))
    registry = getattr(model, _REGISTRY, None)
    if registry is None:
        registry = {}
        setattr(model, _REGISTRY, registry)
    replaced = already = 0
    for i, layer in layers:
        if cfg.layer_filter is not None and i not in cfg.layer_filter:
            continue
        if isinstance(layer.self_attn, DCRLlamaAttention):
            already += 1
            continue
        original = layer.self_attn
        if getattr(original, "layer_idx", None) is None:
            original.layer_idx = i
        registry[i] = original
        layer.self_attn = DCRLlamaAttention(original, cfg)
        replaced += 1
    if already:
        warnings.warn(f"patch_llama_with_dcr: {already} layer(s) were already patched and were "
                      f"skipped; {replaced} newly replaced", UserWarning, stacklevel=2)
    return replaced


def unpatch_llama(model: nn.Module) -> int:
    """Put the original attention modules back; returns how many were
    restored (0 for a model that was never patched)."""
    registry = getattr(model, _REGISTRY, None)
    if registry is None:
        return 0
    restored = 0
    for i, layer in _decoder_layers(model):
        if i in registry and isinstance(layer.self_attn, DCRLlamaAttention):
            layer.self_attn = registry[i]
            restored += 1
    delattr(model, _REGISTRY)
    return restored


def reconfigure_dcr(model: nn.Module, cfg: DCRLlamaConfig) -> int:
    """Give every wrapped layer the configuration ``cfg`` without re-wrapping;
    returns the number of layers updated."""
    n = 0
    for _, layer in _decoder_layers(model):
        if isinstance(layer.self_attn, DCRLlamaAttention):
            layer.self_attn.cfg = cfg
            n += 1
    return n


def patched_layer_indices(model: nn.Module) -> List[int]:
    """Indices of the layers whose attention is currently wrapped ([] for a
    model without a Llama layout)."""
    try:
        return [i for i, layer in _decoder_layers(model) if isinstance(layer.self_attn, DCRLlamaAttention)]
    except ValueError:
        return []


def is_patched(model: nn.Module) -> bool:
    """True when some layer of ``model`` runs through ``DCRLlamaAttention``."""
    return bool(patched_layer_indices(model))
