"""Decode-attention caller glue: the DCR branch and its dense fallback.

``dcr_forward`` is the top-K branch of the reference caller's
``_dcr_forward`` (dcr_attention/models/llama/attention.py:741-813):

  1. k_eff = adaptive_k_window(cfg.k_window, N_kv, cfg.coverage_floor)
     (attention.py:781-785);
  2. k_eff >= N_kv -> dense attention over the whole cache (attention.py:806-807);
  3. otherwise the sparse decode op on the un-repeated cache
     (attention.py:808-812).

Differences, all on purpose:
  * the reference un-repeats a GQA-repeated cache with
    ``K[:, ::n_rep].contiguous()`` -- two full-cache copies per layer-step
    (C2: 2 x 134 MB).  Here ``K[:, ::n_rep]`` is passed as a strided view
    (the kernels take the head stride), and a caller that keeps its cache
    un-repeated passes it directly (``kv_repeated=False``);
  * the reference casts Q/K/V to bf16 because its kernels are bf16-only; the
    HIP kernels take fp32, fp16 or bf16, so the cache dtype is kept.

The reference's rank-local axis sources (attention.py:816-880) run
``rank_local_attention`` over the k_eff keys around the query's rank along an
ordering axis: ``"q"`` uses the query's own direction Q/||Q|| (fp32);
``"pca"`` and ``"positional"`` use the principal direction of each head's
keys (the reference computes both with compute_axis and no positional
embedding, i.e. PCA; here ``kernel.axis.pca_axes``, one batch on the device
instead of a host SVD per head).  With ``enable_adaptive_widening`` a leaky
window (``detect_leaky_boundary``) is retried once at ``widen_factor(k_eff)``.

``sdpa_forward`` is the dense branch (``_sdpa_forward``, attention.py:673-739:
fp32 softmax of Q K^T / sqrt(D), then V).  Decode (N_q == 1) runs the HIP
dense decode kernel on the un-repeated cache; prefill (N_q > 1) runs the
same eager torch math as the reference, with the causal mask.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F

from dcr_attention_amd.kernel.hip.dense import dense_decode_attention
from dcr_attention_amd.kernel.hip.topk_axis import topk_qaxis_attention
from dcr_attention_amd.kernel.axis import pca_axes
from dcr_attention_amd.kernel.rank_local_attention import rank_local_attention
from dcr_attention_amd.llama.adaptive import adaptive_k_window, detect_leaky_boundary, widen_factor
from dcr_attention_amd.llama.config import DCRLlamaConfig


def _unrepeat(K: torch.Tensor, n_rep: int, kv_repeated: bool) -> torch.Tensor:
    return K[:, ::n_rep] if (kv_repeated and n_rep > 1) else K


def sdpa_forward(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor,
                 attention_mask: Optional[torch.Tensor], N_q: int, N_kv: int, *,
                 n_rep: int = 1, kv_repeated: bool = True) -> torch.Tensor:
    """Dense attention.  Q [B, H, N_q, D]; K/V [B, H, N_kv, D] when
    ``kv_repeated`` else [B, H_kv, N_kv, D].  Returns [B, H, N_q, D]."""
    if N_q == 1 and attention_mask is None:
        Kk, Vv = _unrepeat(K, n_rep, kv_repeated), _unrepeat(V, n_rep, kv_repeated)
        return dense_decode_attention(Q.squeeze(-2).contiguous(), Kk, Vv).unsqueeze(-2)
    if not kv_repeated and n_rep > 1:
        K = K.repeat_interleave(n_rep, dim=1)
        V = V.repeat_interleave(n_rep, dim=1)
    D = Q.shape[-1]
    # K^T is materialised: batched products with a transposed right operand
    # are avoided on this platform.
    w = torch.matmul(Q, K.transpose(-2, -1).contiguous()) / math.sqrt(D)
    if attention_mask is not None:
        w = w + attention_mask[:, :, :, :N_kv]
    elif N_q > 1:
        causal = torch.triu(torch.full((N_q, N_kv), torch.finfo(w.dtype).min, dtype=w.dtype,
                                       device=w.device), diagonal=N_kv - N_q + 1)
        w = w + causal
    w = F.softmax(w, dim=-1, dtype=torch.float32).to(Q.dtype)
    return torch.matmul(w, V.contiguous())


def dcr_forward(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, cfg: DCRLlamaConfig, *,
                n_rep: int, kv_repeated: bool = True) -> torch.Tensor:
    """DCR branch for one decode step.  Q [B, H, 1, D]; K/V as in
    ``sdpa_forward``.  Returns [B, H, 1, D] in Q's dtype."""
    N_kv = K.shape[2]
    if cfg.axis_source in ("q", "pca", "positional"):
        return _rank_local_forward(Q, K, V, cfg, n_rep=n_rep, kv_repeated=kv_repeated)
    if not cfg.uses_topk_hip:
        raise NotImplementedError(
            f"axis_source={cfg.axis_source!r} is not built for MI355X; use 'q_topk_hip' "
            "(or its alias 'q_topk_triton'), or a rank-local axis ('q', 'pca', 'positional')")
    k_eff = adaptive_k_window(cfg.k_window, N_kv, cfg.coverage_floor)
    if k_eff >= N_kv:
        return sdpa_forward(Q, K, V, None, 1, N_kv, n_rep=n_rep, kv_repeated=kv_repeated)
    Kk, Vv = _unrepeat(K, n_rep, kv_repeated), _unrepeat(V, n_rep, kv_repeated)
    O = topk_qaxis_attention(Q.squeeze(-2).contiguous(), Kk, Vv, k_eff)
    return O.unsqueeze(-2)


def rank_local_axes(Q: torch.Tensor, K_unrepeated: torch.Tensor, axis_source: str) -> torch.Tensor:
    """Per-(b, h) ordering axes [B, H, D] fp32 of the rank-local branch
    (attention.py:816-843): the query's direction for "q" decode, else the
    principal direction of the head's keys."""
    B, H = Q.shape[0], Q.shape[1]
    if axis_source == "q" and Q.shape[2] == 1:
        q = Q.squeeze(-2).float()
        return q / q.norm(dim=-1, keepdim=True).clamp(min=1e-12)
    a = pca_axes(K_unrepeated)                                          # [B, H_kv, D]
    return a.repeat_interleave(H // K_unrepeated.shape[1], dim=1)


def _rank_local_forward(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, cfg: DCRLlamaConfig, *,
                        n_rep: int, kv_repeated: bool) -> torch.Tensor:
    """Rank-local decode along the configured axis (attention.py:816-880)."""
    N_kv = K.shape[2]
    k_eff = adaptive_k_window(cfg.k_window, N_kv, cfg.coverage_floor)
    Kk, Vv = _unrepeat(K, n_rep, kv_repeated), _unrepeat(V, n_rep, kv_repeated)
    axes = rank_local_axes(Q, Kk, cfg.axis_source)
    out = rank_local_attention(Q, Kk, Vv, axes, k_window=k_eff)
    if cfg.enable_adaptive_widening and k_eff < N_kv and Q.shape[2] == 1:
        B, H, D = axes.shape
        q = Q.squeeze(-2).float()
        q_proj = (q * axes).sum(dim=-1, keepdim=True)                   # [B, H, 1]
        Hkv = Kk.shape[1]
        a5 = axes.reshape(B, Hkv, H // Hkv, D, 1).contiguous()
        k_proj = torch.matmul(Kk.float().unsqueeze(2), a5).reshape(B, H, N_kv)
        leaky = detect_leaky_boundary(q_proj, k_proj, torch.argsort(k_proj, dim=-1), k_eff, slack=0.5)
        if bool(leaky.any()):
            k2 = widen_factor(k_eff, N_kv)
            if k2 > k_eff:
                out = rank_local_attention(Q, Kk, Vv, axes, k_window=k2)
    return out
