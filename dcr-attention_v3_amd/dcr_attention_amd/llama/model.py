"""Llama-3.2-1B-shaped decoder whose decode-step attention runs the DCR path.

The reference wraps HuggingFace's ``LlamaAttention`` (monkey_patch.py:80-192,
attention.py:319-462): per layer it projects Q/K/V, applies RoPE, appends K/V
to a ``DynamicCache``, expands K/V with ``repeat_kv`` and routes the call to
dense attention or to the top-K kernels.  This module is the same decoder
built directly on the kernels of this package, MI355X-first:

* the KV cache is preallocated once, ``[B, H_kv, N_max, D]`` per layer (no
  per-step concatenation, no ``repeat_kv`` expansion); attention reads the
  first N rows of each head through a strided view (the kernels take the
  head stride), so a decode step copies nothing but the new token's K/V row;
* decode attention is routed per layer and step exactly like the reference
  (``route``, ``adaptive_k_window``, dense fallback when k_eff >= N_kv), with
  the reference's class-level branch counters;
* projections, norms, RoPE and the MLP are plain torch ops (hipBLASLt GEMMs),
  as in HuggingFace's eager Llama.

Weights are random (seeded) unless loaded from a HuggingFace-layout state
dict with ``load_hf_state_dict``; there is no network access for checkpoints.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from dcr_attention_amd.llama.attention import dcr_forward, sdpa_forward
from dcr_attention_amd.llama.config import DCRLlamaConfig
from dcr_attention_amd.llama.routing import Branch, route


@dataclass(frozen=True)
class LlamaDecoderConfig:
    """Architecture numbers (Llama-3.2-1B defaults)."""
    vocab_size: int = 128256
    hidden_size: int = 2048
    intermediate_size: int = 8192
    num_layers: int = 16
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 64
    rope_theta: float = 500000.0
    # llama3 RoPE scaling: (factor, low_freq_factor, high_freq_factor,
    # original_max_position_embeddings); None = plain RoPE.
    rope_scaling: Optional[Tuple[float, float, float, int]] = (32.0, 1.0, 4.0, 8192)
    rms_norm_eps: float = 1e-5
    tie_word_embeddings: bool = True

    @property
    def n_rep(self) -> int:
        return self.num_heads // self.num_kv_heads


LLAMA_3_2_1B = LlamaDecoderConfig()


def rope_inv_freq(cfg: LlamaDecoderConfig) -> torch.Tensor:
    """Per-pair inverse frequencies (fp32, [head_dim/2]), with the llama3
    long-context rescaling: wavelengths below orig/high_freq_factor are kept,
    those above orig/low_freq_factor are divided by `factor`, and the band in
    between is interpolated linearly in orig/wavelength."""
    D = cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    if cfg.rope_scaling is None:
        return inv.float()
    factor, low, high, orig = cfg.rope_scaling
    wavelen = 2 * math.pi / inv
    low_wl, high_wl = orig / low, orig / high
    smooth = (orig / wavelen - low) / (high - low)
    scaled = torch.where(wavelen > low_wl, inv / factor, inv)
    mid = (wavelen <= low_wl) & (wavelen >= high_wl)
    scaled = torch.where(mid, (1 - smooth) * inv / factor + smooth * inv, scaled)
    return scaled.float()


def rope_cos_sin(inv_freq: torch.Tensor, positions: torch.Tensor, dtype: torch.dtype):
    """cos/sin tables [T, head_dim] for integer positions [T] (fp32 math,
    halves duplicated as in the rotate-half convention), cast to dtype."""
    ang = positions.to(torch.float32)[:, None] * inv_freq.to(positions.device)[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, H, T, D]; cos/sin [T, D]: x*cos + rotate_half(x)*sin."""
    h = x.shape[-1] // 2
    rot = torch.cat([-x[..., h:], x[..., :h]], dim=-1)
    return x * cos + rot * sin


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Llama RMSNorm: normalise in fp32, cast back, scale."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(x.dtype)


@dataclass
class KVCache:
    """Preallocated per-layer cache [B, H_kv, N_max, D] (K and V) and the
    number of valid positions."""
    k: List[torch.Tensor]
    v: List[torch.Tensor]
    length: int = 0

    @classmethod
    def allocate(cls, cfg: LlamaDecoderConfig, B: int, n_max: int, dtype: torch.dtype,
                 device) -> "KVCache":
        shape = (B, cfg.num_kv_heads, n_max, cfg.head_dim)
        return cls([torch.zeros(shape, dtype=dtype, device=device) for _ in range(cfg.num_layers)],
                   [torch.zeros(shape, dtype=dtype, device=device) for _ in range(cfg.num_layers)])

    @property
    def capacity(self) -> int:
        return self.k[0].shape[2]

    def fill_synthetic(self, n: int, seed: int = 0, scale: float = 1.0) -> None:
        """Fill the first n positions of every layer with seeded N(0, scale^2)
        values (the reference's long-context runtime tests fill the cache the
        same way instead of running a 32K-token prefill)."""
        assert n <= self.capacity
        g = torch.Generator(device=self.k[0].device).manual_seed(seed)
        for kk, vv in zip(self.k, self.v):
            kk[:, :, :n].normal_(0.0, scale, generator=g)
            vv[:, :, :n].normal_(0.0, scale, generator=g)
        self.length = n


class DCRLlamaDecoder:
    """Decoder stack with reference-style routing of every attention call.

    Class-level counters mirror the reference's ``_dcr_invocations`` /
    ``_sdpa_invocations`` (attention.py:93-119)."""

    _dcr_invocations: int = 0
    _sdpa_invocations: int = 0

    @classmethod
    def reset_counters(cls) -> None:
        cls._dcr_invocations = 0
        cls._sdpa_invocations = 0

    @classmethod
    def get_counters(cls) -> Dict[str, int]:
        return {"dcr": cls._dcr_invocations, "sdpa": cls._sdpa_invocations}

    def __init__(self, cfg: LlamaDecoderConfig = LLAMA_3_2_1B,
                 dcr: Optional[DCRLlamaConfig] = None, *, dtype=torch.float16, device="cuda"):
        self.cfg = cfg
        self.dcr = dcr if dcr is not None else DCRLlamaConfig()
        self.dtype = dtype
        self.device = torch.device(device)
        self.inv_freq = rope_inv_freq(cfg).to(self.device)
        self.w: Dict[str, torch.Tensor] = {}
        self.eager_attention = False  # True: decode attention as the reference's eager SDPA

    # ------------------------------------------------------------ weights
    def _shapes(self) -> Dict[str, Tuple[int, ...]]:
        c = self.cfg
        hd, H, Hk, I = c.hidden_size, c.num_heads, c.num_kv_heads, c.intermediate_size
        s = {"embed": (c.vocab_size, hd), "norm": (hd,)}
        for l in range(c.num_layers):
            s.update({f"{l}.q": (H * c.head_dim, hd), f"{l}.k": (Hk * c.head_dim, hd),
                      f"{l}.v": (Hk * c.head_dim, hd), f"{l}.o": (hd, H * c.head_dim),
                      f"{l}.gate": (I, hd), f"{l}.up": (I, hd), f"{l}.down": (hd, I),
                      f"{l}.ln1": (hd,), f"{l}.ln2": (hd,)})
        if not c.tie_word_embeddings:
            s["lm_head"] = (c.vocab_size, hd)
        return s

    def init_random(self, seed: int = 0, std: float = 0.02) -> "DCRLlamaDecoder":
        """Seeded random weights (N(0, std^2) matrices, unit norm weights)."""
        g = torch.Generator(device=self.device).manual_seed(seed)
        for name, shape in self._shapes().items():
            if len(shape) == 1:
                self.w[name] = torch.ones(shape, dtype=self.dtype, device=self.device)
            else:
                t = torch.empty(shape, dtype=torch.float32, device=self.device)
                t.normal_(0.0, std, generator=g)
                self.w[name] = t.to(self.dtype)
        return self

    def load_hf_state_dict(self, sd: Dict[str, torch.Tensor]) -> "DCRLlamaDecoder":
        """Weights from a HuggingFace ``LlamaForCausalLM.state_dict()``."""
        m = {"embed": "model.embed_tokens.weight", "norm": "model.norm.weight"}
        for l in range(self.cfg.num_layers):
            p = f"model.layers.{l}."
            m.update({f"{l}.q": p + "self_attn.q_proj.weight", f"{l}.k": p + "self_attn.k_proj.weight",
                      f"{l}.v": p + "self_attn.v_proj.weight", f"{l}.o": p + "self_attn.o_proj.weight",
                      f"{l}.gate": p + "mlp.gate_proj.weight", f"{l}.up": p + "mlp.up_proj.weight",
                      f"{l}.down": p + "mlp.down_proj.weight",
                      f"{l}.ln1": p + "input_layernorm.weight",
                      f"{l}.ln2": p + "post_attention_layernorm.weight"})
        if not self.cfg.tie_word_embeddings:
            m["lm_head"] = "lm_head.weight"
        for name, key in m.items():
            self.w[name] = sd[key].to(device=self.device, dtype=self.dtype).contiguous()
        return self

    # ------------------------------------------------------------ forward
    def _attention(self, l: int, q: torch.Tensor, cache: KVCache, n_kv: int) -> torch.Tensor:
        """q [B, H, T, D] (post-RoPE); cache rows [0, n_kv) valid."""
        c = self.cfg
        K = cache.k[l][:, :, :n_kv]
        V = cache.v[l][:, :, :n_kv]
        T = q.shape[2]
        branch = route(N_q=T, N_kv=n_kv, layer_idx=l, cfg=self.dcr)
        if branch is Branch.DCR and not self.eager_attention:
            type(self)._dcr_invocations += 1
            return dcr_forward(q, K, V, self.dcr, n_rep=c.n_rep, kv_repeated=False)
        type(self)._sdpa_invocations += 1
        if self.eager_attention or T > 1:
            return eager_sdpa(q, K, V, c.n_rep)
        return sdpa_forward(q, K, V, None, T, n_kv, n_rep=c.n_rep, kv_repeated=False)

    @torch.no_grad()
    def forward(self, tokens: torch.Tensor, cache: KVCache) -> torch.Tensor:
        """tokens [B, T] at positions cache.length .. cache.length+T-1;
        appends their K/V to the cache and returns logits [B, T, vocab] (fp32)."""
        c = self.cfg
        B, T = tokens.shape
        p0 = cache.length
        assert p0 + T <= cache.capacity, "KV cache capacity exceeded"
        pos = torch.arange(p0, p0 + T, device=self.device)
        cos, sin = rope_cos_sin(self.inv_freq, pos, self.dtype)
        x = F.embedding(tokens.to(self.device), self.w["embed"])
        for l in range(c.num_layers):
            h = rms_norm(x, self.w[f"{l}.ln1"], c.rms_norm_eps)
            q = F.linear(h, self.w[f"{l}.q"]).view(B, T, c.num_heads, c.head_dim).transpose(1, 2)
            k = F.linear(h, self.w[f"{l}.k"]).view(B, T, c.num_kv_heads, c.head_dim).transpose(1, 2)
            v = F.linear(h, self.w[f"{l}.v"]).view(B, T, c.num_kv_heads, c.head_dim).transpose(1, 2)
            q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
            cache.k[l][:, :, p0:p0 + T] = k
            cache.v[l][:, :, p0:p0 + T] = v
            a = self._attention(l, q, cache, p0 + T)                     # [B, H, T, D]
            a = a.transpose(1, 2).reshape(B, T, c.num_heads * c.head_dim)
            x = x + F.linear(a, self.w[f"{l}.o"])
            h = rms_norm(x, self.w[f"{l}.ln2"], c.rms_norm_eps)
            x = x + F.linear(F.silu(F.linear(h, self.w[f"{l}.gate"])) * F.linear(h, self.w[f"{l}.up"]),
                             self.w[f"{l}.down"])
        cache.length = p0 + T
        x = rms_norm(x, self.w["norm"], c.rms_norm_eps)
        head = self.w["embed"] if c.tie_word_embeddings else self.w["lm_head"]
        return F.linear(x, head).float()

    def decode_step(self, tokens: torch.Tensor, cache: KVCache) -> torch.Tensor:
        """One token per sequence: tokens [B] -> greedy next tokens [B]."""
        return self.forward(tokens.view(-1, 1), cache)[:, -1].argmax(-1)


def eager_sdpa(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, n_rep: int) -> torch.Tensor:
    """The reference's dense branch as written (attention.py:673-739):
    repeat_kv, Q K^T / sqrt(D) (+ causal mask for T > 1), softmax in fp32,
    cast back, times V.  The product is formed as K @ q^T so that no batched
    product takes a transposed right operand."""
    B, H, T, D = q.shape
    Kr = K.repeat_interleave(n_rep, dim=1)                       # repeat_kv
    Vr = V.repeat_interleave(n_rep, dim=1)
    n_kv = Kr.shape[2]
    w = torch.matmul(Kr, q.transpose(-2, -1).contiguous()).transpose(-2, -1) / math.sqrt(D)
    if T > 1:
        causal = torch.triu(torch.full((T, n_kv), torch.finfo(w.dtype).min, dtype=w.dtype,
                                       device=w.device), diagonal=n_kv - T + 1)
        w = w + causal
    w = F.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(w.contiguous(), Vr)
