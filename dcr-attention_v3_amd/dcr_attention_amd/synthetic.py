"""Seeded synthetic decode-attention inputs for the benchmark configurations.

The reference ships no generator for attention sinks or outlier channels, so
this module defines one (the reference's tests draw plain ``torch.randn``;
tests/kernel/test_m3_fused_attn.py:204-206):

* One CPU ``torch.Generator`` seeded with ``seed``.  Draw order: Q [B,H,D],
  K [B,Hkv,N,D], V [B,Hkv,N,D], i.i.d. N(0,1) in fp32.
* Sinks: for each (b, g) let ``u = normalize(sum_{r<rep} Q[b, rep*g + r])``.
  For tokens n < n_sinks: ``a = K[b,g,n]·u``, ``K[b,g,n] += (sink_scale*max(|a|, 1) - a) u``,
  so the component of the key along the mean query direction is scaled by
  ``sink_scale`` and is at least ``sink_scale``: sinks rank at the top.
* Outliers: ``ch = randperm(D, generator)[:n_outlier]`` drawn after V;
  ``K[..., ch] *= outlier_scale``.
* Finally every tensor is cast to ``dtype`` (round-to-nearest-even).

``device="cuda"`` draws with a CUDA generator instead (same recipe, different
stream of numbers); that is what the benchmark uses for the large configs.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch


@dataclass(frozen=True)
class DecodeConfig:
    """One benchmark configuration (C1..C5) of the single-layer sparse decode op."""
    name: str
    B: int
    H: int
    Hkv: int
    N: int
    D: int
    dtype: torch.dtype
    c: float
    n_sinks: int = 4
    sink_scale: float = 8.0
    n_outlier: int = 0
    outlier_scale: float = 6.0

    @property
    def k(self) -> int:
        """Benchmark rule K = ceil(c*N)."""
        return k_ceil(self.N, self.c)

    @property
    def n_rep(self) -> int:
        return self.H // self.Hkv


def k_ceil(N: int, c: float) -> int:
    """K = ceil(c*N), computed exactly for decimal c (the benchmark configurations).

    ``c`` is interpreted as the decimal it prints as, so 0.15*4096 = 614.4
    gives 615 and 0.15*32768 = 4915.2 gives 4916.
    """
    from fractions import Fraction
    return int(math.ceil(Fraction(repr(c)) * N))


CONFIGS = {
    "C1": DecodeConfig("C1", B=1, H=32, Hkv=8, N=4096, D=64, dtype=torch.float32, c=0.15),
    "C2": DecodeConfig("C2", B=4, H=32, Hkv=8, N=32768, D=64, dtype=torch.float16, c=0.15,
                       n_outlier=2),
    "C4a": DecodeConfig("C4a", B=1, H=32, Hkv=8, N=131072, D=64, dtype=torch.float16, c=0.05,
                        n_outlier=2),
    "C4b": DecodeConfig("C4b", B=1, H=32, Hkv=8, N=131072, D=64, dtype=torch.float16, c=0.15,
                        n_outlier=2),
    "C4c": DecodeConfig("C4c", B=1, H=32, Hkv=8, N=131072, D=64, dtype=torch.float16, c=0.30,
                        n_outlier=2),
    "C5": DecodeConfig("C5", B=16, H=32, Hkv=8, N=65536, D=128, dtype=torch.bfloat16, c=0.10),
}


def make_inputs(cfg: DecodeConfig, seed: int = 0, device: str = "cpu",
                B: Optional[int] = None, N: Optional[int] = None):
    """Return (Q, K, V) for ``cfg`` (optionally overriding B or N)."""
    B = cfg.B if B is None else B
    N = cfg.N if N is None else N
    return make_qkv(B, cfg.H, cfg.Hkv, N, cfg.D, cfg.dtype, seed=seed, device=device,
                    n_sinks=cfg.n_sinks, sink_scale=cfg.sink_scale,
                    n_outlier=cfg.n_outlier, outlier_scale=cfg.outlier_scale)


def make_qkv(B: int, H: int, Hkv: int, N: int, D: int, dtype: torch.dtype, *, seed: int = 0,
             device: str = "cpu", n_sinks: int = 0, sink_scale: float = 8.0,
             n_outlier: int = 0, outlier_scale: float = 6.0):
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    Q = torch.randn(B, H, D, generator=gen, device=dev, dtype=torch.float32)
    K = torch.randn(B, Hkv, N, D, generator=gen, device=dev, dtype=torch.float32)
    V = torch.randn(B, Hkv, N, D, generator=gen, device=dev, dtype=torch.float32)
    rep = H // Hkv
    ns = min(n_sinks, N)
    if ns > 0:
        qm = Q.view(B, Hkv, rep, D).sum(dim=2)                      # [B, Hkv, D]
        u = qm / qm.norm(dim=-1, keepdim=True).clamp(min=1e-12)
        ks = K[:, :, :ns, :]                                         # [B, Hkv, ns, D]
        a = torch.einsum("bgnd,bgd->bgn", ks, u)
        ks += ((sink_scale * a.abs().clamp(min=1.0) - a).unsqueeze(-1)) * u.unsqueeze(2)
    if n_outlier > 0:
        ch = torch.randperm(D, generator=gen, device=dev)[:n_outlier]
        K[..., ch] *= outlier_scale
    return Q.to(dtype), K.to(dtype), V.to(dtype)
