"""Ordering axes for rank-local attention.

``compute_axis`` mirrors the reference's axis resolution
(dcr_attention/dispatcher/stage_b.py:41-100): with an additive positional
embedding P [N, D], the least-squares direction u minimising
||(P - mean P) u - (j - (N-1)/2)||; otherwise the first principal direction of
the rows X [N, D] (the first right singular vector of X - mean X), unit norm.

``pca_axes`` gives the principal direction of every head of a cache
[B, H, N, D] in one batch: the centred covariance C = Xc^T Xc is formed on the
device in fp32 (the N x D x D work), and its top eigenvector is taken from a
float64 ``eigh`` of the small D x D matrices on the host -- the same direction
as the reference's per-head CPU SVD (attention.py:833-843 copies the whole cache
to the host for it), without moving the cache.

A principal direction is defined up to sign; the reference compares axes
sign-agnostically (test_stage_b.py:13-17).  Both functions here fix the sign:
the component of largest magnitude is positive.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

_EPS = 1e-12


def _fix_sign(u: torch.Tensor) -> torch.Tensor:
    """u with its largest-magnitude component made positive (last dim)."""
    i = u.abs().argmax(dim=-1, keepdim=True)
    s = torch.sign(torch.gather(u, -1, i))
    return u * torch.where(s == 0, torch.ones_like(s), s)


def _axis_from_positional(pe: torch.Tensor) -> torch.Tensor:
    N = pe.shape[0]
    pc = pe - pe.mean(dim=0)
    j = torch.arange(N, dtype=pe.dtype, device=pe.device) - (N - 1) / 2.0
    u = torch.linalg.lstsq(pc, j.unsqueeze(1)).solution.squeeze(-1)
    return u / (u.norm() + _EPS)


def _axis_from_pca(X: torch.Tensor) -> torch.Tensor:
    Xc = X - X.mean(dim=0, keepdim=True)
    _, _, Vt = torch.linalg.svd(Xc, full_matrices=False)
    u = _fix_sign(Vt[0])
    return u / (u.norm() + _EPS)


def compute_axis(Q: torch.Tensor, positional_embedding: Optional[torch.Tensor] = None
                 ) -> Tuple[torch.Tensor, str]:
    """Q [N, D] (and optionally P [N, D]) -> (unit axis [D], "positional" | "pca")."""
    if Q.dim() != 2:
        raise ValueError(f"expected Q shape [N, D], got {tuple(Q.shape)}")
    if positional_embedding is not None:
        if positional_embedding.shape != Q.shape:
            raise ValueError(f"positional_embedding shape {tuple(positional_embedding.shape)} "
                             f"must match Q shape {tuple(Q.shape)}")
        return _axis_from_positional(positional_embedding), "positional"
    return _axis_from_pca(Q), "pca"


def pca_axes(X: torch.Tensor) -> torch.Tensor:
    """X [B, H, N, D] -> fp32 [B, H, D]: the unit principal direction of each
    head's rows, on X's device."""
    if X.dim() != 4:
        raise ValueError(f"expected [B, H, N, D], got {tuple(X.shape)}")
    B, H, N, D = X.shape
    Xf = X.float()
    Xc = Xf - Xf.mean(dim=2, keepdim=True)
    C = torch.matmul(Xc.transpose(-1, -2).contiguous(), Xc)          # [B, H, D, D] fp32
    _, vecs = torch.linalg.eigh(C.double().cpu())                    # ascending eigenvalues
    u = _fix_sign(vecs[..., :, -1])
    u = u / (u.norm(dim=-1, keepdim=True) + _EPS)
    return u.to(device=X.device, dtype=torch.float32)
