"""Caller-side sort bookkeeping for rank-local attention (pure torch).

Mirrors ``prepare_sort_indices``, ``gather_by_sort_idx`` and
``scatter_by_inv_perm`` (dcr_attention/kernel/sort_helpers.py): keys and
queries are ordered by their projection onto an axis u,

    z_q = <Q, u>,  z_k = <K, u>,
    sort_idx_k = argsort(z_k), rank_of_k = argsort(sort_idx_k) (the inverse permutation,
    computed with one scatter), sort_idx_q = argsort(z_q), inv_q_perm likewise,
    r_center[t] = #{j : z_k[j] < z_q[sort_idx_q[t]]}  clamped to [0, N_kv - 1]

(the insertion rank of each sorted query among the sorted keys, so r_center
is non-decreasing in t).  Host-side glue around the HIP kernel; the kernel
itself is ``kernel.hip.rank_local_fwd``.
"""
from __future__ import annotations

from typing import NamedTuple

import torch


class SortIndices(NamedTuple):
    sort_idx_k: torch.Tensor
    rank_of_k: torch.Tensor
    sort_idx_q: torch.Tensor
    inv_q_perm: torch.Tensor
    r_center: torch.Tensor
    z_q: torch.Tensor
    z_k: torch.Tensor


def _inverse_permutation(p: torch.Tensor) -> torch.Tensor:
    """argsort of a permutation (last dim), as one scatter instead of a sort."""
    inv = torch.empty_like(p)
    ar = torch.arange(p.shape[-1], device=p.device, dtype=p.dtype).expand_as(p)
    return inv.scatter_(-1, p, ar)


def prepare_sort_indices(Q: torch.Tensor, K: torch.Tensor, axis: torch.Tensor) -> SortIndices:
    """Q [B,H,N_q,D], K [B,H,N_kv,D], axis [D] or [B,H,D] (unit norm by the caller).

    K may also hold H_kv heads with H % H_kv == 0 (an un-repeated GQA cache):
    query head h then orders the keys of KV head h // (H / H_kv), exactly as
    for the repeated cache, without materialising the repeat."""
    if Q.dim() != 4 or K.dim() != 4:
        raise ValueError(f"expected [B,H,N,D] for Q and K, got {tuple(Q.shape)} and {tuple(K.shape)}")
    if (Q.shape[0] != K.shape[0] or Q.shape[3] != K.shape[3] or K.shape[1] == 0
            or Q.shape[1] % K.shape[1] != 0):
        raise ValueError(f"Q shape {tuple(Q.shape)} and K shape {tuple(K.shape)} must agree on (B, D) "
                         "and K's heads must divide Q's")
    B, H, _, D = Q.shape
    Hkv = K.shape[1]
    if axis.dim() == 1:
        if axis.shape[0] != D:
            raise ValueError(f"axis shape {tuple(axis.shape)} must be [D={D}]")
        a = axis.to(Q.dtype).view(1, 1, D, 1)
    elif axis.dim() == 3:
        if axis.shape != (B, H, D):
            raise ValueError(f"axis shape {tuple(axis.shape)} must be [B={B}, H={H}, D={D}]")
        a = axis.to(Q.dtype).unsqueeze(-1)
    else:
        raise ValueError(f"axis must be 1-D [D] or 3-D [B, H, D], got {axis.dim()}-D")
    z_q = torch.matmul(Q, a).squeeze(-1)
    # One product per KV head, all its query heads' axes as columns:
    # [B, Hkv, N, D] @ [B, Hkv, D, n_rep] reads K once (the same values as
    # one matrix-vector product per query head, which re-reads K n_rep times).
    r = H // Hkv
    A = a.to(K.dtype).expand(B, H, D, 1).reshape(B, Hkv, r, D).transpose(-1, -2).contiguous()
    z_k = torch.matmul(K, A).transpose(-1, -2).reshape(B, H, -1)
    sort_idx_k = torch.argsort(z_k, dim=-1)
    rank_of_k = _inverse_permutation(sort_idx_k)
    sort_idx_q = torch.argsort(z_q, dim=-1)
    inv_q_perm = _inverse_permutation(sort_idx_q)
    zq_sorted = torch.gather(z_q, -1, sort_idx_q).contiguous()
    zk_sorted = torch.gather(z_k, -1, sort_idx_k).contiguous()
    r_center = torch.searchsorted(zk_sorted, zq_sorted).clamp_(0, K.shape[-2] - 1)
    return SortIndices(sort_idx_k, rank_of_k, sort_idx_q, inv_q_perm, r_center, z_q, z_k)


def gather_by_sort_idx(X: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """X [B,H,N,D] reordered along N: out[..., t, :] = X[..., idx[..., t], :].

    X may hold H_kv heads dividing idx's H (an un-repeated GQA cache): row t
    of head h is then X[b, h // (H / H_kv), idx[b, h, t]], read through a
    broadcast view (no repeated copy of X)."""
    if idx.dim() != 3:
        raise ValueError(f"idx must be [B,H,N], got {tuple(idx.shape)}")
    B, H, n = idx.shape
    Hkv, D = X.shape[1], X.shape[-1]
    if Hkv == H:
        return torch.gather(X, 2, idx.unsqueeze(-1).expand(-1, -1, -1, D))
    if Hkv == 0 or H % Hkv != 0:
        raise ValueError(f"X heads {Hkv} must divide idx heads {H}")
    r = H // Hkv
    Xb = X.unsqueeze(2).expand(B, Hkv, r, X.shape[2], D)
    ib = idx.reshape(B, Hkv, r, n).unsqueeze(-1).expand(B, Hkv, r, n, D)
    return torch.gather(Xb, 3, ib).reshape(B, H, n, D)


def scatter_by_inv_perm(X_sorted: torch.Tensor, inv_perm: torch.Tensor) -> torch.Tensor:
    """Undo a sort: out[..., i] = X_sorted[..., inv_perm[..., i]] ([B,H,N,D] or [B,H,N])."""
    if inv_perm.dim() != 3:
        raise ValueError(f"inv_perm must be [B,H,N], got {tuple(inv_perm.shape)}")
    if X_sorted.dim() == 4:
        return torch.gather(X_sorted, 2, inv_perm.unsqueeze(-1).expand(-1, -1, -1, X_sorted.shape[-1]))
    if X_sorted.dim() == 3:
        return torch.gather(X_sorted, 2, inv_perm)
    raise ValueError(f"X_sorted must be [B,H,N,D] or [B,H,N], got {tuple(X_sorted.shape)}")
