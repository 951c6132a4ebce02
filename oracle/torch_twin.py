"""The reference's M1 oracle restated with the same torch calls.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Each function follows one step of
``dcr_attention/kernel/qaxis_topk_reference.py`` (file:line cited per
function) using the torch operation the reference uses for that step, so its
bits are the reference's bits wherever those come from torch's CPU kernels
(``torch.linalg.norm``, ``torch.einsum`` -> MKL sgemm, ``torch.argsort``).
It differs from M1 only where M1 cannot run: it accepts fp16/fp32 inputs
(M1 asserts bf16, :220-222) and does not round gathered rows to bf16
(:128-129), which is a no-op for bf16 inputs anyway.
It is used to pin the C oracle (``oracle/cpu.py``) bit for bit.
"""
from __future__ import annotations

import math

import torch

_F32 = torch.float32
_BF16 = torch.bfloat16


def compute_u_Q(Q: torch.Tensor, eps: float) -> torch.Tensor:
    """qaxis_topk_reference.py:42-55."""
    q = Q.to(_F32)
    n = torch.linalg.norm(q, dim=-1, keepdim=True).clamp(min=eps)
    return q / n


def projection_scores(K: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """qaxis_topk_reference.py:58-88 (one einsum per KV head, then bf16)."""
    B, Hkv, N, D = K.shape
    H = u.shape[1]
    rep = H // Hkv
    out = torch.empty(B, H, N, dtype=_BF16)
    for g in range(Hkv):
        kf = K[:, g].to(_F32)
        ug = u[:, g * rep:(g + 1) * rep]
        s = torch.einsum("bnd,bhd->bnh", kf, ug)
        out[:, g * rep:(g + 1) * rep] = s.transpose(-2, -1).to(_BF16)
    return out


def select_topk(scores: torch.Tensor, k: int) -> torch.Tensor:
    """qaxis_topk_reference.py:91-108, int32 like topk_axis_pass2.py:43."""
    order = torch.argsort(scores.float(), dim=-1, descending=True, stable=True)
    top, _ = order[..., :k].sort(dim=-1)
    return top.to(torch.int32)


def gather_kv(K, V, idx):
    """qaxis_topk_reference.py:111-145 (rows kept in their input dtype)."""
    B, Hkv, N, D = K.shape
    H = idx.shape[1]
    rep = H // Hkv
    g = torch.arange(H) // rep
    ii = idx.long()
    Ks = K[torch.arange(B)[:, None, None], g[None, :, None], ii]
    Vs = V[torch.arange(B)[:, None, None], g[None, :, None], ii]
    return Ks, Vs


def fused_softmax_attention(K_sel, V_sel, Q, block: int = 64) -> torch.Tensor:
    """qaxis_topk_reference.py:148-193; returns the fp32 result before the cast."""
    B, H, k, D = K_sel.shape
    scale = 1.0 / math.sqrt(D)
    q = Q.to(_F32)
    m = torch.full((B, H), float("-inf"), dtype=_F32)
    l = torch.zeros(B, H, dtype=_F32)
    o = torch.zeros(B, H, D, dtype=_F32)
    for t0 in range(0, k, block):
        kb = K_sel[:, :, t0:t0 + block].to(_F32)
        vb = V_sel[:, :, t0:t0 + block].to(_F32)
        s = torch.einsum("bhd,bhjd->bhj", q, kb) * scale
        m_new = torch.maximum(m, s.amax(dim=-1))
        alpha = torch.exp(m - m_new)
        beta = torch.exp(s - m_new.unsqueeze(-1))
        l = alpha * l + beta.sum(dim=-1)
        o = alpha.unsqueeze(-1) * o + torch.einsum("bhj,bhjd->bhd", beta, vb)
        m = m_new
    return o / l.unsqueeze(-1)


def sparse_decode(Q, K, V, k: int, eps: float = 1e-12):
    """qaxis_topk_reference.py:200-259; returns dict like oracle.cpu.sparse_decode."""
    N = K.shape[2]
    if N <= k:
        raise ValueError(f"kernel invoked with N={N} <= k_eff={k}; caller must dispatch to SDPA")
    u = compute_u_Q(Q, eps)
    sc = projection_scores(K, u)
    idx = select_topk(sc, k)
    Ks, Vs = gather_kv(K, V, idx)
    out = fused_softmax_attention(Ks, Vs, Q)
    return {"u": u, "scores": sc, "idx": idx, "out_f32": out, "out": out.to(Q.dtype)}


def rank_local_fwd(Q, K_sorted, V_sorted, r_center, k_window: int, scale=None):
    """rank_local_fwd_torch.py:21-113 with the same torch operations: fp32
    upcast, einsum logits * scale, window mask |j - r| <= k//2 as -inf,
    logsumexp, softmax (NaN rows -> 0), einsum with V, cast to Q's dtype.
    Returns (O in Q's dtype, LSE fp32)."""
    B, H, Nq, D = Q.shape
    Nkv = K_sorted.shape[-2]
    if scale is None:
        scale = 1.0 / (D ** 0.5)
    half_k = k_window // 2
    q, k, v = Q.to(_F32), K_sorted.to(_F32), V_sorted.to(_F32)
    pos = torch.arange(Nkv).view(1, 1, 1, Nkv)
    in_win = (pos - r_center.to(torch.int64).unsqueeze(-1)).abs() <= half_k
    s = torch.einsum("bhid,bhjd->bhij", q, k) * scale
    s = s.masked_fill(~in_win, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
    out = torch.einsum("bhij,bhjd->bhid", p, v)
    return out.to(Q.dtype), lse
