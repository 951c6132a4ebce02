"""ctypes wrapper over the C oracle (``oracle/dcr_oracle.c``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Every function takes
CPU torch tensors, calls the C restatement, and returns CPU torch tensors.
bf16 tensors cross the boundary as their raw 16-bit patterns.

Parity status of each function (how it is pinned, see tests/test_oracle.py):
  compute_uq      bit-exact vs torch.linalg.norm twin; unit-norm; eps guard
  scores          bit-exact vs torch.einsum twin; float64 closed form +-1 ulp
  topk            heapq brute force, torch stable argsort, all-equal KAT,
                  arange KAT
  attention       float64 closed form (1e-5 rel), torch twin (1e-5),
                  k=N-1 vs dense brute force
  attention_f64 / dense_f64   exact closed forms (float64 sums)
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libdcr_oracle.so")
_lib = None

DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc) and return the .so path."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.oracle_compute_uq.argtypes = [vp, i, i, i, f, vp]
        L.oracle_scores.argtypes = [vp, i, vp, i, i, i, i, i, vp]
        L.oracle_topk.argtypes = [vp, i, i, i, vp]
        L.oracle_topk.restype = i
        L.oracle_attention.argtypes = [vp, vp, vp, i, vp, i, i, i, i, i, i, vp]
        L.oracle_attention_f64.argtypes = [vp, vp, vp, i, vp, i, i, i, i, i, i, vp]
        L.oracle_dense_f64.argtypes = [vp, vp, vp, i, i, i, i, i, i, vp]
        L.oracle_sparse_decode.argtypes = [vp, vp, vp, i, i, i, i, i, i, i, f, vp, vp, vp, vp]
        L.oracle_sparse_decode.restype = i
        L.oracle_rank_local_f64.argtypes = [vp, vp, vp, i, vp, i, i, i, i, i, ctypes.c_double,
                                            vp, vp]
        _lib = L
    return _lib


def _cpu(t: torch.Tensor) -> torch.Tensor:
    t = t.detach()
    if t.device.type != "cpu":
        t = t.cpu()
    return t.contiguous()


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def compute_uq(Q: torch.Tensor, eps: float = 1e-12) -> torch.Tensor:
    """u = Q / max(||Q||, eps) in fp32, shape of Q (last dim D)."""
    Q = _cpu(Q)
    D = Q.shape[-1]
    rows = Q.numel() // D
    u = torch.empty(Q.shape, dtype=torch.float32)
    lib().oracle_compute_uq(_ptr(Q), DTYPE_CODE[Q.dtype], rows, D, eps, _ptr(u))
    return u


def scores(K: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """bf16 projection scores [B, H, N] from K [B, Hkv, N, D] and u [B, H, D]."""
    K, u = _cpu(K), _cpu(u).float()
    B, Hkv, N, D = K.shape
    H = u.shape[1]
    assert H % Hkv == 0 and D <= 512
    out = torch.empty(B, H, N, dtype=torch.int16)
    lib().oracle_scores(_ptr(K), DTYPE_CODE[K.dtype], _ptr(u), B, Hkv, H // Hkv, N, D, _ptr(out))
    return out.view(torch.bfloat16)


def topk(scores_bf16: torch.Tensor, k: int) -> torch.Tensor:
    """int32 [..., k] ascending indices of the stable descending top-k."""
    s = _cpu(scores_bf16)
    assert s.dtype == torch.bfloat16
    N = s.shape[-1]
    rows = s.numel() // N if N else 0
    out = torch.empty(*s.shape[:-1], k, dtype=torch.int32)
    rc = lib().oracle_topk(_ptr(s.view(torch.int16)), rows, N, k, _ptr(out))
    if rc != 0:
        raise ValueError(f"oracle_topk: k={k} outside (0, N={N}]")
    return out


def attention(Q, K, V, idx) -> torch.Tensor:
    """M1 step 3+4 restated: fp32 [B, H, D] output (before the final cast)."""
    Q, K, V, idx = _cpu(Q), _cpu(K), _cpu(V), _cpu(idx).to(torch.int32)
    B, H, D = Q.shape
    _, Hkv, N, _ = K.shape
    k = idx.shape[-1]
    assert Q.dtype == K.dtype == V.dtype and D <= 512
    out = torch.empty(B, H, D, dtype=torch.float32)
    lib().oracle_attention(_ptr(Q), _ptr(K), _ptr(V), DTYPE_CODE[Q.dtype], _ptr(idx),
                           B, H, Hkv, N, D, k, _ptr(out))
    return out


def attention_f64(Q, K, V, idx) -> torch.Tensor:
    """Exact softmax attention over the selected rows, float64 [B, H, D]."""
    Q, K, V, idx = _cpu(Q), _cpu(K), _cpu(V), _cpu(idx).to(torch.int32)
    B, H, D = Q.shape
    _, Hkv, N, _ = K.shape
    k = idx.shape[-1]
    out = torch.empty(B, H, D, dtype=torch.float64)
    lib().oracle_attention_f64(_ptr(Q), _ptr(K), _ptr(V), DTYPE_CODE[Q.dtype], _ptr(idx),
                               B, H, Hkv, N, D, k, _ptr(out))
    return out


def dense_f64(Q, K, V) -> torch.Tensor:
    """Exact dense decode attention over all N rows, float64 [B, H, D]."""
    Q, K, V = _cpu(Q), _cpu(K), _cpu(V)
    B, H, D = Q.shape
    _, Hkv, N, _ = K.shape
    out = torch.empty(B, H, D, dtype=torch.float64)
    lib().oracle_dense_f64(_ptr(Q), _ptr(K), _ptr(V), DTYPE_CODE[Q.dtype], B, H, Hkv, N, D,
                           _ptr(out))
    return out


def sparse_decode(Q, K, V, k: int, eps: float = 1e-12):
    """Full M1 pipeline; returns dict(u, scores, idx, out_f32, out)."""
    Q, K, V = _cpu(Q), _cpu(K), _cpu(V)
    B, H, D = Q.shape
    _, Hkv, N, _ = K.shape
    if N <= k:
        raise ValueError(f"kernel invoked with N={N} <= k_eff={k}; caller must dispatch to SDPA")
    u = torch.empty(B, H, D, dtype=torch.float32)
    sc = torch.empty(B, H, N, dtype=torch.int16)
    idx = torch.empty(B, H, k, dtype=torch.int32)
    out = torch.empty(B, H, D, dtype=torch.float32)
    rc = lib().oracle_sparse_decode(_ptr(Q), _ptr(K), _ptr(V), DTYPE_CODE[Q.dtype], B, H, Hkv,
                                    N, D, k, eps, _ptr(u), _ptr(sc), _ptr(idx), _ptr(out))
    if rc != 0:
        raise ValueError("oracle_sparse_decode: invalid shapes")
    return {"u": u, "scores": sc.view(torch.bfloat16), "idx": idx, "out_f32": out,
            "out": out.to(Q.dtype)}


def rank_local_f64(Q, K_sorted, V_sorted, r_center, k_window: int, scale=None):
    """Exact rank-local window attention: (O float64 [B,H,Nq,D], LSE float64 [B,H,Nq])."""
    Q, K_sorted, V_sorted = _cpu(Q), _cpu(K_sorted), _cpu(V_sorted)
    B, H, Nq, D = Q.shape
    Nkv = K_sorted.shape[-2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    rc = _cpu(r_center).to(torch.int32).contiguous()
    out = torch.empty(B, H, Nq, D, dtype=torch.float64)
    lse = torch.empty(B, H, Nq, dtype=torch.float64)
    lib().oracle_rank_local_f64(_ptr(Q), _ptr(K_sorted), _ptr(V_sorted), DTYPE_CODE[Q.dtype],
                                _ptr(rc), B * H, Nq, Nkv, D, int(k_window), float(scale),
                                _ptr(out), _ptr(lse))
    return out, lse


def scale_for(D: int) -> float:
    return 1.0 / math.sqrt(D)
