"""HIP rank-local window attention (kernel.hip.rank_local_fwd) against the
float64 oracle, through the C-ABI.

Shape matrix from the reference's GPU suite (test_triton_gpu_correctness.py:
N in {128, 512, 2048}, D in {32, 64, 128}, H in {2, 8}, k in {16, 64, 256})
and its decode-shape suite (test_decode_shape_correctness.py: Q.N = 1).
Tolerances (tighter than the reference's 1e-2 for half types):
  O:   fp32 1e-5 max-abs; fp16 2e-3; bf16 max(5e-3, 1 output ulp)
  LSE: 2e-5 absolute + 1e-6 relative (fp32 natural log)
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import cpu
from dcr_attention_amd.kernel import sort_helpers as sh
from dcr_attention_amd.kernel.hip.rank_local_fwd import rank_local_fwd_hip

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 5e-3}


def _check(out, lse, o64, l64, dtype):
    o = out.double().cpu()
    diff = (o - o64).abs()
    tol = torch.full_like(o64, TOL[dtype])
    if dtype == torch.bfloat16:
        tol = torch.maximum(tol, torch.ldexp(torch.ones_like(o64), torch.frexp(o64)[1] - 8))
    assert (diff <= tol).all(), f"max|dO|={diff.max().item():.3e}"
    dl = (lse.double().cpu() - l64).abs()
    assert (dl <= 2e-5 + 1e-6 * l64.abs()).all(), f"max|dLSE|={dl.max().item():.3e}"
    assert torch.isfinite(o).all()


def _prefill_case(B, H, N, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(B, H, N, D, generator=g).to(dtype)
    K = torch.randn(B, H, N, D, generator=g).to(dtype)
    V = torch.randn(B, H, N, D, generator=g).to(dtype)
    axis = torch.randn(D, generator=g)
    axis = axis / axis.norm()
    idx = sh.prepare_sort_indices(Q.float(), K.float(), axis)
    return (sh.gather_by_sort_idx(Q, idx.sort_idx_q), sh.gather_by_sort_idx(K, idx.sort_idx_k),
            sh.gather_by_sort_idx(V, idx.sort_idx_k), idx)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N,D,H,k", [
    (128, 32, 2, 16), (128, 64, 8, 256), (128, 128, 2, 64),
    (512, 32, 8, 64), (512, 64, 2, 256), (512, 128, 8, 16),
    (2048, 32, 2, 256), (2048, 64, 8, 64), (2048, 128, 2, 16),
    # at least 4096 query rows: the matrix-core prefill path for half types;
    # ragged query blocks, a window of one key, a window wider than N
    (1000, 64, 8, 2000), (1000, 32, 8, 1), (4100, 128, 1, 256),
])
def test_prefill_matches_oracle(dtype, N, D, H, k):
    Qs, Ks, Vs, idx = _prefill_case(1, H, N, D, dtype, seed=N + D + H + k)
    out, lse = rank_local_fwd_hip(Qs.to(DEV), Ks.to(DEV), Vs.to(DEV), idx.rank_of_k.to(DEV),
                                  idx.r_center.to(DEV), k)
    assert out.shape == (1, H, N, D) and out.dtype == dtype and lse.dtype == torch.float32
    o64, l64 = cpu.rank_local_f64(Qs, Ks, Vs, idx.r_center, k)
    _check(out, lse, o64, l64, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N_kv,D,k", [(512, 64, 16), (4096, 64, 64), (32768, 64, 4096),
                                      (2048, 128, 256), (300, 32, 64)])
def test_decode_matches_oracle(dtype, N_kv, D, k):
    B, H = 2, 8
    g = torch.Generator().manual_seed(N_kv + k)
    Q = torch.randn(B, H, 1, D, generator=g).to(dtype)
    K = torch.randn(B, H, N_kv, D, generator=g).to(dtype)
    V = torch.randn(B, H, N_kv, D, generator=g).to(dtype)
    rc = torch.randint(0, N_kv, (B, H, 1), generator=g)
    rc[0, 0, 0] = 0
    rc[0, 1, 0] = N_kv - 1
    out, lse = rank_local_fwd_hip(Q.to(DEV), K.to(DEV), V.to(DEV), None, rc.to(DEV), k)
    o64, l64 = cpu.rank_local_f64(Q, K, V, rc, k)
    _check(out, lse, o64, l64, dtype)


def test_full_window_equals_dense():
    # test_decode_shape_correctness.py:99-124
    from dcr_attention_amd.kernel.hip.dense import dense_decode_attention
    B, H, N, D = 1, 4, 1000, 64
    g = torch.Generator().manual_seed(3)
    Q = torch.randn(B, H, 1, D, generator=g)
    K = torch.randn(B, H, N, D, generator=g)
    V = torch.randn(B, H, N, D, generator=g)
    rc = torch.full((B, H, 1), 500, dtype=torch.int32)
    out, _ = rank_local_fwd_hip(Q.to(DEV), K.to(DEV), V.to(DEV), None, rc.to(DEV), 2 * N)
    dense = dense_decode_attention(Q[:, :, 0].contiguous().to(DEV), K.to(DEV), V.to(DEV))
    assert (out[:, :, 0].cpu() - dense.cpu()).abs().max().item() <= 1e-5


def _check_with_empty_rows(out, lse, o64, l64, dtype):
    """_check, with rows whose window holds no key allowed: there the
    reference gives O = 0 and LSE = -inf (rank_local_fwd_triton.py:194-202)."""
    empty = torch.isinf(l64)
    assert torch.equal(torch.isinf(lse.cpu()), empty)
    assert (out.cpu()[empty] == 0).all()
    assert (lse.cpu()[empty] == -math.inf).all()
    keep = ~empty
    _check(out[keep.to(DEV)], lse[keep.to(DEV)], o64[keep], l64[keep], dtype)


def test_window_of_one_and_out_of_range_centres():
    """r_center as the caller passes it (the reference does not clamp it in the
    kernel): a window of one key outside [0, Nkv) is empty."""
    g = torch.Generator().manual_seed(4)
    Q = torch.randn(1, 2, 3, 64, generator=g)
    K = torch.randn(1, 2, 40, 64, generator=g)
    V = torch.randn(1, 2, 40, 64, generator=g)
    rc = torch.tensor([[[-5, 7, 99], [0, 39, 20]]], dtype=torch.int32)
    out, lse = rank_local_fwd_hip(Q.to(DEV), K.to(DEV), V.to(DEV), None, rc.to(DEV), 1)
    o64, l64 = cpu.rank_local_f64(Q, K, V, rc, 1)
    _check_with_empty_rows(out, lse, o64, l64, torch.float32)
    assert torch.equal(out[0, 0, 1].cpu(), V[0, 0, 7])        # centre 7 -> row 7
    assert (out[0, 0, 0] == 0).all() and (out[0, 0, 2] == 0).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Nq", [9, 4096])     # decode kernel; matrix-core prefill (half types)
def test_centres_at_nkv_and_negative(dtype, Nq):
    """r_center = Nkv (raw searchsorted output) keeps half_k keys, a negative
    centre fewer, and centres past the rows give empty windows -- against the
    float64 oracle, which follows the reference's mask."""
    B, H, Nkv, D, k = 1, 2, 300, 64, 16
    g = torch.Generator().manual_seed(Nq)
    Q = torch.randn(B, H, Nq, D, generator=g).to(dtype)
    K = torch.randn(B, H, Nkv, D, generator=g).to(dtype)
    V = torch.randn(B, H, Nkv, D, generator=g).to(dtype)
    rc = torch.randint(0, Nkv, (B, H, Nq), generator=g, dtype=torch.int32)
    specials = torch.tensor([Nkv, Nkv + 3, -1, -8, -9, Nkv + 8, Nkv + 9, 2**31 - 1, -2**31],
                            dtype=torch.int32)
    rc[:, :, : specials.numel()] = specials
    out, lse = rank_local_fwd_hip(Q.to(DEV), K.to(DEV), V.to(DEV), None, rc.to(DEV), k)
    o64, l64 = cpu.rank_local_f64(Q, K, V, rc, k)
    _check_with_empty_rows(out, lse, o64, l64, dtype)
    assert int(torch.isinf(l64).sum()) == 5 * B * H     # -9, Nkv + 8, Nkv + 9, 2^31 - 1, -2^31


def test_api_path_restores_query_order():
    """The reference's public path: sort, kernel, scatter back (rank_local_attention.py:79-115)."""
    B, H, N, D, k = 1, 2, 256, 64, 32
    g = torch.Generator().manual_seed(5)
    Q = torch.randn(B, H, N, D, generator=g)
    K = torch.randn(B, H, N, D, generator=g)
    V = torch.randn(B, H, N, D, generator=g)
    axis = torch.randn(D, generator=g)
    axis = axis / axis.norm()
    idx = sh.prepare_sort_indices(Q, K, axis)
    Qs, Ks, Vs = (sh.gather_by_sort_idx(Q, idx.sort_idx_q), sh.gather_by_sort_idx(K, idx.sort_idx_k),
                  sh.gather_by_sort_idx(V, idx.sort_idx_k))
    out_s, _ = rank_local_fwd_hip(Qs.to(DEV), Ks.to(DEV), Vs.to(DEV), None, idx.r_center.to(DEV), k)
    out = sh.scatter_by_inv_perm(out_s.cpu(), idx.inv_q_perm)
    o64, _ = cpu.rank_local_f64(Qs, Ks, Vs, idx.r_center, k)
    ref = sh.scatter_by_inv_perm(o64, idx.inv_q_perm)
    assert (out.double() - ref).abs().max().item() <= 1e-5


def _oracle_public(Q, K, V, idx, k):
    """The oracle on the sort bookkeeping the product glue computed (indices
    copied to the host); GQA caches are gathered per query head."""
    ix = [t.cpu() for t in (idx.sort_idx_k, idx.sort_idx_q, idx.r_center, idx.inv_q_perm)]
    Ks, Vs = sh.gather_by_sort_idx(K, ix[0]), sh.gather_by_sort_idx(V, ix[0])
    Qs = sh.gather_by_sort_idx(Q, ix[1])
    o64, _ = cpu.rank_local_f64(Qs, Ks, Vs, ix[2], k)
    return sh.scatter_by_inv_perm(o64, ix[3])


def _close(out, ref, dtype):
    diff = (out.double().cpu() - ref).abs()
    tol = torch.full_like(ref, TOL[dtype])
    if dtype == torch.bfloat16:
        tol = torch.maximum(tol, torch.ldexp(torch.ones_like(ref), torch.frexp(ref)[1] - 8))
    assert (diff <= tol).all(), f"max|dO|={diff.max().item():.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hkv", [8, 2])
def test_public_rank_local_attention(dtype, Hkv):
    """rank_local_attention (rank_local_attention.py:142-200): sort, kernel,
    scatter; an un-repeated GQA cache gives the repeated cache's result."""
    from dcr_attention_amd.kernel.rank_local_attention import _normalize_axis, rank_local_attention
    B, H, N, D, k = 1, 8, 1000, 64, 128
    g = torch.Generator().manual_seed(11 + Hkv)
    Q = torch.randn(B, H, N, D, generator=g).to(dtype)
    K = torch.randn(B, Hkv, N, D, generator=g).to(dtype)
    V = torch.randn(B, Hkv, N, D, generator=g).to(dtype)
    axis = torch.randn(D, generator=g)
    out = rank_local_attention(Q.to(DEV), K.to(DEV), V.to(DEV), axis.to(DEV), k_window=k)
    assert out.shape == (B, H, N, D) and out.dtype == dtype
    idx = sh.prepare_sort_indices(Q.to(DEV), K.to(DEV), _normalize_axis(axis.to(DEV)))
    _close(out, _oracle_public(Q, K, V, idx, k), dtype)


@pytest.mark.parametrize("source", ["q", "pca"])
@pytest.mark.parametrize("widen", [False, True])
@pytest.mark.parametrize("kv_repeated", [False, True])
def test_dcr_forward_rank_local_decode(source, widen, kv_repeated):
    """Rank-local decode (attention.py:816-880): the window along Q/||Q||
    ("q") or the keys' principal direction ("pca") with k_eff =
    adaptive_k_window, optionally widened once."""
    from dcr_attention_amd.kernel.rank_local_attention import _normalize_axis
    from dcr_attention_amd.llama.adaptive import adaptive_k_window, detect_leaky_boundary, widen_factor
    from dcr_attention_amd.llama.attention import dcr_forward, rank_local_axes
    from dcr_attention_amd.llama.config import DCRLlamaConfig
    B, H, Hkv, N, D = 2, 8, 2, 6000, 64
    dtype = torch.float16
    g = torch.Generator().manual_seed(21)
    Q = torch.randn(B, H, 1, D, generator=g).to(dtype)
    K = torch.randn(B, Hkv, N, D, generator=g).to(dtype)
    V = torch.randn(B, Hkv, N, D, generator=g).to(dtype)
    cfg = DCRLlamaConfig(axis_source=source, enable_adaptive_widening=widen)
    Kc, Vc = (K.repeat_interleave(4, dim=1), V.repeat_interleave(4, dim=1)) if kv_repeated else (K, V)
    out = dcr_forward(Q.to(DEV), Kc.to(DEV), Vc.to(DEV), cfg, n_rep=4, kv_repeated=kv_repeated)
    assert out.shape == (B, H, 1, D) and out.dtype == dtype
    k_eff = adaptive_k_window(cfg.k_window, N, cfg.coverage_floor)
    q = Q.squeeze(-2).float().to(DEV)
    axes = rank_local_axes(Q.to(DEV), K.to(DEV), source)
    idx = sh.prepare_sort_indices(Q.to(DEV), K.to(DEV), _normalize_axis(axes))
    k_use = k_eff
    if widen:
        kp = torch.matmul(K.float().to(DEV).unsqueeze(2), axes.reshape(B, Hkv, 4, D, 1)).reshape(B, H, N)
        leaky = detect_leaky_boundary((q * axes).sum(-1, keepdim=True), kp, torch.argsort(kp, dim=-1), k_eff)
        if bool(leaky.any()):
            k_use = widen_factor(k_eff, N)
    _close(out, _oracle_public(Q, K, V, idx, k_use), dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,H,Hkv,Nq,Nkv,D,k,repeated", [
    (2, 8, 2, 1, 5000, 64, 700, False),      # decode (window split over waves)
    (1, 8, 8, 1, 3000, 128, 64, False),
    (1, 8, 2, 4100, 4100, 64, 256, False),   # prefill (matrix cores for fp16/bf16)
    (1, 4, 1, 1000, 1000, 32, 100, True),    # a strided view of a repeated cache
])
def test_gather_path_bit_identical(dtype, B, H, Hkv, Nq, Nkv, D, k, repeated):
    """dcr_rank_local_fwd_gather reads K/V through the sort permutation; it
    must equal the kernel on gathered sorted copies bit for bit."""
    from dcr_attention_amd.kernel.hip.rank_local_fwd import rank_local_fwd_gather_hip
    g = torch.Generator().manual_seed(B + H + Nq + D)
    Q = torch.randn(B, H, Nq, D, generator=g).to(dtype).to(DEV)
    K = torch.randn(B, Hkv, Nkv, D, generator=g).to(dtype).to(DEV)
    V = torch.randn(B, Hkv, Nkv, D, generator=g).to(dtype).to(DEV)
    if repeated:   # the kernel reads K[:, ::n_rep] of the repeated cache in place
        n_rep = H // Hkv
        K = K.repeat_interleave(n_rep, dim=1)[:, ::n_rep]
        V = V.repeat_interleave(n_rep, dim=1)[:, ::n_rep]
    axis = torch.randn(B, H, D, generator=g).to(DEV)
    axis = axis / axis.norm(dim=-1, keepdim=True)
    idx = sh.prepare_sort_indices(Q, K, axis)
    Qs = sh.gather_by_sort_idx(Q, idx.sort_idx_q)
    o_ref, l_ref = rank_local_fwd_hip(Qs, sh.gather_by_sort_idx(K, idx.sort_idx_k),
                                      sh.gather_by_sort_idx(V, idx.sort_idx_k), None, idx.r_center, k)
    o, l = rank_local_fwd_gather_hip(Qs, K, V, idx.sort_idx_k, idx.r_center, k)
    assert torch.equal(o, o_ref) and torch.equal(l, l_ref)


def test_gather_path_clamps_permutation_entries():
    from dcr_attention_amd.kernel.hip.rank_local_fwd import rank_local_fwd_gather_hip
    g = torch.Generator().manual_seed(31)
    B, H, N, D = 1, 2, 300, 64
    Q = torch.randn(B, H, 1, D, generator=g).to(DEV)
    K = torch.randn(B, H, N, D, generator=g).to(DEV)
    V = torch.randn(B, H, N, D, generator=g).to(DEV)
    perm = torch.stack([torch.randperm(N, generator=g) for _ in range(B * H)]).view(B, H, N)
    bad = perm.clone()
    bad[0, 0, :7] = -5
    bad[0, 1, :7] = N + 3
    clamped = bad.clamp(0, N - 1)
    rc = torch.full((B, H, 1), 3, dtype=torch.int32)
    o_bad, _ = rank_local_fwd_gather_hip(Q, K, V, bad.to(DEV), rc.to(DEV), 16)
    o_ok, _ = rank_local_fwd_gather_hip(Q, K, V, clamped.to(DEV), rc.to(DEV), 16)
    assert torch.equal(o_bad, o_ok)


def test_public_api_accepts_any_kv_layout():
    """K/V whose rows are not contiguous are copied once, not rejected (the
    reference's gather accepts any layout)."""
    from dcr_attention_amd.kernel.rank_local_attention import rank_local_attention
    g = torch.Generator().manual_seed(41)
    B, H, N, D = 1, 4, 500, 64
    Q = torch.randn(B, H, 1, D, generator=g).to(DEV)
    Kt = torch.randn(B, H, D, N, generator=g).to(DEV)          # stored transposed
    Vt = torch.randn(B, H, D, N, generator=g).to(DEV)
    K, V = Kt.transpose(-1, -2), Vt.transpose(-1, -2)
    axis = torch.randn(D, generator=g).to(DEV)
    out = rank_local_attention(Q, K, V, axis, k_window=64)
    ref = rank_local_attention(Q, K.contiguous(), V.contiguous(), axis, k_window=64)
    assert torch.equal(out, ref)
