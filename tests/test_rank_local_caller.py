"""Caller-side logic of the rank-local ("q" axis) decode branch, on the CPU:
the widening helpers (adaptive.py:108-221 in the reference) against
brute-force restatements, and the GQA form of the sort helpers against the
repeated-cache form they replace."""
from __future__ import annotations

import pytest
import torch

from dcr_attention_amd.kernel import sort_helpers as sh
from dcr_attention_amd.llama.adaptive import detect_leaky_boundary, widen_factor
from dcr_attention_amd.llama.attention import dcr_forward
from dcr_attention_amd.llama.config import DCRLlamaConfig


@pytest.mark.parametrize("prev,n,want", [(64, 1000, 128), (600, 1000, 1000), (500, 999, 999),
                                         (63, 1000, 126), (1000, 1000, 1002), (2, 3, 4)])
def test_widen_factor(prev, n, want):
    # int(prev * 2) capped at n, rounded up to even (re-capped), never below prev + 2
    assert widen_factor(prev, n) == want


def _leaky_brute(q_proj, k_proj, k_eff, slack):
    B, H, N = k_proj.shape
    out = torch.zeros(B, H, dtype=torch.bool)
    for b in range(B):
        for h in range(H):
            ks = sorted(float(x) for x in k_proj[b, h])
            q = float(q_proj[b, h, 0])
            rank = min(sum(1 for x in ks if x < q), N - 1)          # insertion rank (left)
            start = max(rank - k_eff // 2, 0)
            end = min(start + k_eff, N)
            start = max(end - k_eff, 0)
            d_in = max(abs(ks[i] - q) for i in range(start, end))
            d_out = min(abs(ks[i] - q) for i in range(N) if not (start <= i < end))
            out[b, h] = d_out < slack * d_in
    return out


@pytest.mark.parametrize("seed", range(4))
def test_detect_leaky_boundary_matches_brute_force(seed):
    g = torch.Generator().manual_seed(seed)
    B, H, N, k = 2, 3, 50, 10
    k_proj = torch.randn(B, H, N, generator=g, dtype=torch.float64)
    q_proj = torch.randn(B, H, 1, generator=g, dtype=torch.float64) * 0.5
    # plant a rejected key just outside one window, closer than the window's far end
    k_proj[0, 0, 0] = q_proj[0, 0, 0] + 1e-9
    got = detect_leaky_boundary(q_proj, k_proj, torch.argsort(k_proj, dim=-1), k, slack=0.5)
    assert torch.equal(got, _leaky_brute(q_proj, k_proj, k, 0.5))
    full = detect_leaky_boundary(q_proj, k_proj, torch.argsort(k_proj, dim=-1), N, slack=0.5)
    assert not full.any()


def test_detect_leaky_boundary_clean_and_leaky_cases():
    # evenly spaced keys: the rank window holds the nearest keys -> clean
    k_proj = torch.arange(20, dtype=torch.float32).view(1, 1, 20)
    q = torch.tensor([[[9.5]]])
    assert not detect_leaky_boundary(q, k_proj, torch.argsort(k_proj, dim=-1), 6).any()
    # a gap right of the query: the window (sorted positions 8..11) reaches
    # the far key 100 while key 7 (distance 2.5) is left out -> leaky
    k_gap = torch.tensor([[[0., 1, 2, 3, 4, 5, 6, 7, 8, 9, 9.6, 100, 101, 102]]])
    perm = torch.randperm(14, generator=torch.Generator().manual_seed(0))
    k_gap = k_gap[..., perm]                                   # caller order is arbitrary
    assert detect_leaky_boundary(q, k_gap, torch.argsort(k_gap, dim=-1), 4).all()


@pytest.mark.parametrize("axis_shape", ["shared", "per_head"])
def test_sort_helpers_gqa_equal_repeated_cache(axis_shape):
    g = torch.Generator().manual_seed(7)
    B, H, Hkv, N, D = 2, 8, 2, 40, 16
    Q = torch.randn(B, H, 3, D, generator=g)
    K = torch.randn(B, Hkv, N, D, generator=g)
    axis = torch.randn(D, generator=g) if axis_shape == "shared" else torch.randn(B, H, D, generator=g)
    axis = axis / axis.norm(dim=-1, keepdim=True)
    Krep = K.repeat_interleave(H // Hkv, dim=1)
    a = sh.prepare_sort_indices(Q, K, axis)
    r = sh.prepare_sort_indices(Q, Krep, axis)
    for x, y in zip(a, r):
        assert torch.allclose(x.double(), y.double(), rtol=0, atol=1e-6) if x.is_floating_point() \
            else torch.equal(x, y)
    assert torch.equal(sh.gather_by_sort_idx(K, r.sort_idx_k), sh.gather_by_sort_idx(Krep, r.sort_idx_k))
    with pytest.raises(ValueError):
        sh.prepare_sort_indices(Q, torch.randn(B, 3, N, D), axis)


def test_q_axis_branch_needs_device_tensors():
    Q = torch.randn(1, 4, 1, 64)
    K = torch.randn(1, 4, 512, 64)
    with pytest.raises(RuntimeError):
        dcr_forward(Q, K, K, DCRLlamaConfig(axis_source="q"), n_rep=1)


# ---- ordering axes (stage_b.py:41-100; tests follow test_stage_b.py) -------

from dcr_attention_amd.kernel.axis import compute_axis, pca_axes  # noqa: E402
from dcr_attention_amd.llama.attention import rank_local_axes  # noqa: E402


def _cos_abs(a, b):
    return abs(torch.nn.functional.cosine_similarity(a.flatten().double(), b.flatten().double(), dim=0).item())


def test_pca_recovers_rank_one_axis():
    torch.manual_seed(42)
    N, D = 256, 32
    u = torch.randn(D); u = u / u.norm()
    X = torch.randn(N).unsqueeze(-1) * u + 0.01 * torch.randn(N, D)
    a, src = compute_axis(X)
    assert src == "pca" and abs(a.norm().item() - 1.0) < 1e-5
    assert _cos_abs(a, u) > 0.99
    assert a[a.abs().argmax()] > 0                      # sign rule


def test_positional_axis_noiseless_noisy_and_precedence():
    torch.manual_seed(7)
    N, D = 256, 32
    v = torch.randn(D); v = v / v.norm()
    pos = torch.arange(N, dtype=torch.float32) - (N - 1) / 2.0
    a, src = compute_axis(torch.randn(N, D), positional_embedding=pos.unsqueeze(-1) * v)
    assert src == "positional" and _cos_abs(a, v) > 0.9999
    N = 1024
    pos = torch.arange(N, dtype=torch.float32) - (N - 1) / 2.0
    a, _ = compute_axis(torch.randn(N, D), positional_embedding=pos.unsqueeze(-1) * v + 0.01 * torch.randn(N, D))
    assert _cos_abs(a, v) > 0.95
    with pytest.raises(ValueError):
        compute_axis(torch.randn(4, 3, 2))
    with pytest.raises(ValueError):
        compute_axis(torch.randn(8, 4), positional_embedding=torch.randn(8, 5))


def test_pca_axes_match_per_head_svd():
    """The batched covariance-eigh axes equal the per-head SVD axes of the
    reference's method (first right singular vector of the centred rows), with
    the same sign rule, on inputs with a clear principal direction."""
    g = torch.Generator().manual_seed(3)
    B, H, N, D = 2, 3, 500, 16
    dirs = torch.randn(B, H, D, generator=g)
    dirs = dirs / dirs.norm(dim=-1, keepdim=True)
    X = (torch.randn(B, H, N, 1, generator=g) * 3.0) * dirs.unsqueeze(2) + torch.randn(B, H, N, D, generator=g)
    X = X + 5.0                                          # an offset the centring must remove
    got = pca_axes(X.half())
    for b in range(B):
        for h in range(H):
            ref, _ = compute_axis(X.half()[b, h].double())
            assert torch.allclose(got[b, h].double(), ref, atol=2e-5), (b, h)
            assert _cos_abs(got[b, h], dirs[b, h]) > 0.99


def test_rank_local_axes_per_source():
    g = torch.Generator().manual_seed(5)
    Q = torch.randn(2, 8, 1, 16, generator=g)
    K = torch.randn(2, 2, 300, 16, generator=g)
    aq = rank_local_axes(Q, K, "q")
    assert torch.allclose(aq, Q.squeeze(-2) / Q.squeeze(-2).norm(dim=-1, keepdim=True))
    ap = rank_local_axes(Q, K, "pca")
    assert ap.shape == (2, 8, 16)
    assert torch.equal(ap[:, 0], ap[:, 3]) and torch.equal(ap[:, 4], ap[:, 7])   # one axis per KV group
    assert torch.equal(ap[:, ::4], pca_axes(K))
    assert torch.equal(rank_local_axes(Q, K, "positional"), ap)
