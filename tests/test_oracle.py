"""Pin the CPU oracle (oracle/dcr_oracle.c) before trusting it as the checker.

Each oracle function is checked against something independent of its own
formula:
  * the reference's M1 algorithm restated with the same torch calls
    (oracle/torch_twin.py: torch.linalg.norm, torch.einsum, torch.argsort) --
    bit-exact on this host's MKL/AVX CPU kernels;
  * float64 closed forms (scores, attention);
  * the reference's own known-answer tests and invariants
    (tests/kernel/test_qaxis_topk_reference.py): all-equal ties -> 0..k-1,
    arange top-k, heap-loop equivalence, unit-norm u_Q, zero-query guard,
    hand-built gather, k = N-1 vs full attention, N <= k raises;
  * brute force on tiny inputs.
"""
from __future__ import annotations

import heapq
import math

import pytest
import torch

from oracle import cpu, torch_twin
from dcr_attention_amd.synthetic import CONFIGS, k_ceil, make_inputs, make_qkv

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _rand(*shape, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


# --------------------------------------------------------------------- u_Q

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [64, 128, 12])
def test_uq_bitexact_vs_torch_norm(dtype, D):
    Q = _rand(3, 32, D, seed=D, dtype=dtype)
    a = cpu.compute_uq(Q)
    b = torch_twin.compute_u_Q(Q, 1e-12)
    if D % 8 == 0:
        assert torch.equal(a, b)
    else:  # scalar tail: torch's contraction choice is not pinned, allow 1 ulp
        assert torch.allclose(a, b, rtol=2e-7, atol=0)


def test_uq_unit_norm_and_zero_guard():
    # test_qaxis_topk_reference.py:107-112 and :181-188
    Q = _rand(2, 4, 64, seed=3)
    u = cpu.compute_uq(Q)
    assert torch.allclose(u.norm(dim=-1), torch.ones(2, 4), atol=1e-5)
    Z = torch.zeros(1, 2, 32, dtype=torch.bfloat16)
    uz = cpu.compute_uq(Z)
    assert torch.isfinite(uz).all() and (uz == 0).all()


# ------------------------------------------------------------------ scores

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n_rep,D", [(4, 64), (1, 64), (2, 128), (8, 64)])
def test_scores_bitexact_vs_torch_einsum(dtype, n_rep, D):
    Hkv = 2 if n_rep == 8 else 4
    Q, K, _ = make_qkv(2, Hkv * n_rep, Hkv, 333, D, dtype, seed=7, n_sinks=4, n_outlier=2)
    u = cpu.compute_uq(Q)
    a = cpu.scores(K, u)
    b = torch_twin.projection_scores(K, u)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_scores_vs_float64_closed_form():
    B, H, Hkv, N, D = 1, 32, 8, 2048, 64
    Q, K, _ = make_qkv(B, H, Hkv, N, D, torch.float32, seed=11, n_sinks=4, n_outlier=2)
    u = cpu.compute_uq(Q)
    s = cpu.scores(K, u).double()
    Kr = K.double().repeat_interleave(H // Hkv, dim=1)          # [B, H, N, D]
    exact = torch.einsum("bhnd,bhd->bhn", Kr, u.double())
    mag = torch.einsum("bhnd,bhd->bhn", Kr.abs(), u.double().abs())
    ulp = torch.ldexp(torch.ones_like(exact), torch.frexp(exact)[1] - 8)  # bf16 ulp
    bound = ulp / 2 + D * 2.0 ** -24 * mag
    assert ((s - exact).abs() <= bound).all()
    # the correctly rounded value is hit almost everywhere
    rounded = exact.float().to(torch.bfloat16).double()
    assert (rounded == s).double().mean() > 0.999


# -------------------------------------------------------------------- top-K

def _heap_topk(vals, k):
    """test_qaxis_topk_reference.py:230-254: explicit min-heap over positions."""
    heap = []
    for i, v in enumerate(vals):
        if len(heap) < k:
            heapq.heappush(heap, (v, -i))
        elif (v, -i) > heap[0]:
            heapq.heapreplace(heap, (v, -i))
    return sorted(-i for _, i in heap)


@pytest.mark.parametrize("seed", [0, 1, 99])
def test_topk_vs_heap_bruteforce(seed):
    g = torch.Generator().manual_seed(seed)
    N, k = 300, 37
    # quantised scores: many ties, both zeros
    s = (torch.randint(-20, 21, (4, N), generator=g).float() / 8).to(torch.bfloat16)
    s[0, ::7] = -0.0
    idx = cpu.topk(s, k)
    for r in range(4):
        vals = [0.0 if v == 0 else v for v in s[r].float().tolist()]
        assert idx[r].tolist() == _heap_topk(vals, k)


def test_topk_all_equal_and_arange_kats():
    # test_qaxis_topk_reference.py:167-174 and :142-160
    s = torch.ones(1, 1, 20, dtype=torch.bfloat16)
    assert cpu.topk(s, 5).tolist() == [[list(range(5))]]
    B, H, N, k = 2, 4, 50, 10
    g = torch.Generator().manual_seed(7)
    sc = (torch.arange(B * H * N, dtype=torch.float32).reshape(B, H, N)
          + torch.rand(B, H, N, generator=g) * 0.01).to(torch.bfloat16)
    exp = sc.float().argsort(dim=-1, descending=True, stable=True)[..., :k].sort(dim=-1)[0]
    assert torch.equal(cpu.topk(sc, k).long(), exp)


@pytest.mark.parametrize("N,k", [(1000, 300), (4096, 615), (5000, 4999), (777, 1)])
def test_topk_vs_torch_stable_argsort(N, k):
    g = torch.Generator().manual_seed(N)
    s = torch.randn(8, N, generator=g).to(torch.bfloat16)
    s[:, 5] = float("nan")
    s[:, 6] = -0.0
    s[:, 7] = 0.0
    s[:, 8] = float("inf")
    assert torch.equal(cpu.topk(s, k), torch_twin.select_topk(s, k))


def test_topk_rejects_bad_k():
    with pytest.raises(ValueError):
        cpu.topk(torch.zeros(1, 10, dtype=torch.bfloat16), 11)


# --------------------------------------------------------------- attention

def test_gather_kat():
    # test_qaxis_topk_reference.py:201-212
    K = _rand(1, 2, 16, 8, seed=1)
    V = _rand(1, 2, 16, 8, seed=2)
    idx = torch.tensor([[[0, 3, 7, 11], [1, 2, 5, 9]]])
    Ks, Vs = torch_twin.gather_kv(K, V, idx)
    for h in range(2):
        for j, p in enumerate(idx[0, h].tolist()):
            assert torch.equal(Ks[0, h, j], K[0, h, p]) and torch.equal(Vs[0, h, j], V[0, h, p])


@pytest.mark.parametrize("dtype", DTYPES)
def test_attention_vs_float64_and_twin(dtype):
    Q, K, V = make_qkv(2, 32, 8, 3000, 64, dtype, seed=5, n_sinks=4, n_outlier=2)
    k = 700
    idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), k)
    o = cpu.attention(Q, K, V, idx)
    ex = cpu.attention_f64(Q, K, V, idx)
    assert (o.double() - ex).abs().max() < 1e-5
    Ks, Vs = torch_twin.gather_kv(K, V, idx)
    tw = torch_twin.fused_softmax_attention(Ks, Vs, Q)
    assert (o - tw).abs().max() < 1e-5


def test_attention_f64_vs_direct_softmax():
    Q, K, V = make_qkv(1, 8, 2, 257, 64, torch.float32, seed=9)
    ex = cpu.dense_f64(Q, K, V)
    Kr = K.double().repeat_interleave(4, dim=1)
    Vr = V.double().repeat_interleave(4, dim=1)
    p = torch.softmax(torch.einsum("bhd,bhnd->bhn", Q.double(), Kr) / 8.0, dim=-1)
    ref = torch.einsum("bhn,bhnd->bhd", p, Vr)
    assert (ex - ref).abs().max() < 1e-12
    # selecting every row equals the dense result
    idx = torch.arange(257, dtype=torch.int32).expand(1, 8, 257).contiguous()
    assert (cpu.attention_f64(Q, K, V, idx) - ex).abs().max() < 1e-12


def test_k_near_full_matches_bruteforce():
    # test_qaxis_topk_reference.py:119-135 (k = N-1 drops one key)
    Q, K, V = make_qkv(1, 2, 2, 32, 64, torch.bfloat16, seed=42)
    r = cpu.sparse_decode(Q, K, V, 31)
    full = cpu.dense_f64(Q, K, V)
    assert (r["out"].double() - full).abs().max() < 0.05


def test_degenerate_raises():
    # test_qaxis_topk_reference.py:61-74
    Q, K, V = make_qkv(1, 4, 2, 16, 32, torch.bfloat16, seed=0)
    with pytest.raises(ValueError, match="caller must dispatch to SDPA"):
        cpu.sparse_decode(Q, K, V, 16)


@pytest.mark.parametrize("dtype", DTYPES)
def test_pipeline_vs_twin(dtype):
    Q, K, V = make_qkv(1, 32, 8, 4096, 64, dtype, seed=0, n_sinks=4, n_outlier=2)
    a = cpu.sparse_decode(Q, K, V, 615)
    b = torch_twin.sparse_decode(Q, K, V, 615)
    assert torch.equal(a["u"], b["u"])
    assert torch.equal(a["scores"].view(torch.int16), b["scores"].view(torch.int16))
    assert torch.equal(a["idx"], b["idx"])
    assert (a["out_f32"] - b["out_f32"]).abs().max() < 1e-5


# --------------------------------------------------------------- configs

def test_k_ceil_configs():
    assert [CONFIGS[c].k for c in ("C1", "C2", "C4a", "C4b", "C4c", "C5")] == \
        [615, 4916, 6554, 19661, 39322, 6554]
    assert k_ceil(100, 0.5) == 50


def test_c1_inputs_shape_and_sinks():
    cfg = CONFIGS["C1"]
    Q, K, V = make_inputs(cfg, seed=0)
    assert Q.shape == (1, 32, 64) and K.shape == (1, 8, 4096, 64) and Q.dtype == torch.float32
    # sinks rank at the top of the projection onto the mean query direction
    qm = Q.view(1, 8, 4, 64).sum(2)
    u = qm / qm.norm(dim=-1, keepdim=True)
    proj = torch.einsum("bgnd,bgd->bgn", K, u)
    top4 = proj.topk(4, dim=-1).indices.sort(dim=-1).values
    assert (top4 == torch.arange(4)).all()
