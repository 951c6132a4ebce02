"""Pin the rank-local oracle (oracle_rank_local_f64) and the caller-side sort
helpers before using them as the checker of the HIP rank-local kernel.

Independent checks:
  * the reference's CPU path restated with its own torch calls
    (oracle/torch_twin.rank_local_fwd, rank_local_fwd_torch.py:21-113);
  * the reference's known answers: a window covering every key equals dense
    softmax attention (test_decode_shape_correctness.py:99-124); a window of
    one key returns that key's value row;
  * permutation equivariance of the query rows (test_permutation_equivariance.py);
  * brute force on tiny inputs (plain Python loops in float64);
  * the sort bookkeeping's defining properties (r_center is the insertion
    rank, non-decreasing in sorted-query order; gather/scatter invert).
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import cpu, torch_twin
from dcr_attention_amd.kernel import sort_helpers as sh


def _inputs(B, H, Nq, Nkv, D, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(B, H, Nq, D, generator=g).to(dtype)
    K = torch.randn(B, H, Nkv, D, generator=g).to(dtype)
    V = torch.randn(B, H, Nkv, D, generator=g).to(dtype)
    axis = torch.randn(D, generator=g)
    return Q, K, V, axis / axis.norm()


def _sorted(Q, K, V, axis):
    idx = sh.prepare_sort_indices(Q.float(), K.float(), axis)
    return (sh.gather_by_sort_idx(Q, idx.sort_idx_q), sh.gather_by_sort_idx(K, idx.sort_idx_k),
            sh.gather_by_sort_idx(V, idx.sort_idx_k), idx)


@pytest.mark.parametrize("Nq,Nkv,D,k", [(128, 128, 32, 16), (128, 128, 64, 64), (64, 64, 128, 256),
                                        (1, 512, 64, 16), (1, 512, 64, 64), (1, 2048, 128, 256)])
def test_oracle_matches_reference_torch_path_fp32(Nq, Nkv, D, k):
    Q, K, V, axis = _inputs(1, 2, Nq, Nkv, D, torch.float32, seed=Nq + D + k)
    if Nq == Nkv:
        Qs, Ks, Vs, idx = _sorted(Q, K, V, axis)
        rc = idx.r_center
    else:
        Qs, Ks, Vs = Q, K, V
        rc = torch.randint(0, Nkv, (1, 2, Nq), generator=torch.Generator().manual_seed(k))
    o64, l64 = cpu.rank_local_f64(Qs, Ks, Vs, rc, k)
    ot, lt = torch_twin.rank_local_fwd(Qs, Ks, Vs, rc, k)
    assert (ot.double() - o64).abs().max().item() <= 2e-6
    assert (lt.double() - l64).abs().max().item() <= 2e-6


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_oracle_matches_reference_torch_path_half(dtype):
    Q, K, V, axis = _inputs(1, 2, 256, 256, 64, dtype, seed=3)
    Qs, Ks, Vs, idx = _sorted(Q, K, V, axis)
    o64, l64 = cpu.rank_local_f64(Qs, Ks, Vs, idx.r_center, 64)
    ot, lt = torch_twin.rank_local_fwd(Qs, Ks, Vs, idx.r_center, 64)
    # the twin rounds its output to the input dtype once
    ulp = torch.ldexp(torch.ones_like(o64), torch.frexp(o64)[1] - (11 if dtype == torch.float16 else 8))
    if dtype == torch.float16:
        ulp = ulp.clamp(min=2.0 ** -24)   # fp16 subnormal spacing
    # one output ulp, plus the twin's fp32 error (relative to the summed
    # terms, not to a small result)
    assert ((ot.double() - o64).abs() <= ulp + 2e-7).all()
    assert (lt.double() - l64).abs().max().item() <= 2e-6


def test_full_window_equals_dense_attention():
    # test_decode_shape_correctness.py:99-124: k_window = 2 * N_kv covers every key.
    Q, K, V, _ = _inputs(1, 2, 1, 300, 64, torch.float32, seed=5)
    rc = torch.tensor([[[7], [299]]], dtype=torch.int32)
    o64, l64 = cpu.rank_local_f64(Q, K, V, rc, 2 * 300)
    s = torch.einsum("bhid,bhjd->bhij", Q.double(), K.double()) / math.sqrt(64)
    dense = torch.einsum("bhij,bhjd->bhid", torch.softmax(s, dim=-1), V.double())
    assert (o64 - dense).abs().max().item() <= 1e-12
    assert (l64 - torch.logsumexp(s, dim=-1)).abs().max().item() <= 1e-12


def test_window_of_one_key_returns_its_value_row():
    Q, K, V, _ = _inputs(1, 1, 5, 40, 32, torch.float32, seed=6)
    rc = torch.tensor([[[0, 3, 17, 39, 39]]], dtype=torch.int32)
    o64, l64 = cpu.rank_local_f64(Q, K, V, rc, 1)   # half = 0
    for i, r in enumerate(rc[0, 0].tolist()):
        assert torch.equal(o64[0, 0, i], V[0, 0, r].double())
        lg = float((Q[0, 0, i].double() * K[0, 0, r].double()).sum()) / math.sqrt(32)
        assert abs(float(l64[0, 0, i]) - lg) <= 1e-12


def test_brute_force_tiny():
    Q, K, V, _ = _inputs(1, 1, 4, 9, 4, torch.float32, seed=7)
    rc = torch.tensor([[[0, 2, 5, 8]]], dtype=torch.int32)
    k_window, scale = 5, 0.37
    o64, l64 = cpu.rank_local_f64(Q, K, V, rc, k_window, scale=scale)
    for i in range(4):
        r = int(rc[0, 0, i])
        js = [j for j in range(9) if abs(j - r) <= k_window // 2]
        lg = [scale * sum(float(Q[0, 0, i, d]) * float(K[0, 0, j, d]) for d in range(4)) for j in js]
        mx = max(lg)
        w = [math.exp(x - mx) for x in lg]
        tot = sum(w)
        for d in range(4):
            ref = sum(wj * float(V[0, 0, j, d]) for wj, j in zip(w, js)) / tot
            assert abs(float(o64[0, 0, i, d]) - ref) <= 1e-12
        assert abs(float(l64[0, 0, i]) - (mx + math.log(tot))) <= 1e-12


def test_query_permutation_equivariance():
    Q, K, V, _ = _inputs(1, 2, 32, 64, 32, torch.float32, seed=8)
    rc = torch.randint(0, 64, (1, 2, 32), generator=torch.Generator().manual_seed(1), dtype=torch.int32)
    perm = torch.randperm(32, generator=torch.Generator().manual_seed(2))
    o1, l1 = cpu.rank_local_f64(Q, K, V, rc, 16)
    o2, l2 = cpu.rank_local_f64(Q[:, :, perm], K, V, rc[:, :, perm], 16)
    assert torch.equal(o1[:, :, perm], o2) and torch.equal(l1[:, :, perm], l2)


def test_out_of_range_centres_follow_the_reference_mask():
    """r_center is used as given (rank_local_fwd_torch.py:84-87): r = Nkv keeps
    half_k keys, r = -2 keeps half_k - 1, and a window past every row is empty,
    giving O = 0 and LSE = -inf (the reference's nan_to_num / empty-row case)."""
    Nkv, k = 50, 8                                     # half_k = 4
    Q, K, V, _ = _inputs(1, 1, 8, Nkv, 32, torch.float32, seed=9)
    rc = torch.tensor([[[-7, -2, 0, 49, 50, 53, 60, 2**31 - 1]]], dtype=torch.int32)
    o64, l64 = cpu.rank_local_f64(Q, K, V, rc, k)
    ot, lt = torch_twin.rank_local_fwd(Q, K, V, rc, k)
    assert (o64 - ot.double()).abs().max().item() <= 1e-5
    finite = torch.isfinite(lt)
    assert torch.equal(finite, torch.isfinite(l64))
    assert (l64[finite] - lt[finite].double()).abs().max().item() <= 1e-5
    for i in (0, 6, 7):                                # empty windows
        assert (o64[0, 0, i] == 0).all() and l64[0, 0, i].item() == -math.inf
    # r = Nkv: rows Nkv-4 .. Nkv-1 (half_k of them) -- the window of r = Nkv - 1
    # minus its lowest row, not the window of r = Nkv - 1 itself
    o_a, _ = cpu.rank_local_f64(Q[:, :, 4:5], K[:, :, 46:], V[:, :, 46:],
                                torch.tensor([[[4]]], dtype=torch.int32), 100)
    assert (o64[0, 0, 4] - o_a[0, 0, 0]).abs().max().item() <= 1e-12


def test_sort_bookkeeping_definitions():
    Q, K, V, axis = _inputs(2, 3, 40, 40, 16, torch.float32, seed=10)
    idx = sh.prepare_sort_indices(Q, K, axis)
    zq = torch.einsum("bhnd,d->bhn", Q, axis)
    zk = torch.einsum("bhnd,d->bhn", K, axis)
    for b in range(2):
        for h in range(3):
            zk_sorted = zk[b, h, idx.sort_idx_k[b, h]]
            assert (zk_sorted[1:] >= zk_sorted[:-1]).all()
            assert torch.equal(idx.sort_idx_k[b, h][idx.rank_of_k[b, h]], torch.arange(40))
            rc = idx.r_center[b, h]
            assert (rc[1:] >= rc[:-1]).all()                 # non-decreasing in sorted-Q order
            for t in range(40):
                zq_t = float(zq[b, h, idx.sort_idx_q[b, h, t]])
                count = int((zk[b, h] < zq_t).sum())
                assert int(rc[t]) == min(count, 39)
    X = torch.randn(2, 3, 40, 16)
    Xs = sh.gather_by_sort_idx(X, idx.sort_idx_q)
    assert torch.equal(sh.scatter_by_inv_perm(Xs, idx.inv_q_perm), X)


def test_shim_validation_errors():
    from dcr_attention_amd.kernel.hip.rank_local_fwd import rank_local_fwd_hip
    Q, K, V, _ = _inputs(1, 2, 8, 8, 32, torch.float32)
    rc = torch.zeros(1, 2, 8, dtype=torch.int32)
    with pytest.raises(RuntimeError):
        rank_local_fwd_hip(Q, K, V, None, rc, 4)          # host tensors
    if torch.cuda.is_available():
        d = torch.device("cuda")
        with pytest.raises(ValueError):
            rank_local_fwd_hip(Q.to(d), K.to(d), V[:, :, :4].to(d), None, rc.to(d), 4)
        with pytest.raises(ValueError):
            rank_local_fwd_hip(Q.to(d), K.to(d), V.to(d), None, rc[:, :, :3].to(d), 4)
