"""The sparse decode launch sequences against each other and the CPU oracle,
through the C ABI:

* DCR_PATH_AUTO (default) / DCR_PATH_CLASSIC: score, select (index lists),
  index-list attention;
* DCR_PATH_FUSED: the whole step in one launch (csrc/fused.hip) where the
  shape allows it;
* DCR_PATH_UNION: score, select (selection in closed form), union-gather
  attention (csrc/attn.hip union_attn_kernel).

Every shape here is one the one-launch path serves (fp16/bf16, D 64/128, n_rep
1/2/4, B*Hkv a multiple of 8 with B*Hkv/8 dividing 32).  For each: indices
bit-identical across the paths and to the oracle (ties toward the lower index,
including ties that straddle workgroups' position ranges), outputs within the
path's tolerance of the float64 oracle and within fp32 rounding of each other,
the same output with and without the index list, and the one-launch path's
barrier error word still 0.
"""
from __future__ import annotations

import pytest
import torch

from oracle import cpu
from dcr_attention_amd import _lib
from dcr_attention_amd.kernel.hip import topk_qaxis_attention
from dcr_attention_amd.synthetic import make_qkv

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float16: 2e-3, torch.bfloat16: 5e-3}
PATHS = {"classic": _lib.PATH_CLASSIC, "fused": _lib.PATH_FUSED, "union": _lib.PATH_UNION}


def _run_paths(Q, K, V, k):
    """{path: (O with indices requested, indices, O without)}."""
    Qd, Kd, Vd = Q.to(DEV), K.to(DEV), V.to(DEV)
    out = {}
    prev = _lib.set_sparse_path(_lib.PATH_CLASSIC)
    try:
        for name, code in PATHS.items():
            _lib.set_sparse_path(code)
            o, i = topk_qaxis_attention(Qd, Kd, Vd, k, return_indices=True)
            o2 = topk_qaxis_attention(Qd, Kd, Vd, k)
            out[name] = (o, i, o2)
    finally:
        _lib.set_sparse_path(prev)
    torch.cuda.synchronize()
    return out


def _check(Q, K, V, k, dtype):
    print(f"paths: B={Q.shape[0]} H={Q.shape[1]} Hkv={K.shape[1]} N={K.shape[2]} "
          f"D={K.shape[3]} k={k} {dtype}", flush=True)
    B, H, D = Q.shape
    Hkv, N = K.shape[1], K.shape[2]
    lib = _lib.load()
    prev = _lib.set_sparse_path(_lib.PATH_FUSED)
    try:
        launches = lib.dcr_sparse_decode_launches(B, H, Hkv, N, D, k, _lib.DTYPE_CODE[dtype])
    finally:
        _lib.set_sparse_path(prev)
    assert launches == 1, "shape expected to run in one launch under DCR_PATH_FUSED"
    assert _lib.fused_errors(clear=True) == 0
    res = _run_paths(Q, K, V, k)
    assert _lib.fused_errors() == 0, "a phase barrier of the one-launch path gave up"
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), k)
    for name, (_, i, _) in res.items():
        assert torch.equal(i.cpu(), ref_idx), f"{name}: indices differ from the oracle"
    ref = cpu.attention_f64(Q, K, V, ref_idx)
    tol = torch.full_like(ref, TOL[dtype])
    if dtype == torch.bfloat16:
        tol = torch.maximum(tol, torch.ldexp(torch.ones_like(ref), torch.frexp(ref)[1] - 8))
    for name, (o, _, o2) in res.items():
        for x in (o, o2):
            diff = (x.double().cpu() - ref).abs()
            assert (diff <= tol).all(), f"{name}: max|O - f64| = {diff.max().item():.3e}"
            cos = torch.nn.functional.cosine_similarity(x.double().cpu().flatten(1), ref.flatten(1), dim=-1)
            assert cos.min().item() >= 0.9999
        assert torch.equal(o, o2), f"{name}: output depends on whether the indices are written"
    # the paths differ only in fp32 summation order and softmax reference points
    one_ulp = torch.ldexp(torch.ones_like(ref), torch.frexp(ref)[1] - (11 if dtype == torch.float16 else 8))
    bound = torch.maximum(one_ulp, torch.full_like(ref, 1e-4))
    base = res["classic"][0].double().cpu()
    for name in ("fused", "union"):
        d = (res[name][0].double().cpu() - base).abs()
        assert (d <= bound).all(), f"{name} vs classic: max diff {d.max().item():.3e}"


@pytest.mark.parametrize("B,Hkv,n_rep,N,D,k,dtype", [
    (4, 8, 4, 32768, 64, 4916, torch.float16),     # C2: 4 groups per XCD, 8 chunks per group
    (1, 8, 4, 4096, 64, 615, torch.float16),       # one group per XCD, 32 chunks of 128 positions
    (1, 8, 4, 131072, 64, 39322, torch.float16),   # C4c shape, 32 chunks of 4096
    (2, 8, 4, 20000, 64, 3000, torch.bfloat16),    # ragged N, 16 chunks
    (8, 4, 4, 9000, 64, 1351, torch.float16),      # 32 groups from 8 batches x 4 KV heads
    (16, 8, 4, 8192, 64, 1229, torch.float16),     # 128 groups: 2 chunks per group
    (32, 8, 4, 3000, 64, 450, torch.bfloat16),     # 256 groups: one chunk per group
    (1, 8, 1, 5000, 64, 750, torch.float16),       # n_rep 1
    (2, 8, 2, 7777, 64, 1000, torch.bfloat16),     # n_rep 2, odd N
    (1, 8, 4, 500, 64, 100, torch.float16),        # N below 32 * 64: most chunks empty
    (4, 8, 4, 8192, 128, 820, torch.bfloat16),     # D = 128
    (2, 8, 2, 4100, 128, 600, torch.float16),      # D = 128, n_rep 2
])
def test_fused_matches_classic_and_oracle(B, Hkv, n_rep, N, D, k, dtype):
    Q, K, V = make_qkv(B, Hkv * n_rep, Hkv, N, D, dtype, seed=N + k + D, n_sinks=4, n_outlier=2)
    _check(Q, K, V, k, dtype)


@pytest.mark.parametrize("case", range(12))
def test_paths_random_shapes(case):
    """Seeded random shapes of the one-launch family (B*Hkv = 8B with B | 32,
    n_rep 1/2/4, D 64/128, fp16/bf16), ragged N and k from 1 to N - 1: the
    three paths against each other and the oracle."""
    import math
    import random
    r = random.Random(3000 + case)
    B = r.choice([1, 2, 4, 8, 16, 32])
    n_rep = r.choice([1, 2, 4])
    D = r.choice([64, 128])
    dtype = r.choice([torch.float16, torch.bfloat16])
    n_max = max(64, 200000 // B)
    N = max(2, int(round(math.exp(r.uniform(math.log(64), math.log(n_max))))))
    k = r.choice([1, N - 1, max(1, N // 10), r.randint(1, N - 1)])
    Q, K, V = make_qkv(B, 8 * n_rep, 8, N, D, dtype, seed=case, n_sinks=2, n_outlier=1)
    _check(Q, K, V, k, dtype)


def test_fused_c5_full_size():
    """C5: B=16, N=65536, D=128, bf16, k=6554 (2 chunks of 32768 per group, 16
    sub-chunks per workgroup)."""
    B, Hkv, N, D, k = 16, 8, 65536, 128, 6554
    Qd, Kd, Vd = make_qkv(B, 32, Hkv, N, D, torch.bfloat16, seed=5, device=DEV, n_sinks=4)
    _check(Qd.cpu(), Kd.cpu(), Vd.cpu(), k, torch.bfloat16)


@pytest.mark.parametrize("k", [1, 77, 2000, 4095])
def test_fused_ties_straddle_chunks(k):
    """Keys with many equal scores: all K rows of a group equal in blocks, so
    the k-th score is shared by hundreds of positions spread over several
    workgroups' chunks, and the tie quota must go to the lowest positions."""
    B, Hkv, n_rep, N, D = 1, 8, 4, 4096, 64
    Q, K, V = make_qkv(B, Hkv * n_rep, Hkv, N, D, torch.float16, seed=k)
    g = torch.Generator().manual_seed(k)
    base = torch.randn(B, Hkv, 16, D, generator=g).to(torch.float16)
    K = base.repeat_interleave(N // 16, dim=2)[:, :, torch.randperm(N, generator=g)]
    _check(Q, K.contiguous(), V, k, torch.float16)


@pytest.fixture(params=["classic", "fused", "union"])
def path(request):
    prev = _lib.set_sparse_path(PATHS[request.param])
    yield request.param
    _lib.set_sparse_path(prev)


def test_strided_cache_and_repeated_calls(path):
    """A preallocated cache (row stride between KV heads > N) and repeated
    calls on one workspace (the one-launch path's barrier tags advance per
    launch; the merge tickets are cleared by each select launch)."""
    B, Hkv, n_rep, N, N_max, D, k = 4, 8, 4, 6000, 8192, 64, 900
    Q, K, V = make_qkv(B, Hkv * n_rep, Hkv, N, D, torch.float16, seed=3, n_sinks=4)
    Kc = torch.zeros(B, Hkv, N_max, D, dtype=torch.float16, device=DEV)
    Vc = torch.zeros_like(Kc)
    Kc[:, :, :N] = K.to(DEV)
    Vc[:, :, :N] = V.to(DEV)
    assert _lib.fused_errors(clear=True) == 0
    first = topk_qaxis_attention(Q.to(DEV), Kc[:, :, :N], Vc[:, :, :N], k)
    for _ in range(20):
        again = topk_qaxis_attention(Q.to(DEV), Kc[:, :, :N], Vc[:, :, :N], k)
        assert torch.equal(again, first)
    assert _lib.fused_errors() == 0
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), k)
    assert (first.double().cpu() - cpu.attention_f64(Q, K, V, ref_idx)).abs().max().item() <= 2e-3


def test_graph_replays_match_eager(path):
    """The sparse decode step captured in a HIP graph (for the one-launch
    path the host-side nonce is frozen at capture, and the per-XCD launch
    counter in the workspace still advances per replay).  Each replay, on new
    query values written between replays, must equal the eager call on the
    same values."""
    B, Hkv, n_rep, N, D, k = 4, 8, 4, 8192, 64, 1229
    Q, K, V = make_qkv(B, Hkv * n_rep, Hkv, N, D, torch.float16, seed=11, n_sinks=4)
    Qd, Kd, Vd = Q.to(DEV), K.to(DEV), V.to(DEV)
    assert _lib.fused_errors(clear=True) == 0
    topk_qaxis_attention(Qd, Kd, Vd, k)                     # load the library before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        O, idx = topk_qaxis_attention(Qd, Kd, Vd, k, return_indices=True)
    gen = torch.Generator().manual_seed(12)
    for rep in range(5):
        Qd.copy_(torch.randn(B, Hkv * n_rep, D, generator=gen).to(torch.float16))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        o_e, i_e = topk_qaxis_attention(Qd, Kd, Vd, k, return_indices=True)
        torch.cuda.synchronize()
        print(f"{path}: graph replay {rep}", flush=True)
        assert torch.equal(idx, i_e) and torch.equal(O, o_e)
    assert _lib.fused_errors() == 0
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Qd.cpu())), k)
    assert torch.equal(idx.cpu(), ref_idx)


def test_launch_count_by_shape():
    lib = _lib.load()
    f16, bf16, f32 = (_lib.DTYPE_CODE[t] for t in (torch.float16, torch.bfloat16, torch.float32))
    prev = _lib.set_sparse_path(_lib.PATH_FUSED)
    try:
        assert lib.dcr_sparse_decode_launches(4, 32, 8, 32768, 64, 4916, f16) == 1      # C2
        assert lib.dcr_sparse_decode_launches(16, 32, 8, 65536, 128, 6554, bf16) == 1   # C5
        assert lib.dcr_sparse_decode_launches(4, 32, 8, 32768, 64, 4916, f32) == 3      # fp32
        assert lib.dcr_sparse_decode_launches(1, 32, 4, 32768, 64, 4916, f16) == 3      # 4 groups
        assert lib.dcr_sparse_decode_launches(3, 32, 8, 32768, 64, 4916, f16) == 3      # 24 groups
        assert lib.dcr_sparse_decode_launches(1, 64, 8, 32768, 64, 4916, f16) == 3      # n_rep 8
        assert lib.dcr_sparse_decode_launches(1, 32, 8, 32768, 96, 4916, f16) < 0       # D = 96: rejected
        for path in (_lib.PATH_AUTO, _lib.PATH_CLASSIC, _lib.PATH_UNION):
            _lib.set_sparse_path(path)
            assert lib.dcr_sparse_decode_launches(4, 32, 8, 32768, 64, 4916, f16) == 3
    finally:
        _lib.set_sparse_path(prev)


@pytest.mark.parametrize("B,Hkv,n_rep,N,D,k,dtype", [
    (4, 8, 4, 32768, 64, 4916, torch.float16),      # C2 (MFMA chain by default)
    (2, 8, 8, 9000, 64, 1351, torch.bfloat16),      # two 4-head chains
    (2, 8, 4, 8192, 128, 820, torch.bfloat16),      # D = 128, u read from LDS
    (1, 8, 8, 4096, 128, 615, torch.float16),       # VALU either way
    (4, 8, 4, 40000, 64, 6000, torch.float16),      # grid capped at the resident workgroups
])
def test_score_forms_bit_identical(B, Hkv, n_rep, N, D, k, dtype):
    """The MFMA and VALU forms of the score pass (dcr_set_score_form) give the
    same score bits, hence the same indices and the same output bits."""
    Q, K, V = make_qkv(B, Hkv * n_rep, Hkv, N, D, dtype, seed=N + D, device=DEV, n_sinks=4, n_outlier=2)
    outs = {}
    prev = _lib.set_score_form(_lib.SCORE_AUTO)
    try:
        for form in (_lib.SCORE_AUTO, _lib.SCORE_VALU):
            _lib.set_score_form(form)
            outs[form] = topk_qaxis_attention(Q, K, V, k, return_indices=True)
    finally:
        _lib.set_score_form(prev)
    torch.cuda.synchronize()
    print(f"score forms: B={B} n_rep={n_rep} N={N} D={D} {dtype}", flush=True)
    assert torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][0], outs[1][0])
    ref_idx = cpu.topk(cpu.scores(K.cpu(), cpu.compute_uq(Q.cpu())), k)
    assert torch.equal(outs[1][1].cpu(), ref_idx)
