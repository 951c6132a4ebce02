"""HIP path vs the CPU oracle on the same seeded inputs (MI355X).

Bar (the path's parity contract):
  * u_Q, bf16 scores and top-K indices: bit-exact (ties toward lower index);
  * attention output vs the float64 closed form over the same indices:
      fp32  max|diff| <= 1e-5
      fp16  max|diff| <= 2e-3
      bf16  |diff| <= max(5e-3, one bf16 ulp of the exact value) per element
            (5e-3 is the reference's gate, kernel_spec.md section 5.1.2; a bf16
            output of magnitude >= 1 already carries up to half an ulp =
            3.9e-3 of rounding, so the ulp term covers sink-dominated heads)
    plus cosine >= 0.9999 and RMSE^2 <= 1e-6 everywhere.
Sizes go up to the full C2 (B=4, N=32768) and C4 (N=131072) shapes, and rows of
262144 and 1048576 positions for the chunked select; the
oracle finishes those in seconds.
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import cpu
from dcr_attention_amd.kernel.hip import (compute_u_Q, dense_decode_attention,
                                          fused_topk_attention, topk_pass1_projection,
                                          topk_pass2_select, topk_qaxis_attention,
                                          topk_qaxis_select)
from dcr_attention_amd.synthetic import CONFIGS, make_inputs, make_qkv

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 5e-3}


def _dev(*ts):
    return [t.to(DEV) for t in ts]


def _assert_close_out(out, ref64, dtype):
    o = out.detach().double().cpu()
    diff = (o - ref64).abs()
    tol = torch.full_like(ref64, TOL[dtype])
    if dtype == torch.bfloat16:
        ulp = torch.ldexp(torch.ones_like(ref64), torch.frexp(ref64)[1] - 8)
        tol = torch.maximum(tol, ulp)
    bad = diff > tol
    assert not bad.any(), f"max|diff|={diff.max().item():.3e}, {int(bad.sum())} elements over tolerance"
    # mean squared error: 1e-6, or twice what rounding the exact result to the
    # output dtype costs by itself (bf16 outputs of magnitude ~1, as sink-
    # dominated heads give, carry ~1e-6 of it), whichever is larger
    rounding2 = ((ref64.to(dtype).double() - ref64) ** 2).mean().item()
    mse = (diff ** 2).mean().item()
    assert mse <= max(1e-6, 2.0 * rounding2), f"mse={mse:.3e}, rounding alone {rounding2:.3e}"
    cos = torch.nn.functional.cosine_similarity(o.flatten(1), ref64.flatten(1), dim=-1)
    assert cos.min().item() >= 0.9999
    assert torch.isfinite(o).all()


# --------------------------------------------------------------------- u_Q

@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128, 100])   # 100: the runtime-D kernel with its scalar tail
def test_uq_bitexact(dtype, D):
    Q, _, _ = make_qkv(3, 32, 8, 1, D, dtype, seed=D + 1)
    Q[0, 5] = 0  # zero query: eps guard
    u = compute_u_Q(Q.to(DEV))
    assert torch.equal(u.cpu(), cpu.compute_uq(Q))


# ------------------------------------------------------------------ scores

@pytest.mark.parametrize("dtype,D,n_rep,N,B", [
    (torch.float32, 64, 4, 4096, 1),     # C1
    (torch.float16, 64, 4, 1000, 2),
    (torch.bfloat16, 64, 4, 63, 1),
    (torch.bfloat16, 64, 4, 65, 1),
    (torch.bfloat16, 64, 4, 2000, 4),
    (torch.float16, 64, 1, 500, 1),
    (torch.float16, 64, 2, 777, 1),
    (torch.float16, 64, 8, 513, 1),
    (torch.bfloat16, 128, 4, 333, 2),
    (torch.float16, 128, 8, 1025, 1),
    (torch.float32, 128, 2, 300, 1),
    # D = 128 reads u from LDS inside the MFMA chain: every n_rep it serves
    (torch.float16, 128, 1, 4100, 1),
    (torch.bfloat16, 128, 2, 2049, 1),
    (torch.float16, 128, 4, 8192, 2),
])
def test_scores_bitexact(dtype, D, n_rep, N, B):
    Hkv = 8 if n_rep <= 4 else 4
    Q, K, _ = make_qkv(B, Hkv * n_rep, Hkv, N, D, dtype, seed=N, n_sinks=4, n_outlier=2)
    u = cpu.compute_uq(Q)
    s = topk_pass1_projection(K.to(DEV), u.to(DEV))
    assert s.dtype == torch.bfloat16 and s.shape == (B, Hkv * n_rep, N)
    ref = cpu.scores(K, u)
    assert torch.equal(s.cpu().view(torch.int16), ref.view(torch.int16))


# ------------------------------------------------------------------ select

def _scores(rows, N, seed, kind):
    g = torch.Generator().manual_seed(seed)
    if kind == "randn":
        s = torch.randn(rows, N, generator=g)
    elif kind == "ties":  # few distinct values: the tie quota decides membership
        s = torch.randint(-6, 7, (rows, N), generator=g).float() / 4
    else:  # "special": zeros of both signs, inf, nan sprinkled in
        s = torch.randn(rows, N, generator=g)
        s[:, ::11] = 0.0
        s[:, 1::13] = -0.0
        s[:, 2::97] = float("inf")
        s[:, 3::101] = float("-inf")
        s[:, 4::211] = float("nan")
    return s.to(torch.bfloat16)


@pytest.mark.parametrize("N,k,kind", [
    (8, 3, "randn"), (100, 1, "randn"), (100, 99, "ties"), (1000, 300, "ties"),
    (4096, 615, "randn"), (4096, 614, "special"), (8193, 4000, "ties"),
    (32768, 4916, "randn"), (32768, 4916, "ties"), (32768, 32767, "special"),
    (131072, 6554, "randn"), (131072, 39322, "ties"), (131071, 19661, "special"),
    # odd and just-past-a-multiple row lengths (keys per thread not a multiple of 8)
    (33, 5, "ties"), (1025, 100, "special"), (32769, 4916, "randn"), (32770, 4916, "ties"),
    (65537, 9831, "ties"), (98305, 14746, "randn"),
])
def test_select_exact(N, k, kind):
    rows = 4 if N > 50000 else 16
    s = _scores(rows, N, seed=N + k, kind=kind)
    idx = topk_pass2_select(s.to(DEV), k)
    assert idx.dtype == torch.int32 and idx.shape == (rows, k)
    assert torch.equal(idx.cpu(), cpu.topk(s, k))


@pytest.mark.parametrize("rows,N,k,kind", [
    (128, 32768, 4916, "randn"),     # one workgroup per row
    (128, 131072, 19661, "ties"),
    (32, 131072, 6554, "randn"),     # rows split into chunks over two launches
    (32, 131072, 39322, "special"),
    (8, 100000, 15000, "ties"),
    (1, 131072, 19661, "randn"),
    (64, 32769, 4916, "ties"),
    # rows longer than one workgroup's 131072 positions: always chunked
    (2, 262144, 39322, "randn"),
    (128, 196609, 29492, "ties"),
    (1, 1048576, 157287, "special"),
    # one workgroup per row at every keys-per-thread size (8/16/24/32/40/48/64/96/128;
    # 40 and above use 64-bit masks): C5's rows are 512 of 65536 (64 per thread)
    (128, 8000, 1200, "special"),
    (128, 16000, 2400, "ties"),
    (128, 20000, 3000, "ties"),
    (128, 40000, 6000, "special"),
    (128, 49152, 7373, "ties"),
    (128, 65536, 6554, "ties"),
    (128, 65536, 6554, "special"),
    (128, 98304, 14746, "special"),
    (128, 98304, 9831, "ties"),
    # up to 128 rows the rows above take two workgroups each (keys per thread <= 64);
    # more rows take one workgroup per row at the same sizes
    (256, 8000, 1200, "special"),
    (256, 20000, 3000, "ties"),
    (256, 32768, 4916, "ties"),
    (256, 40000, 6000, "special"),
    (256, 65536, 6554, "ties"),
    # two workgroups per row with a row length whose thread count is not a multiple of 128
    # (the decode caller's growing cache: N = 32770 at 40 keys per thread)
    (128, 32770, 4916, "ties"),
    (16, 32833, 4926, "special"),
    (100, 9000, 1350, "randn"),
])
def test_select_paths(rows, N, k, kind):
    s = _scores(rows, N, seed=rows + N + k, kind=kind)
    idx = topk_pass2_select(s.to(DEV), k)
    assert torch.equal(idx.cpu(), cpu.topk(s, k))


def test_select_all_equal_picks_lowest_indices():
    s = torch.ones(2, 3, 5000, dtype=torch.bfloat16, device=DEV)
    idx = topk_pass2_select(s, 777)
    assert torch.equal(idx.cpu(), torch.arange(777, dtype=torch.int32).expand(2, 3, 777))


@pytest.mark.parametrize("k", [100, 16383, 16384, 16385, 20000, 32767])
def test_select_two_workgroup_halves_all_ties(k):
    """Rows of 32768 equal keys take the two-workgroups-per-row select: each half
    emits its share of the tie quota, the second at the first half's count."""
    s = torch.ones(4, 32768, dtype=torch.bfloat16, device=DEV)
    idx = topk_pass2_select(s, k)
    assert torch.equal(idx.cpu(), torch.arange(k, dtype=torch.int32).expand(4, k))


@pytest.mark.parametrize("k", [16384, 16385, 20000, 30000])
def test_select_two_workgroup_halves_offsets(k):
    """The second half holds every key above the threshold and the first half the
    ties: the first half's output (the lowest tied indices) precedes the second's."""
    s = torch.ones(8, 32768, dtype=torch.bfloat16)
    s[:, 16384:] = 2.0
    s[1, 100] = 3.0  # one row with a key above both halves' values in the first half
    idx = topk_pass2_select(s.to(DEV), k)
    assert torch.equal(idx.cpu(), cpu.topk(s, k))


def test_select_structure():
    # test_pass2_topk.py:49-81: int32, in range, strictly ascending, unique
    s = _scores(32, 800, seed=3, kind="ties").view(1, 32, 800)
    idx = topk_pass2_select(s.to(DEV), 400).cpu()
    assert idx.min() >= 0 and idx.max() < 800
    assert (idx[..., 1:] > idx[..., :-1]).all()


# ------------------------------------------------- select from the pipeline

@pytest.mark.parametrize("name,B", [("C1", None), ("C2", 1), ("C4b", None)])
def test_qaxis_select_bitexact(name, B):
    cfg = CONFIGS[name]
    Q, K, _ = make_inputs(cfg, seed=0, B=B)
    idx = topk_qaxis_select(Q.to(DEV), K.to(DEV), cfg.k)
    u = cpu.compute_uq(Q)
    ref = cpu.topk(cpu.scores(K, u), cfg.k)
    assert torch.equal(idx.cpu(), ref)


# --------------------------------------------------------------- attention

@pytest.mark.parametrize("dtype,D,n_rep,N,k,B", [
    (torch.float32, 64, 4, 4096, 615, 1),
    (torch.float16, 64, 4, 2000, 500, 2),
    (torch.bfloat16, 64, 4, 1000, 200, 1),
    (torch.bfloat16, 64, 4, 20000, 10000, 1),   # long k: fp32 state drift (test_m3:111-134)
    (torch.float16, 128, 4, 3000, 301, 1),
    (torch.bfloat16, 128, 8, 1500, 77, 1),
    (torch.float16, 64, 1, 700, 33, 2),
    (torch.float32, 128, 2, 900, 450, 1),
])
def test_attention_given_indices(dtype, D, n_rep, N, k, B):
    Hkv = 8 if n_rep <= 4 else 4
    H = Hkv * n_rep
    Q, K, V = make_qkv(B, H, Hkv, N, D, dtype, seed=k, n_sinks=4, n_outlier=2)
    idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), k)
    out = fused_topk_attention(*_dev(Q, K, V, idx))
    assert out.dtype == dtype and out.shape == (B, H, D)
    _assert_close_out(out, cpu.attention_f64(Q, K, V, idx), dtype)


@pytest.mark.parametrize("name,B", [("C1", None), ("C2", None), ("C4a", None), ("C4b", None),
                                    ("C4c", None), ("C5", 1)])
def test_full_pipeline(name, B):
    cfg = CONFIGS[name]
    print(f"full pipeline {name}: B={cfg.B if B is None else B} N={cfg.N} k={cfg.k}", flush=True)
    Q, K, V = make_inputs(cfg, seed=0, B=B)
    out, idx = topk_qaxis_attention(*_dev(Q, K, V), cfg.k, return_indices=True)
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), cfg.k)
    assert torch.equal(idx.cpu(), ref_idx)
    _assert_close_out(out, cpu.attention_f64(Q, K, V, ref_idx), cfg.dtype)


@pytest.mark.timeout(400)
def test_full_pipeline_c5_full_batch():
    """C5 at its own batch size: B=16, N=65536, D=128, bf16, k=6554 -- 512 rows of
    65536 positions take the one-workgroup-per-row select (64 keys per thread, 64-bit
    masks) and the D=128 score and attention kernels at their full grids.  Inputs are
    drawn on the device (CONFIGS["C5"]'s recipe with the device generator) and copied
    to the host for the oracle."""
    cfg = CONFIGS["C5"]
    print(f"C5 full: B={cfg.B} N={cfg.N} D={cfg.D} k={cfg.k} bf16 (4.3 GB of K/V)", flush=True)
    Qd, Kd, Vd = make_inputs(cfg, seed=0, device=DEV)
    out, idx = topk_qaxis_attention(Qd, Kd, Vd, cfg.k, return_indices=True)
    torch.cuda.synchronize()
    print("C5 full: device done, copying to host", flush=True)
    Q, K, V = Qd.cpu(), Kd.cpu(), Vd.cpu()
    del Kd, Vd
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), cfg.k)
    print("C5 full: oracle indices done", flush=True)
    assert torch.equal(idx.cpu(), ref_idx)
    _assert_close_out(out, cpu.attention_f64(Q, K, V, ref_idx), cfg.dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("qnorm,sinks", [(30.0, 4), (50.0, 4), (40.0, 0)])
def test_large_norm_queries(dtype, qnorm, sinks):
    """Post-RoPE decode queries have norms of 20-50, so logits reach well past 10
    (the sinks' past 100).  The fp16/bf16 path rebuilds its logits from the bf16
    score key plus an 8-bit residual (relative error <= 2^-16 of K.u) and scales
    them by ||q||/sqrt(D), so the absolute logit error grows with ||q||; the
    outputs must still meet the same bar (fp16 2e-3, bf16 max(5e-3, 1 ulp),
    cosine >= 0.9999) against the float64 oracle on the same indices."""
    B, H, Hkv, N, D, k = 2, 32, 8, 32768, 64, 4916
    Q, K, V = make_qkv(B, H, Hkv, N, D, torch.float32, seed=int(qnorm) + sinks, n_sinks=sinks,
                       n_outlier=2)
    Q = Q * (qnorm / Q.norm(dim=-1, keepdim=True))
    Q, K, V = Q.to(dtype), K.to(dtype), V.to(dtype)
    logits = torch.einsum("bgrd,bgnd->bgrn", Q.float().view(B, Hkv, H // Hkv, D), K.float()) / 8.0
    print(f"|q|={qnorm} sinks={sinks} {dtype}: max logit {logits.max().item():.1f}", flush=True)
    out, idx = topk_qaxis_attention(*_dev(Q, K, V), k, return_indices=True)
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), k)
    assert torch.equal(idx.cpu(), ref_idx)
    ref = cpu.attention_f64(Q, K, V, ref_idx)
    diff = out.double().cpu() - ref
    rnd = ref.to(dtype).double() - ref
    print(f"  max|out - f64| = {diff.abs().max().item():.3e} (rounding the exact result alone: "
          f"{rnd.abs().max().item():.3e}); mse {(diff ** 2).mean().item():.3e} "
          f"(rounding alone {(rnd ** 2).mean().item():.3e})", flush=True)
    _assert_close_out(out, ref, dtype)


@pytest.mark.parametrize("dtype,D,n_rep,N,k,B", [
    (torch.float16, 64, 1, 3000, 450, 2),
    (torch.float16, 64, 2, 2049, 308, 1),
    (torch.bfloat16, 64, 8, 4100, 615, 1),
    (torch.float16, 128, 8, 1500, 225, 1),    # u from a separate launch (VALU score variant)
    (torch.float32, 128, 2, 1200, 180, 1),
    (torch.float32, 64, 4, 10001, 1500, 1),
    (torch.float16, 64, 4, 32769, 4916, 1),   # first decode step after a 32K prefill
    (torch.bfloat16, 64, 4, 262145, 39322, 1),  # past the one-workgroup select
    # score grids capped at one resident round of workgroups, the rows left
    # over dealt one tile per wave in turn: one more round for some waves
    # (34816), for every wave (36000), one or two (40000), up to 17 (100003)
    (torch.float16, 64, 4, 34816, 5223, 4),
    (torch.bfloat16, 128, 4, 36000, 5400, 4),
    (torch.float16, 64, 4, 40000, 6000, 4),
    (torch.float16, 64, 4, 100003, 15001, 4),
    (torch.bfloat16, 128, 8, 48000, 7200, 8),  # the VALU kernel (u from a separate launch), 3-4 each
    (torch.float32, 64, 4, 36000, 5400, 4),    # fp32 (one tile in flight per wave, K gathered)
    (torch.float16, 64, 4, 8000, 1200, 40),    # 320 groups: the uncapped grid takes fewer rounds
    # D = 128 (u read from LDS in the fused score kernel), n_rep 1 / 2 / 4
    (torch.float16, 128, 4, 8192, 1229, 2),
    (torch.bfloat16, 128, 1, 3000, 450, 1),
    (torch.float16, 128, 2, 5000, 750, 1),
])
def test_pipeline_shapes(dtype, D, n_rep, N, k, B):
    """Every (dtype, D, n_rep) family of the fused score kernel, ragged N."""
    Hkv = 8 if n_rep <= 4 else 4
    Q, K, V = make_qkv(B, Hkv * n_rep, Hkv, N, D, dtype, seed=N + k, n_sinks=4, n_outlier=2)
    out, idx = topk_qaxis_attention(*_dev(Q, K, V), k, return_indices=True)
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), k)
    assert torch.equal(idx.cpu(), ref_idx)
    _assert_close_out(out, cpu.attention_f64(Q, K, V, ref_idx), dtype)
    assert torch.equal(topk_qaxis_select(*_dev(Q, K), k).cpu(), ref_idx)


def _random_case(i):
    """Shape of random-sweep case i (deterministic): B, Hkv, n_rep, N, D, k, dtype."""
    import random
    r = random.Random(1000 + i)
    n_rep = r.choice([1, 2, 4, 8])
    Hkv = r.choice([1, 2, 4]) if n_rep == 8 else r.choice([1, 2, 4, 8])
    D = r.choice([64, 128])
    dtype = r.choice([torch.float16, torch.bfloat16, torch.float32])
    N = int(round(math.exp(r.uniform(math.log(2), math.log(20000)))))
    N = max(N, 2)
    k = r.choice([1, N - 1, max(1, N // 7), r.randint(1, N - 1)])
    return r.choice([1, 2, 3]), Hkv, n_rep, N, D, k, dtype


@pytest.mark.parametrize("case", range(24))
def test_random_shapes_sweep(case):
    """Seeded random shapes through the full pipeline: ragged N from 2 to 20000,
    k from 1 to N - 1, every n_rep, D and dtype, against the oracle."""
    B, Hkv, n_rep, N, D, k, dtype = _random_case(case)
    print(f"random case {case}: B={B} Hkv={Hkv} n_rep={n_rep} N={N} D={D} k={k} {dtype}", flush=True)
    Q, K, V = make_qkv(B, Hkv * n_rep, Hkv, N, D, dtype, seed=case, n_sinks=2, n_outlier=1)
    out, idx = topk_qaxis_attention(*_dev(Q, K, V), k, return_indices=True)
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), k)
    assert torch.equal(idx.cpu(), ref_idx)
    _assert_close_out(out, cpu.attention_f64(Q, K, V, ref_idx), dtype)
    assert torch.equal(topk_qaxis_attention(*_dev(Q, K, V), k).cpu(), out.cpu())


@pytest.mark.parametrize("case", range(12))
def test_random_dense_sweep(case):
    """The dense kernel (comparator and k >= N fallback) over seeded random
    shapes: N from 1 to 20000, every n_rep, D and dtype, strided cache views,
    against exact float64 softmax attention over all rows."""
    import random
    r = random.Random(2000 + case)
    n_rep = r.choice([1, 2, 4, 8])
    Hkv = r.choice([1, 2, 4]) if n_rep == 8 else r.choice([1, 2, 4, 8])
    D = r.choice([64, 128])
    dtype = r.choice([torch.float16, torch.bfloat16, torch.float32])
    N = max(1, int(round(math.exp(r.uniform(0.0, math.log(20000))))))
    B = r.choice([1, 2, 3])
    pad = r.choice([0, 0, 5, 64])   # rows past N in the cache (a strided view)
    print(f"random dense case {case}: B={B} Hkv={Hkv} n_rep={n_rep} N={N}+{pad} D={D} {dtype}", flush=True)
    Q, K, V = make_qkv(B, Hkv * n_rep, Hkv, N + pad, D, dtype, seed=case, n_sinks=2, n_outlier=1)
    Qd, Kd, Vd = _dev(Q, K, V)
    out = dense_decode_attention(Qd, Kd[:, :, :N], Vd[:, :, :N])
    allrows = torch.arange(N, dtype=torch.int32).expand(B, Hkv * n_rep, N).contiguous()
    _assert_close_out(out, cpu.attention_f64(Q, K[:, :, :N], V[:, :, :N], allrows), dtype)


def test_max_row_length():
    """N = 2^24, the top-K limit: the score pass with 8192 slabs per row and
    the chunked select at its largest (256 chunks of 65536 positions)."""
    N, k = 1 << 24, 2048
    print(f"max-N case: B=1 H=4 Hkv=1 N={N} k={k} fp16", flush=True)
    Q, K, V = make_qkv(1, 4, 1, N, 64, torch.float16, seed=7, device=DEV, n_sinks=4, n_outlier=2)
    out, idx = topk_qaxis_attention(Q, K, V, k, return_indices=True)
    Qc, Kc = Q.cpu(), K.cpu()
    ref_idx = cpu.topk(cpu.scores(Kc, cpu.compute_uq(Qc)), k)
    assert torch.equal(idx.cpu(), ref_idx)
    _assert_close_out(out, cpu.attention_f64(Qc, Kc, V.cpu(), ref_idx), torch.float16)


def test_logits_at_bf16_rounding_ties():
    """fp16/bf16 logits are rebuilt from the bf16 score key plus an 8-bit residual.  With
    Q = e_0 the score of key n is K[n, 0] exactly, so K[:, :, :, 0] is set to values whose fp32
    pattern sits on a bf16 rounding tie (worst case of the residual, clamped at 127/256 ulp),
    that round up across a binade, negative ties, zeros and values near the fp16 maximum."""
    B, H, Hkv, N, D, k = 1, 4, 1, 4096, 64, 600
    g = torch.Generator().manual_seed(11)
    Q = torch.zeros(B, H, D)
    Q[..., 0] = torch.tensor([1.0, 0.5, 2.0, 0.25]).view(1, H)
    K = torch.randn(B, Hkv, N, D, generator=g) * 0.1
    specials = torch.tensor([1.00390625, -1.00390625, 1.99951171875, -1.99951171875, 0.0, -0.0,
                             3.0078125, 0.0078277587890625, 60000.0, -60000.0, 1.5009765625])
    col = (torch.rand(N, generator=g) * 8 - 4).to(torch.float16).float()
    col[: specials.numel() * 40] = specials.repeat(40)
    col = col[torch.randperm(N, generator=g)]
    K[0, 0, :, 0] = col / 8.0          # keeps logits moderate; /8 is exact in fp16
    V = torch.randn(B, Hkv, N, D, generator=g)
    for dt in (torch.float16, torch.bfloat16):
        Qd, Kd, Vd = Q.to(dt), K.to(dt), V.to(dt)
        out, idx = topk_qaxis_attention(*_dev(Qd, Kd, Vd), k, return_indices=True)
        ref_idx = cpu.topk(cpu.scores(Kd, cpu.compute_uq(Qd)), k)
        assert torch.equal(idx.cpu(), ref_idx)
        _assert_close_out(out, cpu.attention_f64(Qd, Kd, Vd, ref_idx), dt)


def test_pipeline_matches_oracle_fp32_steps():
    """C1 in fp32: the HIP output also tracks the oracle's own fp32 restatement."""
    cfg = CONFIGS["C1"]
    Q, K, V = make_inputs(cfg, seed=1)
    out = topk_qaxis_attention(*_dev(Q, K, V), cfg.k)
    ref = cpu.sparse_decode(Q, K, V, cfg.k)["out_f32"]
    assert (out.cpu() - ref).abs().max().item() <= 1e-5


# ------------------------------------------------------------ edge cases

def test_k_equals_n_minus_1_and_k_1():
    Q, K, V = make_qkv(1, 32, 8, 100, 64, torch.bfloat16, seed=0)
    for k in (99, 1):
        out, idx = topk_qaxis_attention(*_dev(Q, K, V), k, return_indices=True)
        ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), k)
        assert torch.equal(idx.cpu(), ref_idx)
        _assert_close_out(out, cpu.attention_f64(Q, K, V, ref_idx), torch.bfloat16)


def test_single_kv_head_group():
    # test_m3_fused_attn.py:141-159: H=4, H_kv=1
    Q, K, V = make_qkv(1, 4, 1, 1000, 64, torch.bfloat16, seed=7)
    out, idx = topk_qaxis_attention(*_dev(Q, K, V), 100, return_indices=True)
    assert out.shape == (1, 4, 64) and torch.isfinite(out).all()
    assert torch.equal(idx.cpu(), cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), 100))


def test_b8_memory():
    # test_m3_fused_attn.py:171-192: B=8, N=5000 stays well under 4 GB
    torch.cuda.reset_peak_memory_stats()
    Q, K, V = _dev(*make_qkv(8, 32, 8, 5000, 64, torch.bfloat16, seed=0))
    out = topk_qaxis_attention(Q, K, V, 2500)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert torch.cuda.max_memory_allocated() / 1e9 < 4.0


def test_zero_query():
    Q, K, V = make_qkv(1, 32, 8, 256, 64, torch.float16, seed=2)
    Q[0, :4] = 0
    out, idx = topk_qaxis_attention(*_dev(Q, K, V), 64, return_indices=True)
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), 64)
    assert torch.equal(idx.cpu(), ref_idx)
    _assert_close_out(out, cpu.attention_f64(Q, K, V, ref_idx), torch.float16)


def test_non_default_stream():
    Q, K, V = make_qkv(2, 32, 8, 3000, 64, torch.float16, seed=4)
    s = torch.cuda.Stream()
    Qd, Kd, Vd = _dev(Q, K, V)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        out = topk_qaxis_attention(Qd, Kd, Vd, 450)
    s.synchronize()
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), 450)
    _assert_close_out(out, cpu.attention_f64(Q, K, V, ref_idx), torch.float16)


def test_shape_errors_raise_assertion():
    Q, K, V = _dev(*make_qkv(1, 32, 8, 64, 64, torch.float16, seed=0))
    with pytest.raises(AssertionError):
        topk_qaxis_attention(Q, K, V, 64)          # k == N
    with pytest.raises(AssertionError):
        topk_qaxis_attention(Q, K, V, 0)
    with pytest.raises(AssertionError):
        topk_qaxis_attention(Q.float(), K, V, 8)   # dtype mismatch


# ------------------------------------------------------------------ dense

@pytest.mark.parametrize("dtype,D,N,B", [(torch.float16, 64, 4097, 2), (torch.float32, 64, 1000, 1),
                                         (torch.bfloat16, 128, 2048, 1)])
def test_dense_decode(dtype, D, N, B):
    Q, K, V = make_qkv(B, 32, 8, N, D, dtype, seed=N, n_sinks=4)
    out = dense_decode_attention(*_dev(Q, K, V))
    _assert_close_out(out, cpu.dense_f64(Q, K, V), dtype)


def test_dense_tickets_any_workspace_contents_repeats_and_graph_replays():
    """dcr_dense_decode merges in its own launch through tickets that reset
    themselves: a workspace of random bytes (no ticket carries the tag), calls
    repeated on it, and replays of a captured graph (with new queries between
    replays) all match the float64 reference and each other."""
    from dcr_attention_amd import _lib
    lib = _lib.load()
    B, H, Hkv, N, D, dtype = 2, 32, 8, 5000, 64, torch.float16
    Q, K, V = make_qkv(B, H, Hkv, N, D, dtype, seed=5, n_sinks=4)
    Qd, Kd, Vd = _dev(Q, K, V)
    nws = lib.dcr_dense_decode_workspace_bytes(B, H, Hkv, N, D)
    gen = torch.Generator().manual_seed(1)
    ws = torch.randint(0, 256, (nws,), dtype=torch.uint8, generator=gen).to(DEV)
    O = torch.empty(B, H, D, dtype=dtype, device=DEV)
    assert _lib.fused_errors(clear=True) == 0

    def call():
        _lib.check(lib.dcr_dense_decode(Qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(), _lib.DTYPE_CODE[dtype],
                                        O.data_ptr(), B, H, Hkv, N, N, D, ws.data_ptr(), nws,
                                        torch.cuda.current_stream().cuda_stream), "dcr_dense_decode")

    outs = []
    for _ in range(3):
        call()
        torch.cuda.synchronize()
        outs.append(O.clone())
    _assert_close_out(outs[0], cpu.dense_f64(Q, K, V), dtype)
    assert all(torch.equal(o, outs[0]) for o in outs)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for rep in range(4):
        Qd.copy_(torch.randn(B, H, D, generator=gen).to(dtype))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        o_g = O.clone()
        call()
        torch.cuda.synchronize()
        print(f"dense graph replay {rep}", flush=True)
        assert torch.equal(o_g, O)
    _assert_close_out(O, cpu.dense_f64(Qd.cpu(), K, V), dtype)
    assert _lib.fused_errors() == 0


# ------------------------------------------------------------ strided caches

def test_prefix_of_preallocated_cache_matches_contiguous():
    """K/V as the first N rows of a [B, H_kv, N_max, D] cache (ldn = N_max):
    identical indices and outputs to the contiguous call."""
    B, N, N_max = 2, 3000, 4096
    Q, K, V = make_qkv(B, 32, 8, N, 64, torch.float16, seed=11, n_sinks=4)
    Qd, Kd, Vd = _dev(Q, K, V)
    Kc = torch.full((B, 8, N_max, 64), float("nan"), dtype=torch.float16, device=DEV)
    Vc = torch.full_like(Kc, float("nan"))
    Kc[:, :, :N] = Kd
    Vc[:, :, :N] = Vd
    out_c, idx_c = topk_qaxis_attention(Qd, Kd, Vd, 451, return_indices=True)
    out_s, idx_s = topk_qaxis_attention(Qd, Kc[:, :, :N], Vc[:, :, :N], 451, return_indices=True)
    assert torch.equal(idx_c, idx_s)
    assert torch.equal(out_c, out_s)
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), 451)
    assert torch.equal(idx_s.cpu(), ref_idx)
    dense_c = dense_decode_attention(Qd, Kd, Vd)
    dense_s = dense_decode_attention(Qd, Kc[:, :, :N], Vc[:, :, :N])
    assert torch.equal(dense_c, dense_s)
    sc = topk_pass1_projection(Kc[:, :, :N], compute_u_Q(Qd))
    assert torch.equal(sc.view(torch.int16).cpu(),
                       cpu.scores(K, cpu.compute_uq(Q)).view(torch.int16))
    out_f = fused_topk_attention(Qd, Kc[:, :, :N], Vc[:, :, :N], idx_c)
    # fused_topk_attention gathers K for its logits; the fp16 decode path
    # reuses the score pass's dot products, equal up to fp32 rounding.
    assert (out_f.float() - out_c.float()).abs().max().item() <= 1e-3
    _assert_close_out(out_f, cpu.attention_f64(Q, K, V, ref_idx), torch.float16)


def test_unrepeat_view_of_repeated_cache():
    """The reference caller un-repeats a GQA-repeated cache with
    K[:, ::n_rep].contiguous() (attention.py:810-811); the strided view gives
    the same result without the copy."""
    B, N, n_rep = 2, 2500, 4
    Q, K, V = make_qkv(B, 32, 8, N, 64, torch.bfloat16, seed=12, n_sinks=4)
    Qd, Kd, Vd = _dev(Q, K, V)
    Kr = Kd.repeat_interleave(n_rep, dim=1)      # [B, 32, N, D], like repeat_kv
    Vr = Vd.repeat_interleave(n_rep, dim=1)
    out_c, idx_c = topk_qaxis_attention(Qd, Kd, Vd, 376, return_indices=True)
    out_v, idx_v = topk_qaxis_attention(Qd, Kr[:, ::n_rep], Vr[:, ::n_rep], 376,
                                        return_indices=True)
    assert torch.equal(idx_c, idx_v)
    assert torch.equal(out_c, out_v)
