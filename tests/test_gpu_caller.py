"""Decode caller glue on the GPU (reference _dcr_forward q_topk branch,
dcr_attention/models/llama/attention.py:805-813): k_eff from
adaptive_k_window, the un-repeat of a GQA-repeated cache, and the dense
fallback when k_eff >= N_kv.  Checked against the CPU oracle."""
from __future__ import annotations

import pytest
import torch

from oracle import cpu
from dcr_attention_amd.llama import DCRLlamaConfig, adaptive_k_window
from dcr_attention_amd.llama.attention import dcr_forward, sdpa_forward
from dcr_attention_amd.synthetic import make_qkv

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 5e-3}


def _close(out, ref64, dtype):
    """Same bar as the op parity tests: TOL per dtype, for bf16 at least one
    bf16 ulp of the exact value (output rounding alone can reach half of it)."""
    o = out.double().cpu().reshape(ref64.shape)
    tol = torch.full_like(ref64, TOL[dtype])
    if dtype == torch.bfloat16:
        tol = torch.maximum(tol, torch.ldexp(torch.ones_like(ref64), torch.frexp(ref64)[1] - 8))
    diff = (o - ref64).abs()
    assert not (diff > tol).any(), diff.max().item()
    cos = torch.nn.functional.cosine_similarity(o.flatten(1), ref64.flatten(1), dim=-1)
    assert cos.min().item() >= 0.9999


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dcr_forward_repeated_cache(dtype):
    B, N = 2, 4096
    Q, K, V = make_qkv(B, 32, 8, N, 64, dtype, seed=21, n_sinks=4)
    cfg = DCRLlamaConfig()
    k_eff = adaptive_k_window(cfg.k_window, N, cfg.coverage_floor)
    assert k_eff == 614
    Qd = Q.cuda().unsqueeze(-2)                              # [B, H, 1, D]
    Kr = K.cuda().repeat_interleave(4, dim=1)                # post-repeat_kv [B, H, N, D]
    Vr = V.cuda().repeat_interleave(4, dim=1)
    out = dcr_forward(Qd, Kr, Vr, cfg, n_rep=4)
    assert out.shape == (B, 32, 1, 64) and out.dtype == dtype
    ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(Q)), k_eff)
    _close(out, cpu.attention_f64(Q, K, V, ref_idx), dtype)
    out_u = dcr_forward(Qd, K.cuda(), V.cuda(), cfg, n_rep=4, kv_repeated=False)
    assert torch.equal(out, out_u)


def test_dcr_forward_falls_back_to_dense_when_k_covers_cache():
    N = 64                                                   # k_window 64 -> k_eff = N
    Q, K, V = make_qkv(1, 32, 8, N, 64, torch.float16, seed=22)
    out = dcr_forward(Q.cuda().unsqueeze(-2), K.cuda(), V.cuda(), DCRLlamaConfig(), n_rep=4,
                      kv_repeated=False)
    _close(out, cpu.dense_f64(Q, K, V), torch.float16)


def test_sdpa_forward_decode_and_prefill():
    Q, K, V = make_qkv(1, 32, 8, 300, 64, torch.float32, seed=23)
    out = sdpa_forward(Q.cuda().unsqueeze(-2), K.cuda(), V.cuda(), None, 1, 300, n_rep=4,
                       kv_repeated=False)
    _close(out, cpu.dense_f64(Q, K, V), torch.float32)
    # prefill: causal eager path, last query row equals decode attention
    Qp = torch.randn(1, 32, 5, 64, generator=torch.Generator().manual_seed(1))
    Qp[:, :, -1] = Q
    outp = sdpa_forward(Qp.cuda(), K.cuda(), V.cuda(), None, 5, 300, n_rep=4, kv_repeated=False)
    assert (outp[:, :, -1].cpu().double() - cpu.dense_f64(Q, K, V)).abs().max() <= 1e-5
