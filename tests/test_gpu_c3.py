"""C3 at its own size: the Llama-3.2-1B-shaped decoder (16 layers, hidden 2048,
FFN 8192, 32 Q / 8 KV heads, D = 64, vocab 128256, random fp16 weights), B = 4,
a KV cache holding 32768 synthetic positions, greedy decode steps through the
reference-style routing (the reference's Llama runtime tests:
tests/models/llama/test_dcr_llama_unit.py; acceptance at long context:
test_m1_acceptance.py:143-213).

* Every layer's DCR attention call of one decode step is checked on its real
  inputs (post-RoPE query, the strided 32769-row cache view) against the CPU
  oracle: top-K indices bit-exact, output within 2e-3 (fp16) of the float64
  closed form, cosine >= 0.9999.
* Four decode steps route every layer to the DCR branch: counters
  {"dcr": 64, "sdpa": 0}; all logits finite.
* With coverage_floor = 0.99999 (k_eff = 32768 of 32769 keys: the sparse path
  drops one key per head) a decode step's logits equal the dense branch's
  within 0.05 absolute and give the same greedy tokens.  The bound: one
  dropped key out of 32769 moves each attention output by about its softmax
  weight (~1e-4 here, near-uniform logits), and the two kernels' fp16 output
  roundings (2^-11 relative) differ per layer; through 16 layers and the
  128256-way lm_head (logits of magnitude ~1) that stays far below 0.05.
"""
from __future__ import annotations

import pytest
import torch

from oracle import cpu
from dcr_attention_amd.llama import DCRLlamaConfig
from dcr_attention_amd.llama.model import LLAMA_3_2_1B, DCRLlamaDecoder, KVCache

pytestmark = pytest.mark.gpu
DEV = "cuda"
B, N_CTX = 4, 32768


class _CapturingDecoder(DCRLlamaDecoder):
    """Copies each DCR attention call's inputs and output to the host."""

    capture = False

    def __init__(self, *a, **kw):
        super().__init__(*a, **kw)
        self.calls = []

    def _attention(self, l, q, cache, n_kv):
        out = super()._attention(l, q, cache, n_kv)
        if self.capture:
            self.calls.append((l, q.squeeze(2).cpu(), cache.k[l][:, :, :n_kv].cpu(),
                               cache.v[l][:, :, :n_kv].cpu(), out.squeeze(2).cpu()))
        return out


def _model(dcr):
    dec = _CapturingDecoder(LLAMA_3_2_1B, dcr, dtype=torch.float16, device=DEV).init_random(0)
    cache = KVCache.allocate(LLAMA_3_2_1B, B, N_CTX + 16, torch.float16, DEV)
    cache.fill_synthetic(N_CTX, seed=1)
    return dec, cache


@pytest.mark.timeout(400)
def test_c3_decode_step_every_layer_matches_oracle_and_routes_dcr():
    print(f"C3: {LLAMA_3_2_1B.num_layers} layers, B={B}, cache {N_CTX} positions, fp16", flush=True)
    dec, cache = _model(DCRLlamaConfig())
    tok = torch.tensor([1, 17, 4242, 128000], device=DEV)
    counters = type(dec)          # class-level counters, as the reference's (attention.py:93-119)
    counters.reset_counters()
    dec.capture = True
    logits = dec.forward(tok.view(-1, 1), cache)[:, -1]
    dec.capture = False
    assert torch.isfinite(logits).all()
    assert len(dec.calls) == LLAMA_3_2_1B.num_layers
    n_kv = N_CTX + 1
    k_eff = 4916                                   # adaptive_k_window(64, 32769, 0.15)
    for l, q, K, V, out in dec.calls:
        assert K.shape == (B, 8, n_kv, 64)
        ref_idx = cpu.topk(cpu.scores(K, cpu.compute_uq(q)), k_eff)
        ref = cpu.attention_f64(q, K, V, ref_idx)
        err = (out.double() - ref).abs().max().item()
        cos = torch.nn.functional.cosine_similarity(out.double().flatten(1), ref.flatten(1), dim=-1)
        print(f"  layer {l:2d}: max|out - f64| = {err:.2e}, min cos = {cos.min().item():.6f}", flush=True)
        assert err <= 2e-3 and cos.min().item() >= 0.9999, l
    # the indices themselves, through the select entry point on the same inputs
    from dcr_attention_amd.kernel.hip import topk_qaxis_select
    l, q, K, _, _ = dec.calls[-1]
    idx = topk_qaxis_select(q.to(DEV), K.to(DEV), k_eff)
    assert torch.equal(idx.cpu(), cpu.topk(cpu.scores(K, cpu.compute_uq(q)), k_eff))
    dec.calls.clear()

    for _ in range(3):
        tok = dec.decode_step(tok, cache)
    torch.cuda.synchronize()
    assert counters.get_counters() == {"dcr": 4 * LLAMA_3_2_1B.num_layers, "sdpa": 0}
    assert cache.length == N_CTX + 4
    assert ((0 <= tok) & (tok < LLAMA_3_2_1B.vocab_size)).all()


@pytest.mark.timeout(300)
def test_c3_near_full_coverage_matches_dense_branch():
    dec, cache = _model(DCRLlamaConfig(coverage_floor=0.99999))
    tok = torch.tensor([[3], [99], [5000], [77777]], device=DEV)
    counters = type(dec)
    counters.reset_counters()
    sparse = dec.forward(tok, cache)[:, -1]
    assert counters.get_counters() == {"dcr": LLAMA_3_2_1B.num_layers, "sdpa": 0}
    cache.length = N_CTX                           # the same step again, dense branch
    dec.dcr = DCRLlamaConfig(enable_dcr=False)
    dense = dec.forward(tok, cache)[:, -1]
    assert counters.get_counters()["sdpa"] == LLAMA_3_2_1B.num_layers
    diff = (sparse - dense).abs().max().item()
    print(f"C3 k_eff = N-1: max|logits(sparse) - logits(dense)| = {diff:.3e} "
          f"(|logits| <= {dense.abs().max().item():.2f})", flush=True)
    assert torch.isfinite(sparse).all() and torch.isfinite(dense).all()
    assert diff <= 0.05
    assert torch.equal(sparse.argmax(-1), dense.argmax(-1))
