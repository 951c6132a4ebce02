"""The HuggingFace plugin on the GPU: a random-init transformers
``LlamaForCausalLM`` (GQA 8 Q / 2 KV heads, D = 64) patched with
``patch_llama_with_dcr``.  After the reference's integration tests
(tests/models/llama/test_dcr_llama_integration.py: enable_dcr=False matches
the unpatched model, the DCR branch triggers on long-context decode, the
parameter count is unchanged):

* ``enable_dcr=False``: prefill and decode logits equal the unpatched model's
  (HF's own attention) within fp32 rounding;
* long-context decode (T_dispatch below the cache length) takes the DCR branch
  in every layer, and its logits equal those of the same model whose DCR
  branch is computed by the CPU oracle (the reference's M1 algorithm) on the
  same inputs;
* ``generate`` runs through the patched layers and gives the oracle model's
  greedy tokens; unpatching restores the original model's logits exactly.
"""
from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import DynamicCache, LlamaConfig, LlamaForCausalLM  # noqa: E402

from oracle import cpu  # noqa: E402
from dcr_attention_amd.llama import DCRLlamaConfig, adaptive_k_window  # noqa: E402
from dcr_attention_amd.llama.hf_attention import DCRLlamaAttention  # noqa: E402
from dcr_attention_amd.llama.monkey_patch import (patch_llama_with_dcr, reconfigure_dcr,  # noqa: E402
                                                  unpatch_llama)

pytestmark = pytest.mark.gpu
DEV = "cuda"
PREFILL = 700


def _model(dtype, seed=0):
    cfg = LlamaConfig(vocab_size=1000, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                      max_position_embeddings=4096, rope_theta=500000.0, attn_implementation="sdpa")
    torch.manual_seed(seed)
    return LlamaForCausalLM(cfg).to(device=DEV, dtype=dtype).eval()


class _OracleDCRAttention(DCRLlamaAttention):
    """The DCR branch computed by the CPU oracle (M1: u_Q, bf16 scores, stable
    top-k, 64-row online softmax) instead of the HIP kernels."""

    def _dcr_branch(self, q, k, v):
        n_kv = k.shape[-2]
        k_eff = adaptive_k_window(self.cfg.k_window, n_kv, self.cfg.coverage_floor)
        assert k_eff < n_kv
        out = cpu.sparse_decode(q.squeeze(2), k, v, k_eff)["out"]
        return out.to(q.device).unsqueeze(2)


def _oracle_patch(model, dcr):
    patch_llama_with_dcr(model, dcr)
    for layer in model.model.layers:
        layer.self_attn.__class__ = _OracleDCRAttention


def _decode(model, ids, steps):
    """Prefill ids, then `steps` greedy decode steps; returns the decode logits [steps, B, V]."""
    cache = DynamicCache()
    with torch.no_grad():
        out = model(ids, past_key_values=cache, use_cache=True)
        tok = out.logits[:, -1:].argmax(-1)
        logits = []
        for _ in range(steps):
            out = model(tok, past_key_values=cache, use_cache=True)
            logits.append(out.logits[:, -1].float())
            tok = out.logits[:, -1:].argmax(-1)
    return torch.stack(logits)


def _ids(B=2, n=PREFILL, seed=5):
    return torch.randint(0, 1000, (B, n), generator=torch.Generator().manual_seed(seed)).to(DEV)


def test_enable_dcr_false_matches_unpatched():
    ref = _model(torch.float32, seed=1)
    pat = _model(torch.float32, seed=1)
    n_params = sum(p.numel() for p in pat.parameters())
    patch_llama_with_dcr(pat, DCRLlamaConfig(enable_dcr=False))
    assert sum(p.numel() for p in pat.parameters()) == n_params
    ids = _ids()
    a, b = _decode(ref, ids, 3), _decode(pat, ids, 3)
    print(f"enable_dcr=False vs unpatched: max|dlogits| = {(a - b).abs().max().item():.2e}", flush=True)
    assert (a - b).abs().max().item() < 1e-4


class _CapturingDCRAttention(DCRLlamaAttention):
    """The HIP DCR branch, recording each call's inputs and output on the host."""

    calls = []

    def _dcr_branch(self, q, k, v):
        out = super()._dcr_branch(q, k, v)
        type(self).calls.append((q.squeeze(2).cpu(), k.cpu(), v.cpu(), out.squeeze(2).cpu()))
        return out


@pytest.mark.parametrize("dtype,tol,logit_bound", [(torch.float32, 1e-5, 1e-4),
                                                   (torch.float16, 2e-3, 0.1)])
def test_long_context_decode_takes_dcr_and_matches_oracle(dtype, tol, logit_bound):
    """Every DCR call of the patched model checked on its real inputs (indices
    bit-exact, output within the path's tolerance of the float64 oracle), then
    the decode logits against the same model with the oracle's DCR branch.  The
    logits bound is tight in fp32; in fp16 one-ulp differences of attention
    outputs run through fp16 GEMMs, so it only guards against gross errors
    (greedy tokens must still agree)."""
    dcr = DCRLlamaConfig(T_dispatch=256)
    hip = _model(dtype, seed=2)
    ora = _model(dtype, seed=2)
    patch_llama_with_dcr(hip, dcr)
    for layer in hip.model.layers:
        layer.self_attn.__class__ = _CapturingDCRAttention
    _CapturingDCRAttention.calls = []
    _oracle_patch(ora, dcr)
    ids = _ids(seed=6)
    _CapturingDCRAttention.reset_counters()
    a = _decode(hip, ids, 4)
    assert _CapturingDCRAttention.get_counters() == {"dcr": 2 * 4, "sdpa": 2}   # prefill: dense
    assert len(_CapturingDCRAttention.calls) == 8
    from dcr_attention_amd.kernel.hip import topk_qaxis_select
    for q, k, v, out in _CapturingDCRAttention.calls:
        k_eff = adaptive_k_window(dcr.k_window, k.shape[-2], dcr.coverage_floor)
        ref_idx = cpu.topk(cpu.scores(k, cpu.compute_uq(q)), k_eff)
        assert torch.equal(topk_qaxis_select(q.to(DEV), k.to(DEV), k_eff).cpu(), ref_idx)
        err = (out.double() - cpu.attention_f64(q, k, v, ref_idx)).abs().max().item()
        assert err <= tol, err
    b = _decode(ora, ids, 4)
    d = (a - b).abs().max().item()
    print(f"{dtype}: HIP-patched vs oracle-patched decode logits: max|d| = {d:.2e}", flush=True)
    assert torch.isfinite(a).all() and d < logit_bound
    assert torch.equal(a.argmax(-1), b.argmax(-1))


def test_generate_and_unpatch():
    dcr = DCRLlamaConfig(T_dispatch=256)
    m = _model(torch.float32, seed=3)
    ids = _ids(B=1, seed=7)
    with torch.no_grad():
        base = m(ids).logits
    patch_llama_with_dcr(m, dcr)
    DCRLlamaAttention.reset_counters()
    with torch.no_grad():
        gen = m.generate(ids, max_new_tokens=4, do_sample=False)
    assert DCRLlamaAttention.get_counters()["dcr"] >= 2 * 3
    ora = _model(torch.float32, seed=3)
    _oracle_patch(ora, dcr)
    with torch.no_grad():
        gen_o = ora.generate(ids, max_new_tokens=4, do_sample=False)
    assert torch.equal(gen, gen_o)
    assert reconfigure_dcr(m, DCRLlamaConfig(enable_dcr=False)) == 2
    assert unpatch_llama(m) == 2
    with torch.no_grad():
        assert torch.equal(m(ids).logits, base)
