"""The Llama decode caller (dcr_attention_amd.llama.model) against
HuggingFace transformers' Llama on the same weights (CPU, fp32), and its DCR
decode steps against the same decoder with the CPU oracle's sparse attention.

The reference's own tests of this layer (tests/models/llama/
test_dcr_llama_unit.py, test_routing.py) run HF's Llama with the DCR wrapper
patched in; here the decoder is this build's, so HF is the pin for
everything but the attention branch, and the oracle pins the branch."""
from __future__ import annotations

import pytest
import torch

from oracle import cpu
from dcr_attention_amd.llama import DCRLlamaConfig, adaptive_k_window
from dcr_attention_amd.llama.model import (DCRLlamaDecoder, KVCache, LlamaDecoderConfig,
                                           eager_sdpa, rope_inv_freq)

TINY = LlamaDecoderConfig(vocab_size=1000, hidden_size=256, intermediate_size=512, num_layers=2,
                          num_heads=8, num_kv_heads=2, head_dim=64, rope_theta=500000.0,
                          rope_scaling=(32.0, 1.0, 4.0, 8192))


def _hf_model(cfg: LlamaDecoderConfig, seed=0):
    transformers = pytest.importorskip("transformers")
    hc = transformers.LlamaConfig(
        vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
        intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_layers,
        num_attention_heads=cfg.num_heads, num_key_value_heads=cfg.num_kv_heads,
        head_dim=cfg.head_dim, rope_theta=cfg.rope_theta, max_position_embeddings=131072,
        rope_scaling={"rope_type": "llama3", "factor": cfg.rope_scaling[0],
                      "low_freq_factor": cfg.rope_scaling[1], "high_freq_factor": cfg.rope_scaling[2],
                      "original_max_position_embeddings": cfg.rope_scaling[3]},
        rms_norm_eps=cfg.rms_norm_eps, tie_word_embeddings=cfg.tie_word_embeddings,
        attn_implementation="eager")
    torch.manual_seed(seed)
    m = transformers.LlamaForCausalLM(hc).eval()
    with torch.no_grad():  # non-trivial norm weights
        for n, p in m.named_parameters():
            if "norm" in n:
                p.uniform_(0.5, 1.5)
    return m


def test_rope_inv_freq_matches_hf():
    m = _hf_model(TINY)
    hf = m.model.rotary_emb.inv_freq.float()
    ours = rope_inv_freq(TINY)
    assert torch.allclose(ours, hf, rtol=1e-6, atol=0)


def test_prefill_logits_match_hf():
    m = _hf_model(TINY)
    dec = DCRLlamaDecoder(TINY, dtype=torch.float32, device="cpu").load_hf_state_dict(m.state_dict())
    ids = torch.randint(0, TINY.vocab_size, (2, 37), generator=torch.Generator().manual_seed(1))
    cache = KVCache.allocate(TINY, 2, 64, torch.float32, "cpu")
    DCRLlamaDecoder.reset_counters()
    ours = dec.forward(ids, cache)
    with torch.no_grad():
        ref = m(ids).logits
    assert (ours - ref).abs().max().item() < 2e-4
    assert cache.length == 37
    # prefill always routes dense (route: N_q > 1), once per layer
    assert DCRLlamaDecoder.get_counters() == {"dcr": 0, "sdpa": TINY.num_layers}


def test_eager_sdpa_causal_matches_plain_softmax():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 8, 5, 64, generator=g, dtype=torch.float64)
    K = torch.randn(1, 2, 9, 64, generator=g, dtype=torch.float64)
    V = torch.randn(1, 2, 9, 64, generator=g, dtype=torch.float64)
    out = eager_sdpa(q, K, V, 4)
    Kr, Vr = K.repeat_interleave(4, 1), V.repeat_interleave(4, 1)
    for t in range(5):  # query t sees keys 0 .. 4 + t
        s = (q[:, :, t:t + 1] @ Kr[:, :, :5 + t].transpose(-1, -2)) / 8.0
        ref = torch.softmax(s, -1) @ Vr[:, :, :5 + t]
        assert torch.allclose(out[:, :, t:t + 1], ref, atol=1e-6)  # softmax runs in fp32


def test_cache_capacity_guard():
    dec = DCRLlamaDecoder(TINY, dtype=torch.float32, device="cpu").init_random(0)
    cache = KVCache.allocate(TINY, 1, 8, torch.float32, "cpu")
    with pytest.raises(AssertionError, match="capacity"):
        dec.forward(torch.zeros(1, 9, dtype=torch.long), cache)


# ----------------------------------------------------------------- GPU

class _OracleDecoder(DCRLlamaDecoder):
    """Same decoder on the CPU; decode-step DCR attention by the C oracle."""

    def _attention(self, l, q, cache, n_kv):
        if q.shape[2] == 1 and n_kv >= self.dcr.T_dispatch:
            k_eff = adaptive_k_window(self.dcr.k_window, n_kv, self.dcr.coverage_floor)
            K = cache.k[l][:, :, :n_kv].contiguous()
            V = cache.v[l][:, :, :n_kv].contiguous()
            Q = q.squeeze(2).contiguous()
            if k_eff >= n_kv:
                return cpu.dense_f64(Q, K, V).float().unsqueeze(2)
            return cpu.sparse_decode(Q, K, V, k_eff)["out_f32"].unsqueeze(2)
        return super()._attention(l, q, cache, n_kv)


@pytest.mark.gpu
def test_decode_steps_dense_branch_match_hf():
    m = _hf_model(TINY)
    dec = DCRLlamaDecoder(TINY, DCRLlamaConfig(enable_dcr=False), dtype=torch.float32,
                          device="cuda").load_hf_state_dict(m.state_dict())
    ids = torch.randint(0, TINY.vocab_size, (2, 40), generator=torch.Generator().manual_seed(2))
    cache = KVCache.allocate(TINY, 2, 64, torch.float32, "cuda")
    dec.forward(ids[:, :36].cuda(), cache)
    for t in range(36, 40):  # decode steps: dense HIP kernel on the strided cache
        step = dec.forward(ids[:, t:t + 1].cuda(), cache)[:, -1].cpu()
        with torch.no_grad():
            ref = m(ids[:, :t + 1]).logits[:, -1]
        assert (step - ref).abs().max().item() < 2e-4, t


@pytest.mark.gpu
def test_decode_steps_dcr_branch_match_oracle_decoder():
    m = _hf_model(TINY, seed=4)
    sd = m.state_dict()
    dcr = DCRLlamaConfig(T_dispatch=0, coverage_floor=0.25)
    gpu = DCRLlamaDecoder(TINY, dcr, dtype=torch.float32, device="cuda").load_hf_state_dict(sd)
    ref = _OracleDecoder(TINY, dcr, dtype=torch.float32, device="cpu").load_hf_state_dict(sd)
    ids = torch.randint(0, TINY.vocab_size, (2, 305), generator=torch.Generator().manual_seed(5))
    cg = KVCache.allocate(TINY, 2, 320, torch.float32, "cuda")
    cc = KVCache.allocate(TINY, 2, 320, torch.float32, "cpu")
    gpu.forward(ids[:, :300].cuda(), cg)
    ref.forward(ids[:, :300], cc)
    DCRLlamaDecoder.reset_counters()
    for t in range(300, 305):
        a = gpu.forward(ids[:, t:t + 1].cuda(), cg)[:, -1].cpu()
        b = ref.forward(ids[:, t:t + 1], cc)[:, -1]
        assert (a - b).abs().max().item() < 1e-3, t
        assert torch.equal(a.argmax(-1), b.argmax(-1))
    n_dcr = DCRLlamaDecoder.get_counters()["dcr"]
    assert n_dcr >= 5 * TINY.num_layers  # every decode step of every layer took the DCR branch


@pytest.mark.gpu
def test_decode_on_synthetic_32k_cache_routes_dcr():
    cfg = LlamaDecoderConfig(num_layers=2)  # Llama-3.2-1B layer shapes, 2 layers
    dec = DCRLlamaDecoder(cfg, dtype=torch.float16, device="cuda").init_random(0)
    cache = KVCache.allocate(cfg, 2, 32768 + 8, torch.float16, "cuda")
    cache.fill_synthetic(32768, seed=1)
    DCRLlamaDecoder.reset_counters()
    tok = torch.tensor([1, 2], device="cuda")
    for _ in range(3):
        tok = dec.decode_step(tok, cache)
    torch.cuda.synchronize()
    assert cache.length == 32771
    assert DCRLlamaDecoder.get_counters() == {"dcr": 6, "sdpa": 0}
    assert tok.shape == (2,) and (0 <= tok).all() and (tok < cfg.vocab_size).all()
