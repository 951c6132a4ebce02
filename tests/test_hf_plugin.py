"""The HuggingFace plugin (llama.monkey_patch, llama.hf_attention) on the CPU.

Follows the reference's lifecycle and wrapper tests
(tests/models/llama/test_monkey_patch_lifecycle.py, test_dcr_llama_unit.py,
test_hf_5x_contract.py): patch / unpatch / re-patch, idempotence with a
warning, layer_filter, projections shared by reference, no parameter copies,
errors on non-Llama models, shape resolution from the transformers 5.x layout,
the two-value return, counters.  The prefill (dense) branch is pure torch and
is checked here against the unpatched HF model on the same weights; decode
branches run HIP kernels (tests/test_gpu_hf_plugin.py) and, with CPU tensors,
must raise instead of falling back.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig, LlamaForCausalLM  # noqa: E402

from dcr_attention_amd.llama import DCRLlamaConfig  # noqa: E402
from dcr_attention_amd.llama.hf_attention import DCRLlamaAttention  # noqa: E402
from dcr_attention_amd.llama.monkey_patch import (is_patched, patch_llama_with_dcr,  # noqa: E402
                                                  patched_layer_indices, reconfigure_dcr,
                                                  unpatch_llama)


class _Attn(nn.Module):
    """Stand-in for LlamaAttention with the transformers 4.x attribute layout."""

    def __init__(self, layer_idx, hidden=128, heads=4, kv_heads=2, head_dim=32):
        super().__init__()
        self.num_heads, self.num_key_value_heads, self.head_dim = heads, kv_heads, head_dim
        self.layer_idx = layer_idx
        self.q_proj = nn.Linear(hidden, heads * head_dim, bias=False)
        self.k_proj = nn.Linear(hidden, kv_heads * head_dim, bias=False)
        self.v_proj = nn.Linear(hidden, kv_heads * head_dim, bias=False)
        self.o_proj = nn.Linear(heads * head_dim, hidden, bias=False)


class _Layer(nn.Module):
    def __init__(self, i):
        super().__init__()
        self.self_attn = _Attn(i)


class _Inner(nn.Module):
    def __init__(self, n):
        super().__init__()
        self.layers = nn.ModuleList(_Layer(i) for i in range(n))


class _CausalLM(nn.Module):
    def __init__(self, n=4):
        super().__init__()
        self.model = _Inner(n)


def _tiny_hf(attn="eager", seed=0, layers=2):
    cfg = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=32,
                      max_position_embeddings=4096, rope_theta=500000.0, attn_implementation=attn)
    torch.manual_seed(seed)
    return LlamaForCausalLM(cfg).eval()


# ------------------------------------------------------------------ lifecycle

def test_patch_replaces_every_layer_and_unpatch_restores_the_originals():
    m = _CausalLM(4)
    originals = [l.self_attn for l in m.model.layers]
    assert patch_llama_with_dcr(m) == 4
    assert is_patched(m) and patched_layer_indices(m) == [0, 1, 2, 3]
    assert all(isinstance(l.self_attn, DCRLlamaAttention) for l in m.model.layers)
    assert unpatch_llama(m) == 4
    assert not is_patched(m)
    assert all(l.self_attn is o for l, o in zip(m.model.layers, originals))
    assert unpatch_llama(m) == 0                      # never patched (any more): no-op


def test_bare_model_layout():
    inner = _Inner(3)
    assert patch_llama_with_dcr(inner) == 3 and is_patched(inner)


def test_projections_shared_and_no_parameter_copied():
    m = _CausalLM(2)
    q0 = m.model.layers[0].self_attn.q_proj
    n0 = sum(p.numel() for p in m.parameters())
    patch_llama_with_dcr(m)
    assert m.model.layers[0].self_attn.q_proj is q0
    assert sum(p.numel() for p in m.parameters()) == n0


def test_double_patch_warns_and_replaces_nothing():
    m = _CausalLM(3)
    patch_llama_with_dcr(m)
    with pytest.warns(UserWarning, match="already patched"):
        assert patch_llama_with_dcr(m) == 0
    for l in m.model.layers:
        assert isinstance(l.self_attn, DCRLlamaAttention)
        assert not isinstance(l.self_attn.base_layer, DCRLlamaAttention)


def test_patch_unpatch_patch_roundtrip_and_layer_filter():
    m = _CausalLM(8)
    assert patch_llama_with_dcr(m, DCRLlamaConfig(layer_filter=frozenset({2, 5, 7}))) == 3
    assert patched_layer_indices(m) == [2, 5, 7]
    assert isinstance(m.model.layers[0].self_attn, _Attn)
    assert unpatch_llama(m) == 3
    assert patch_llama_with_dcr(m, DCRLlamaConfig(layer_filter=frozenset({1, 4}))) == 2
    assert patched_layer_indices(m) == [1, 4]


def test_reconfigure_updates_every_wrapped_layer():
    m = _CausalLM(3)
    patch_llama_with_dcr(m)
    new = DCRLlamaConfig(enable_dcr=False, coverage_floor=0.3)
    assert reconfigure_dcr(m, new) == 3
    assert all(l.self_attn.cfg is new for l in m.model.layers)


def test_rejects_models_without_a_llama_layout():
    class Foo(nn.Module):
        pass

    with pytest.raises(ValueError, match="Cannot find transformer layers"):
        patch_llama_with_dcr(Foo())

    class NoAttn(nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = nn.ModuleList([nn.Linear(2, 2)])

    with pytest.raises(ValueError, match="self_attn"):
        patch_llama_with_dcr(NoAttn())
    assert not is_patched(Foo()) and patched_layer_indices(Foo()) == []


# --------------------------------------------------------- wrapper construction

def test_wrapper_resolves_shapes_from_the_5x_layout():
    m = _tiny_hf()
    base = m.model.layers[0].self_attn                # 5.x: head counts only on the config
    w = DCRLlamaAttention(base)
    assert (w.num_heads, w.num_key_value_heads, w.head_dim, w.n_rep) == (8, 2, 32, 4)
    assert w.layer_idx == 0 and w.q_proj is base.q_proj
    assert "axis_source='q_topk_hip'" in w.extra_repr()


def test_wrapper_rejects_bad_gqa_and_missing_shapes():
    a = _Attn(0, heads=6, kv_heads=4)
    with pytest.raises(ValueError, match="divisible"):
        DCRLlamaAttention(a)
    b = _Attn(0)
    del b.num_heads
    b.head_dim = None
    with pytest.raises(ValueError, match="head_dim"):
        DCRLlamaAttention(b)


# ------------------------------------------------------------- forward (CPU)

@pytest.mark.parametrize("attn", ["eager", "sdpa"])
def test_patched_prefill_matches_unpatched_hf(attn):
    """Prefill routes to the dense branch (fp32-softmax eager attention with the
    causal mask), which must equal HF's own attention on the same weights."""
    ref = _tiny_hf(attn, seed=3)
    pat = _tiny_hf(attn, seed=3)
    pat.load_state_dict(ref.state_dict())
    assert patch_llama_with_dcr(pat) == 2
    ids = torch.randint(0, 512, (2, 40), generator=torch.Generator().manual_seed(1))
    DCRLlamaAttention.reset_counters()
    with torch.no_grad():
        a = ref(ids).logits
        b = pat(ids).logits
    assert DCRLlamaAttention.get_counters() == {"dcr": 0, "sdpa": 2}
    assert (a - b).abs().max().item() < 1e-5
    assert pat.state_dict().keys() == ref.state_dict().keys()


def test_forward_returns_two_values_and_refuses_attention_weights():
    m = _tiny_hf()
    w = DCRLlamaAttention(m.model.layers[0].self_attn)
    x = torch.randn(1, 5, 256)
    pos = torch.arange(5).view(1, 5)
    cos_sin = m.model.rotary_emb(x, pos)
    out = w(x, position_embeddings=cos_sin)
    assert isinstance(out, tuple) and len(out) == 2 and out[1] is None
    assert out[0].shape == (1, 5, 256)
    with pytest.raises(NotImplementedError):
        w(x, position_embeddings=cos_sin, output_attentions=True)


def test_decode_on_cpu_raises_instead_of_falling_back():
    """Decode steps run HIP kernels only (DCR branch and dense decode kernel)."""
    m = _tiny_hf()
    patch_llama_with_dcr(m, DCRLlamaConfig(T_dispatch=0))
    ids = torch.randint(0, 512, (1, 12), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        out = m(ids, use_cache=True)
        with pytest.raises(RuntimeError, match="HIP"):
            m(ids[:, -1:], past_key_values=out.past_key_values, use_cache=True)
