"""Caller logic of the sparse decode path: k_eff policy, routing, config.

Cases follow the reference's own tests of the same functions
(tests/models/llama/test_routing.py, the adaptive_k_window docstring table at
dcr_attention/models/llama/adaptive.py:53-63) plus the C1..C5 k_eff values.
"""
from __future__ import annotations

import itertools
import math
import warnings

import pytest
import torch

from dcr_attention_amd.llama import (Branch, DCRLlamaConfig, adaptive_k_window, explain_route,
                                     route)
from dcr_attention_amd.llama.attention import dcr_forward
from dcr_attention_amd.synthetic import CONFIGS


# ------------------------------------------------------------ adaptive_k_window

@pytest.mark.parametrize("n_kv,expect", [(64, 64), (100, 80), (256, 204), (1000, 800),
                                          (4096, 3276)])
def test_adaptive_docstring_table(n_kv, expect):
    assert adaptive_k_window(64, n_kv, 0.8) == expect


def test_adaptive_config_values():
    # caller rule (floor, then up to even) vs the benchmark rule ceil(c*N)
    assert adaptive_k_window(64, 4096, 0.15) == 614 and CONFIGS["C1"].k == 615
    assert adaptive_k_window(64, 32768, 0.15) == 4916 == CONFIGS["C2"].k
    assert adaptive_k_window(64, 32769, 0.15) == 4916      # decode step after a 32K prefill
    assert adaptive_k_window(64, 131072, 0.15) == 19660 and CONFIGS["C4b"].k == 19661
    assert adaptive_k_window(64, 131072, 0.05) == 6554 == CONFIGS["C4a"].k
    assert adaptive_k_window(64, 131072, 0.30) == 39322 == CONFIGS["C4c"].k
    assert adaptive_k_window(64, 65536, 0.10) == 6554 == CONFIGS["C5"].k


def test_adaptive_invariants_bruteforce():
    for n_kv, kmin, c in itertools.product(range(1, 300), (2, 64), (0.0, 0.1, 0.15, 0.5, 1.0)):
        k = adaptive_k_window(kmin, n_kv, c)
        assert 1 <= k <= n_kv
        assert k >= min(kmin, n_kv)
        assert k % 2 == 0 or k == n_kv
        base = min(max(kmin, math.floor(n_kv * c)), n_kv)
        assert k in (base, base + 1)


def test_adaptive_rejects_bad_args():
    with pytest.raises(ValueError):
        adaptive_k_window(64, 0, 0.15)
    with pytest.raises(ValueError):
        adaptive_k_window(64, 100, 1.5)


# ------------------------------------------------------------------- routing

def test_prefill_always_sdpa():
    cfg = DCRLlamaConfig()
    for N_q, N_kv in itertools.product((2, 16, 512), (1, 4096, 65536)):
        assert route(N_q, N_kv, 0, cfg) is Branch.SDPA


def test_decode_threshold():
    cfg = DCRLlamaConfig(T_dispatch=4096)
    for N_kv in (1, 100, 4095):
        assert route(1, N_kv, 0, cfg) is Branch.SDPA
    for N_kv in (4096, 4097, 32769, 131072):
        assert route(1, N_kv, 0, cfg) is Branch.DCR


def test_enable_dcr_false_and_layer_filter():
    off = DCRLlamaConfig(enable_dcr=False)
    assert all(route(nq, nk, 0, off) is Branch.SDPA for nq in (1, 8) for nk in (1, 10 ** 6))
    cfg = DCRLlamaConfig(layer_filter=frozenset({16, 17, 18}), T_dispatch=4096)
    assert route(1, 8192, 16, cfg) is Branch.DCR
    assert route(1, 8192, 0, cfg) is Branch.SDPA and route(1, 8192, 19, cfg) is Branch.SDPA
    assert route(100, 100, 16, cfg) is Branch.SDPA          # filter never forces DCR
    assert route(1, 1024, 16, cfg) is Branch.SDPA


def test_T_dispatch_extremes():
    assert route(1, 1, 0, DCRLlamaConfig(T_dispatch=0)) is Branch.DCR
    assert route(1, 100_000, 0, DCRLlamaConfig(T_dispatch=10 ** 9)) is Branch.SDPA


def test_explain_route_agrees():
    cfg = DCRLlamaConfig(T_dispatch=4096, layer_filter=frozenset({1}))
    for N_q, N_kv, layer in itertools.product((1, 7), (10, 4096, 9000), (0, 1)):
        b, e = route(N_q, N_kv, layer, cfg), explain_route(N_q, N_kv, layer, cfg)
        assert e.startswith("DCR" if b is Branch.DCR else "SDPA"), e
    e = explain_route(1, 1024, 1, cfg)
    assert "N_kv=1024" in e and "T_dispatch=4096" in e


# -------------------------------------------------------------------- config

def test_config_validation():
    for bad in (dict(k_window=63), dict(k_window=0), dict(T_dispatch=-1),
                dict(axis_source="random"), dict(coverage_floor=1.5)):
        with pytest.raises(ValueError):
            DCRLlamaConfig(**bad)
    with pytest.warns(RuntimeWarning):
        DCRLlamaConfig(coverage_floor=0.05)
    with pytest.warns(RuntimeWarning):
        DCRLlamaConfig(coverage_floor=0.12)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        DCRLlamaConfig(coverage_floor=0.15)
    # the reference's selector value is accepted as an alias of the HIP path
    assert DCRLlamaConfig(axis_source="q_topk_triton").uses_topk_hip
    assert DCRLlamaConfig().uses_topk_hip
    assert not DCRLlamaConfig(axis_source="pca").uses_topk_hip


def test_unbuilt_axis_source_raises_before_any_launch():
    Q = torch.zeros(1, 32, 1, 64)
    K = torch.zeros(1, 32, 8192, 64)
    with pytest.raises(NotImplementedError, match="q_topk_reference"):
        dcr_forward(Q, K, K, DCRLlamaConfig(axis_source="q_topk_reference"), n_rep=4)
