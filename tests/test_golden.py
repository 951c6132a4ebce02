"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU: the seeded inputs still hash to what the fixtures were made from, and
the C oracle reproduces every fixture bit for bit.
GPU: the HIP path through the C-ABI reproduces u_Q, the bf16 scores and the
index sets bit for bit, and the output within the fp32 bar (1e-5).
"""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import cpu
from dcr_attention_amd.synthetic import CONFIGS, make_inputs

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
META = json.load(open(os.path.join(HERE, "golden_meta.json")))


def _sha(t):
    t = t.contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.view(torch.int16)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()


def _fixture(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _inputs(name):
    m = META[name]
    Q, K, V = make_inputs(CONFIGS[m["config"]], seed=m["seed"], B=m.get("B"))
    assert (_sha(Q), _sha(K), _sha(V)) == (m["Q_sha256"], m["K_sha256"], m["V_sha256"]), \
        "seeded input stream changed; regenerate with tests/golden/make_golden.py"
    return Q, K, V


def _bf16(a):
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)


def test_c1_oracle_matches_fixture():
    Q, K, V = _inputs("c1_seed0")
    fx = _fixture("c1_seed0")
    u = cpu.compute_uq(Q)
    assert np.array_equal(u.numpy(), fx["u"])
    sc = cpu.scores(K, u)
    assert np.array_equal(sc.view(torch.int16).numpy().view(np.uint16), fx["scores"])
    for k in (615, 614):
        assert np.array_equal(cpu.topk(sc, k).numpy(), fx[f"idx{k}"])
    out = cpu.attention_f64(Q, K, V, torch.from_numpy(fx["idx615"])).float()
    assert np.abs(out.numpy() - fx["out615"]).max() <= 1e-6


def test_c1_fixture_structure():
    fx = _fixture("c1_seed0")
    for k in (615, 614):
        idx = fx[f"idx{k}"]
        assert idx.shape == (1, 32, k) and idx.dtype == np.int32
        assert (np.diff(idx, axis=-1) > 0).all()
    # the 614-set is the 615-set minus one element (same ranking, k one smaller)
    a, b = fx["idx615"][0], fx["idx614"][0]
    for h in range(32):
        assert len(np.setdiff1d(a[h], b[h])) == 1 and len(np.setdiff1d(b[h], a[h])) == 0


def test_c2b1_oracle_matches_fixture():
    Q, K, V = _inputs("c2b1_idx")
    fx = _fixture("c2b1_idx")
    sc = cpu.scores(K, cpu.compute_uq(Q))
    assert _sha(sc) == META["c2b1_idx"]["scores_sha256"]
    assert np.array_equal(cpu.topk(sc, META["c2b1_idx"]["k"]).numpy(), fx["idx"])


@pytest.mark.gpu
def test_c1_hip_matches_fixture():
    from dcr_attention_amd.kernel.hip import (compute_u_Q, topk_pass1_projection,
                                              topk_pass2_select, topk_qaxis_attention)
    Q, K, V = _inputs("c1_seed0")
    fx = _fixture("c1_seed0")
    Qd, Kd, Vd = Q.cuda(), K.cuda(), V.cuda()
    u = compute_u_Q(Qd, 1e-12)
    assert np.array_equal(u.cpu().numpy(), fx["u"])
    sc = topk_pass1_projection(Kd, u)
    assert np.array_equal(sc.cpu().view(torch.int16).numpy().view(np.uint16), fx["scores"])
    for k in (615, 614):
        assert np.array_equal(topk_pass2_select(sc, k).cpu().numpy(), fx[f"idx{k}"])
    out, idx = topk_qaxis_attention(Qd, Kd, Vd, 615, return_indices=True)
    assert np.array_equal(idx.cpu().numpy(), fx["idx615"])
    assert np.abs(out.cpu().numpy() - fx["out615"]).max() <= 1e-5


@pytest.mark.gpu
def test_c2b1_hip_matches_fixture():
    from dcr_attention_amd.kernel.hip import topk_qaxis_select
    Q, K, V = _inputs("c2b1_idx")
    fx = _fixture("c2b1_idx")
    idx = topk_qaxis_select(Q.cuda(), K.cuda(), META["c2b1_idx"]["k"])
    assert np.array_equal(idx.cpu().numpy(), fx["idx"])
