"""Write the golden fixtures of tests/golden/ (run from the repository root).

    python tests/golden/make_golden.py

The reference ships no golden vectors (its tests draw torch.randn from a
seed), so these fixtures are regression vectors of this build's oracle: the
inputs are regenerated from the seed (dcr_attention_amd.synthetic), and the
expected outputs come from the torch restatement of the reference's M1 path
(oracle/torch_twin.py: the same torch calls as
dcr_attention/kernel/qaxis_topk_reference.py:42-193) and are checked against
the C oracle before they are written.  Input checksums are stored so a test
notices if the generator's stream ever changes.

Fixtures (numpy .npz, no pickles; metadata in golden_meta.json):
  c1_seed0.npz   C1 (B=1, H=32, Hkv=8, N=4096, D=64, fp32), seed 0:
                 u [1,32,64] f32, scores [1,32,4096] u16 (bf16 bits),
                 idx615 / idx614 [1,32,k] i32 (k = ceil(0.15 N) and the
                 caller's adaptive_k_window value), out615 [1,32,64] f32
                 (float64 softmax over the selected rows, rounded once).
  c2b1_idx.npz   C2 with B=1 (N=32768, fp16, outliers), seed 0:
                 idx [1,32,4916] i32 and scores sha256.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
for p in (ROOT, os.path.join(ROOT, "dcr-attention_v3_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import cpu, torch_twin  # noqa: E402
from dcr_attention_amd.synthetic import CONFIGS, make_inputs  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def sha(t: torch.Tensor) -> str:
    t = t.contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.view(torch.int16)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main():
    meta = {}
    cfg = CONFIGS["C1"]
    Q, K, V = make_inputs(cfg, seed=0)
    u = torch_twin.compute_u_Q(Q, 1e-12)
    sc = torch_twin.projection_scores(K, u)
    assert torch.equal(u, cpu.compute_uq(Q)), "twin and C oracle disagree on u"
    assert torch.equal(sc.view(torch.int16), cpu.scores(K, u).view(torch.int16))
    fx = {"u": u.numpy(), "scores": bits16(sc)}
    for k in (615, 614):
        idx = torch_twin.select_topk(sc, k).to(torch.int32)
        assert torch.equal(idx, cpu.topk(sc, k)), f"twin and C oracle disagree on idx k={k}"
        fx[f"idx{k}"] = idx.numpy()
    fx["out615"] = cpu.attention_f64(Q, K, V, torch.from_numpy(fx["idx615"])).float().numpy()
    np.savez_compressed(os.path.join(HERE, "c1_seed0.npz"), **fx)
    meta["c1_seed0"] = {"config": "C1", "seed": 0, "k": [615, 614], "eps": 1e-12,
                        "Q_sha256": sha(Q), "K_sha256": sha(K), "V_sha256": sha(V),
                        "generator": "dcr_attention_amd.synthetic.make_inputs (CPU)"}

    cfg = CONFIGS["C2"]
    Q, K, V = make_inputs(cfg, seed=0, B=1)
    u = cpu.compute_uq(Q)
    sc = cpu.scores(K, u)
    assert torch.equal(sc.view(torch.int16), torch_twin.projection_scores(K, u).view(torch.int16))
    idx = cpu.topk(sc, cfg.k)
    assert torch.equal(idx, torch_twin.select_topk(sc, cfg.k).to(torch.int32))
    np.savez_compressed(os.path.join(HERE, "c2b1_idx.npz"), idx=idx.numpy())
    meta["c2b1_idx"] = {"config": "C2", "B": 1, "seed": 0, "k": cfg.k, "eps": 1e-12,
                        "Q_sha256": sha(Q), "K_sha256": sha(K), "V_sha256": sha(V),
                        "scores_sha256": sha(sc),
                        "generator": "dcr_attention_amd.synthetic.make_inputs (CPU), B=1"}
    with open(os.path.join(HERE, "golden_meta.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
