"""Per-call branch choice of the decode caller.

Same decision as the reference's ``route`` / ``explain_route``
(dcr_attention/models/llama/routing.py:28-91): pure integer logic, in order
  enable_dcr off -> dense; layer not in layer_filter -> dense;
  prefill (N_q > 1) -> dense; N_kv < T_dispatch -> dense; else DCR.
"""
from __future__ import annotations

from enum import Enum

from dcr_attention_amd.llama.config import DCRLlamaConfig


class Branch(Enum):
    SDPA = "sdpa"
    DCR = "dcr"


def _reason(N_q: int, N_kv: int, layer_idx: int, cfg: DCRLlamaConfig):
    if not cfg.enable_dcr:
        return Branch.SDPA, "SDPA: enable_dcr=False"
    if cfg.layer_filter is not None and layer_idx not in cfg.layer_filter:
        return Branch.SDPA, f"SDPA: layer_idx={layer_idx} not in layer_filter"
    if N_q > 1:
        return Branch.SDPA, f"SDPA: prefill (N_q={N_q})"
    if N_kv < cfg.T_dispatch:
        return Branch.SDPA, f"SDPA: short context (N_kv={N_kv} < T_dispatch={cfg.T_dispatch})"
    return Branch.DCR, f"DCR: decode + long context (N_kv={N_kv} >= T_dispatch={cfg.T_dispatch})"


def route(N_q: int, N_kv: int, layer_idx: int, cfg: DCRLlamaConfig) -> Branch:
    """Dense (SDPA) or DCR for one attention call."""
    return _reason(N_q, N_kv, layer_idx, cfg)[0]


def explain_route(N_q: int, N_kv: int, layer_idx: int, cfg: DCRLlamaConfig) -> str:
    """Human-readable reason for ``route``'s decision (starts with the branch)."""
    return _reason(N_q, N_kv, layer_idx, cfg)[1]
