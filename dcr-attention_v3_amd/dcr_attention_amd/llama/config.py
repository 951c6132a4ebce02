"""Caller configuration of the sparse decode path.

Mirrors ``DCRLlamaConfig`` (reference dcr_attention/models/llama/config.py:17-134):
same field names, defaults and validation, so a configuration written for the
reference loads unchanged.  ``axis_source`` accepts the reference's values
plus ``"q_topk_hip"``; ``"q_topk_triton"`` is treated as an alias of it (the
caller's drop-in point, attention.py:805); ``"q"``, ``"pca"`` and
``"positional"`` run the rank-local window (attention.py:816-880) along the
query's direction or the keys' principal direction.  The pure-torch M1
reference (``"q_topk_reference"``) is accepted by the validator, for
loading, but not run: the decode caller raises NotImplementedError for it.
"""
from __future__ import annotations

import warnings
from dataclasses import dataclass
from typing import FrozenSet, Literal, Optional

AxisSource = Literal["pca", "positional", "q", "q_topk_reference", "q_topk_triton", "q_topk_hip"]

AXIS_SOURCES = ("pca", "positional", "q", "q_topk_reference", "q_topk_triton", "q_topk_hip")
#: axis sources that route to the HIP top-K path of this build
TOPK_HIP_SOURCES = ("q_topk_hip", "q_topk_triton")


@dataclass(frozen=True)
class DCRLlamaConfig:
    """Knobs of the DCR decode caller.

    k_window        minimum top-K size (positive, even); ``adaptive_k_window``
                    raises it to the coverage floor.
    T_dispatch      decode steps with fewer cached keys than this go dense.
    axis_source     which selection path the DCR branch runs (see module doc).
    enable_dcr      master switch; False routes everything to dense attention.
    layer_filter    if set, only these layer indices use DCR.
    coverage_floor  c in k_eff = max(k_window, int(N_kv * c)) (capped at N_kv,
                    rounded up to even).  Below 0.15 the reference documents a
                    perplexity cost and warns; below 0.10 it calls the result
                    unusable.
    enable_adaptive_widening  rank-local windows only: retry a leaky
                    window once at twice the size; the top-K path has no
                    widening step.
    """

    k_window: int = 64
    T_dispatch: int = 4096
    axis_source: AxisSource = "q_topk_hip"
    enable_dcr: bool = True
    layer_filter: Optional[FrozenSet[int]] = None
    coverage_floor: float = 0.15
    enable_adaptive_widening: bool = False

    def __post_init__(self) -> None:
        if self.k_window <= 0 or self.k_window % 2 != 0:
            raise ValueError(f"k_window must be a positive even integer, got {self.k_window}")
        if self.T_dispatch < 0:
            raise ValueError(f"T_dispatch must be >= 0, got {self.T_dispatch}")
        if self.axis_source not in AXIS_SOURCES:
            raise ValueError(f"axis_source must be one of {AXIS_SOURCES}, got {self.axis_source!r}")
        if not (0.0 <= self.coverage_floor <= 1.0):
            raise ValueError(f"coverage_floor must be in [0, 1], got {self.coverage_floor}")
        if self.coverage_floor < 0.10:
            warnings.warn(f"coverage_floor={self.coverage_floor} is below the validated range "
                          "(the reference reports > 2% perplexity loss); use >= 0.15.",
                          RuntimeWarning, stacklevel=3)
        elif self.coverage_floor < 0.15:
            warnings.warn(f"coverage_floor={self.coverage_floor} is in the permissive regime "
                          "(~1% perplexity loss at N=32K in the reference); 0.15 is strict.",
                          RuntimeWarning, stacklevel=3)

    @property
    def uses_topk_hip(self) -> bool:
        return self.axis_source in TOPK_HIP_SOURCES


DEFAULT_DCR_LLAMA_CONFIG = DCRLlamaConfig()
