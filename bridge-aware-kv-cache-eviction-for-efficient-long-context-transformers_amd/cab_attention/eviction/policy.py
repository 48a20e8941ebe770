"""Three-component eviction policy: local window, importance (highest
cumulative attention) and bridges.

Same classes, arguments and return values as the reference's
``cab_attention/eviction/policy.py`` (:17-225); the selection runs in one
HIP kernel (``cab_evict_select``). Decisions where the reference leaves the
result to ``torch.topk``'s unspecified tie order: equal scores go to the
lower position, NaN ranks above +inf, and a position already kept is never
chosen again.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from ._select import (BRIDGE_MEDIAN, BRIDGE_NONE, BRIDGE_POSITIONAL, BRIDGE_SCORES, connectivity,
                      select_positions)


@dataclass
class EvictionConfig:
    """Budget split of the kept positions (policy.py:17-27)."""
    local_ratio: float = 0.3
    bridge_ratio: float = 0.2
    importance_ratio: float = 0.5

    def __post_init__(self):
        total = self.local_ratio + self.bridge_ratio + self.importance_ratio
        if abs(total - 1.0) >= 1e-6:
            raise ValueError(f"Ratios must sum to 1.0, got {total}")


class ThreeComponentEvictionPolicy:
    """Keeps the local window, the most attended positions, and bridge
    positions (policy.py:29-225)."""

    def __init__(self, config: EvictionConfig):
        self.config = config

    def select_indices(self, cache_len: int, keep_size: int,
                       importance_scores: Optional[torch.Tensor],
                       attention_matrix: Optional[torch.Tensor] = None,
                       device: str = "cuda") -> Tuple[torch.Tensor, dict]:
        """Positions to keep (ascending int64) and a diagnostics dict.

        Budgets: local = int(keep * local_ratio), bridge = int(keep *
        bridge_ratio), importance = the rest, each at most cache_len.
        Importance takes the highest ``importance_scores`` (zero-padded or
        truncated to cache_len) outside the local window; bridges take, among
        the positions still free, the highest attention-matrix connectivity
        to the importance positions when ``attention_matrix`` is given, else
        the scores nearest their lower median, else the middle third.
        """
        c = self.config
        local = min(int(keep_size * c.local_ratio), cache_len)
        bridge = min(int(keep_size * c.bridge_ratio), cache_len)
        imp = min(keep_size - int(keep_size * c.local_ratio) - int(keep_size * c.bridge_ratio),
                  cache_len)
        imp = max(imp, 0)
        scores = importance_scores
        if bridge <= 0:
            mode = BRIDGE_NONE
        elif attention_matrix is not None:
            mode = BRIDGE_SCORES
        elif scores is not None:
            mode = BRIDGE_MEDIAN
        else:
            mode = BRIDGE_POSITIONAL
        bridge_scores = None
        if mode == BRIDGE_SCORES:
            # the importance positions first, then their connectivity
            _, (_, n_imp, _), cat, _ = select_positions(cache_len, scores, local, imp, 0, True,
                                                        BRIDGE_NONE, device, category=True)
            if n_imp > 0:
                bridge_scores = connectivity(attention_matrix, cat)
        keep, (n_loc, n_imp, n_br), _, _ = select_positions(
            cache_len, scores, local, imp, bridge, True, mode, device, bridge_scores=bridge_scores)
        total = keep.numel()
        diagnostics = {
            "cache_len": cache_len,
            "keep_size": total,
            "local_count": n_loc,
            "importance_count": n_imp,
            "bridge_count": n_br,
            "local_ratio_actual": n_loc / total if total > 0 else 0,
            "importance_ratio_actual": n_imp / total if total > 0 else 0,
            "bridge_ratio_actual": n_br / total if total > 0 else 0,
        }
        return keep, diagnostics
