"""H2O (heavy-hitter) selection: local window + highest cumulative attention.

Same function, arguments and return values as the reference's
``cab_attention/eviction/h2o.py`` (:16-94); the selection runs in the HIP
kernel ``cab_evict_select`` (ties to the lower position, NaN above +inf).
"""

from __future__ import annotations

from typing import Tuple

import torch

from ._select import BRIDGE_NONE, select_positions


def h2o_select_indices(cache_len: int, keep_size: int, importance_scores: torch.Tensor,
                       local_ratio: float = 0.2, device: str = "cuda") -> Tuple[torch.Tensor, dict]:
    """Keeps the last ``max(1, int(keep_size * local_ratio))`` positions and
    the highest-scoring others, up to ``keep_size`` in all (ascending int64),
    with a diagnostics dict."""
    local_size = max(1, int(keep_size * local_ratio))
    important_size = keep_size - local_size
    local_size = min(local_size, cache_len)
    important_size = min(important_size, cache_len - local_size)
    imp = important_size if (importance_scores is not None and important_size > 0) else 0
    keep, (n_loc, n_imp, _), _, _ = select_positions(cache_len, importance_scores, local_size, imp,
                                                     0, False, BRIDGE_NONE, device)
    diagnostics = {
        "local_count": n_loc,
        "important_count": n_imp,
        "total_kept": keep.numel(),
        "cache_len": cache_len,
        "target_size": keep_size,
    }
    return keep, diagnostics
