"""H2O KV cache: keeps the positions with the highest cumulative attention.

Drop-in for the reference's ``H2OCache`` (cab_attention/cache/h2o_cache.py:18-197):
same constructor arguments, ``update``, HF cache queries and statistics
keys, on the shared eviction core (``store.py``); the top-k runs in
``cab_evict_select`` through the importance tracker.
"""

from __future__ import annotations

import torch

from .store import EvictingCache


class H2OCache(EvictingCache):
    """Evicts to the ``keep_size`` most attended positions, in position order."""

    def __init__(self, max_cache_size: int = 4096, sparsity: float = 0.9,
                 eviction_interval: int = 10, device: str = "cuda"):
        super().__init__(max_cache_size, sparsity, eviction_interval, device,
                         floor=float("-inf"), selector=self._select)

    def _select(self, cache_len: int, keep_size: int) -> torch.Tensor:
        top = self.importance_tracker.get_top_k_indices(k=keep_size)
        return torch.sort(top).values
