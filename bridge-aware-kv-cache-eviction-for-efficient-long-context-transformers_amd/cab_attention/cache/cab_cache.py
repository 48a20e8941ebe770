"""CAB KV cache: local window + importance + bridge positions.

Drop-in for the reference's ``CABCache`` / ``CABCacheConfig``
(cab_attention/cache/cab_cache.py:20-267): same constructor arguments,
``update(key_states, value_states, layer_idx, attention_weights)``, the HF
cache queries and the statistics keys. The eviction core, the device store
and the selection (``ThreeComponentEvictionPolicy`` on ``cab_evict_select``)
are this package's own (``store.py``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict

import torch

from ..eviction import EvictionConfig, ThreeComponentEvictionPolicy
from .store import EvictingCache


@dataclass
class CABCacheConfig:
    """The cache's settings (cab_cache.py:20-38). ``use_triton`` is accepted
    and ignored: the kernels are HIP only."""
    max_cache_size: int = 4096
    sparsity: float = 0.9
    local_ratio: float = 0.3
    bridge_ratio: float = 0.2
    importance_ratio: float = 0.5
    eviction_interval: int = 10
    frc_update_interval: int = 10
    use_triton: bool = True
    device: str = "cuda"


class CABCache(EvictingCache):
    """Evicts to the three-component policy's positions. It never evicts
    while a layer holds at most ``max_cache_size * (1 - sparsity)`` rows;
    ``stats['avg_cache_size']`` is the mean number of positions kept per
    eviction."""

    def __init__(self, max_cache_size: int = 4096, sparsity: float = 0.9, local_ratio: float = 0.3,
                 bridge_ratio: float = 0.2, importance_ratio: float = 0.5,
                 eviction_interval: int = 10, frc_update_interval: int = 10,
                 use_triton: bool = True, device: str = "cuda"):
        self.config = CABCacheConfig(max_cache_size=max_cache_size, sparsity=sparsity,
                                     local_ratio=local_ratio, bridge_ratio=bridge_ratio,
                                     importance_ratio=importance_ratio,
                                     eviction_interval=eviction_interval,
                                     frc_update_interval=frc_update_interval,
                                     use_triton=use_triton, device=device)
        self.eviction_policy = ThreeComponentEvictionPolicy(
            EvictionConfig(local_ratio=local_ratio, bridge_ratio=bridge_ratio,
                           importance_ratio=importance_ratio))
        super().__init__(max_cache_size, sparsity, eviction_interval, device,
                         floor=max_cache_size * (1.0 - sparsity), selector=self._select)
        self.stats["avg_cache_size"] = 0.0

    def _select(self, cache_len: int, keep_size: int) -> torch.Tensor:
        # The O(N) bridge rule (median of the importance scores): no
        # attention matrix is formed.
        keep, _ = self.eviction_policy.select_indices(
            cache_len=cache_len, keep_size=keep_size,
            importance_scores=self.importance_tracker.get_scores(), attention_matrix=None,
            device=self.config.device)
        return keep

    def _on_evicted(self, cache_len: int, kept: int):
        super()._on_evicted(cache_len, kept)
        n = self.total_evictions
        self.stats["avg_cache_size"] += (kept - self.stats["avg_cache_size"]) / n

    def get_stats(self) -> Dict[str, Any]:
        out = super().get_stats()
        m = self.max_cache_size
        out["effective_sparsity"] = 1.0 - out["current_cache_size"] / m if m > 0 else 0.0
        return out
