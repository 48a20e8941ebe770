"""CAB KV cache: three-component eviction (reference:
``cab_attention/cache/cab_cache.py`` :20-267). Same configuration, update /
evict control flow and statistics; the selection runs in ``cab_evict_select``
and the pruning of every layer in ``cab_kv_gather``."""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, Optional, Tuple

import torch

from ..eviction import EvictionConfig, ThreeComponentEvictionPolicy
from ..scoring import ImportanceTracker
from .prune import prune_layers


@dataclass
class CABCacheConfig:
    max_cache_size: int = 4096
    sparsity: float = 0.9
    local_ratio: float = 0.3
    bridge_ratio: float = 0.2
    importance_ratio: float = 0.5
    eviction_interval: int = 10
    frc_update_interval: int = 10
    use_triton: bool = True  # accepted, ignored (HIP kernels only)
    device: str = "cuda"


class CABCache:
    """Per-layer K/V storage with amortised three-component eviction."""

    def __init__(self, max_cache_size: int = 4096, sparsity: float = 0.9, local_ratio: float = 0.3,
                 bridge_ratio: float = 0.2, importance_ratio: float = 0.5,
                 eviction_interval: int = 10, frc_update_interval: int = 10,
                 use_triton: bool = True, device: str = "cuda"):
        self.config = CABCacheConfig(max_cache_size, sparsity, local_ratio, bridge_ratio,
                                     importance_ratio, eviction_interval, frc_update_interval,
                                     use_triton, device)
        self.key_cache = []
        self.value_cache = []
        self.importance_tracker = ImportanceTracker(device=device)
        self.eviction_policy = ThreeComponentEvictionPolicy(
            EvictionConfig(local_ratio=local_ratio, bridge_ratio=bridge_ratio,
                           importance_ratio=importance_ratio))
        self.tokens_since_last_eviction = 0
        self.total_evictions = 0
        self.stats = {"total_tokens_processed": 0, "total_evictions": 0,
                      "total_tokens_evicted": 0, "avg_cache_size": 0.0}

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               attention_weights: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """Appends one step's K/V of a layer ([B, H, n, D]) and evicts when
        due; returns the layer's cache."""
        while len(self.key_cache) <= layer_idx:
            self.key_cache.append(None)
            self.value_cache.append(None)
        if self.key_cache[layer_idx] is None:
            self.key_cache[layer_idx] = key_states
            self.value_cache[layer_idx] = value_states
        else:
            self.key_cache[layer_idx] = torch.cat([self.key_cache[layer_idx], key_states], dim=2)
            self.value_cache[layer_idx] = torch.cat([self.value_cache[layer_idx], value_states], dim=2)
        if layer_idx == 0 and attention_weights is not None:
            self.importance_tracker.update(attention_weights)
        self.stats["total_tokens_processed"] += 1
        self.tokens_since_last_eviction += 1
        cache_len = self.key_cache[layer_idx].shape[2]
        should_evict = (cache_len > int(self.config.max_cache_size * 1.1)
                        or self.tokens_since_last_eviction >= self.config.eviction_interval)
        if should_evict and cache_len > self.config.max_cache_size * (1 - self.config.sparsity):
            self._evict()
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def _evict(self):
        if len(self.key_cache) == 0 or self.key_cache[0] is None:
            return
        cache_len = min(k.shape[2] for k in self.key_cache if k is not None)
        keep_size = int(self.config.max_cache_size * (1.0 - self.config.sparsity) * 0.9)
        if cache_len <= keep_size:
            return
        keep_indices, _ = self.eviction_policy.select_indices(
            cache_len=cache_len, keep_size=keep_size,
            importance_scores=self.importance_tracker.get_scores(), attention_matrix=None,
            device=self.config.device)
        prune_layers(self.key_cache, self.value_cache, keep_indices)
        self.importance_tracker.prune(keep_indices)
        self.tokens_since_last_eviction = 0
        self.total_evictions += 1
        self.stats["total_evictions"] += 1
        self.stats["total_tokens_evicted"] += cache_len - keep_indices.numel()
        self.stats["avg_cache_size"] = ((self.stats["avg_cache_size"] * (self.total_evictions - 1)
                                         + keep_indices.numel()) / self.total_evictions)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if layer_idx >= len(self.key_cache) or self.key_cache[layer_idx] is None:
            return 0
        return self.key_cache[layer_idx].shape[2]

    def get_max_length(self) -> int:
        return self.config.max_cache_size

    def reset(self):
        self.key_cache = []
        self.value_cache = []
        self.importance_tracker.reset()
        self.tokens_since_last_eviction = 0
        self.total_evictions = 0

    def get_stats(self) -> Dict[str, Any]:
        cur = self.get_seq_length(0) if len(self.key_cache) > 0 else 0
        m = self.config.max_cache_size
        return {**self.stats, "current_cache_size": cur, "max_cache_size": m,
                "effective_sparsity": 1.0 - (cur / m) if m > 0 else 0.0}

    def __len__(self) -> int:
        return self.get_seq_length(0)

    def __repr__(self) -> str:
        return (f"CABCache(size={self.get_seq_length(0)}/{self.config.max_cache_size}, "
                f"sparsity={self.config.sparsity:.0%}, evictions={self.total_evictions})")
