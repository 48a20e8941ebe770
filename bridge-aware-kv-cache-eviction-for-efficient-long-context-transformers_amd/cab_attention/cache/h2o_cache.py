"""H2O KV cache: keeps the positions with the highest cumulative attention
(reference: ``cab_attention/cache/h2o_cache.py`` :18-197). Selection in
``cab_evict_select`` (via the tracker), pruning in ``cab_kv_gather``."""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch

from ..scoring import ImportanceTracker
from .prune import prune_layers


class H2OCache:
    def __init__(self, max_cache_size: int = 4096, sparsity: float = 0.9,
                 eviction_interval: int = 10, device: str = "cuda"):
        self.max_cache_size = max_cache_size
        self.sparsity = sparsity
        self.eviction_interval = eviction_interval
        self.device = device
        self.key_cache = []
        self.value_cache = []
        self.importance_tracker = ImportanceTracker(device=device)
        self.tokens_since_last_eviction = 0
        self.total_evictions = 0
        self.stats = {"total_tokens_processed": 0, "total_evictions": 0, "total_tokens_evicted": 0}

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               attention_weights: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
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
        if (cache_len > int(self.max_cache_size * 1.1)
                or self.tokens_since_last_eviction >= self.eviction_interval):
            self._evict()
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def _evict(self):
        if len(self.key_cache) == 0 or self.key_cache[0] is None:
            return
        cache_len = min(k.shape[2] for k in self.key_cache if k is not None)
        keep_size = int(self.max_cache_size * (1.0 - self.sparsity) * 0.9)
        if cache_len <= keep_size:
            return
        keep_indices = self.importance_tracker.get_top_k_indices(k=keep_size).sort().values
        prune_layers(self.key_cache, self.value_cache, keep_indices)
        self.importance_tracker.prune(keep_indices)
        self.tokens_since_last_eviction = 0
        self.total_evictions += 1
        self.stats["total_evictions"] += 1
        self.stats["total_tokens_evicted"] += cache_len - keep_indices.numel()

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if layer_idx >= len(self.key_cache) or self.key_cache[layer_idx] is None:
            return 0
        return self.key_cache[layer_idx].shape[2]

    def get_max_length(self) -> int:
        return self.max_cache_size

    def reset(self):
        self.key_cache = []
        self.value_cache = []
        self.importance_tracker.reset()
        self.tokens_since_last_eviction = 0
        self.total_evictions = 0

    def get_stats(self) -> Dict[str, Any]:
        cur = self.get_seq_length(0) if len(self.key_cache) > 0 else 0
        return {**self.stats, "current_cache_size": cur, "max_cache_size": self.max_cache_size}

    def __len__(self) -> int:
        return self.get_seq_length(0)

    def __repr__(self) -> str:
        return (f"H2OCache(size={self.get_seq_length(0)}/{self.max_cache_size}, "
                f"sparsity={self.sparsity:.0%}, evictions={self.total_evictions})")
