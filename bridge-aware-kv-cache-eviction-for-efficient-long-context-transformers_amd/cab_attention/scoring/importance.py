"""Cumulative-attention (H2O) importance tracking (reference:
``cab_attention/scoring/importance.py`` :17-133). The running totals are
torch bookkeeping; the top-k runs in ``cab_evict_select``."""

from __future__ import annotations

from typing import Optional

import torch

from ..eviction._select import BRIDGE_NONE, select_positions


class ImportanceTracker:
    """Running sum of the attention each cached position receives."""

    def __init__(self, device: str = "cuda"):
        self.device = device
        self.cumulative_scores = None
        self.total_queries = 0

    def reset(self):
        self.cumulative_scores = None
        self.total_queries = 0

    def update(self, attention_weights: torch.Tensor):
        """Adds ``attention_weights [B, H, N_q, N_kv]`` summed over batch,
        heads and queries; a longer N_kv extends the totals with zeros."""
        position_scores = attention_weights.sum(dim=(0, 1, 2)).float()
        if self.cumulative_scores is None:
            self.cumulative_scores = position_scores
        else:
            cur, cached = position_scores.numel(), self.cumulative_scores.numel()
            if cur > cached:
                self.cumulative_scores = torch.cat([
                    self.cumulative_scores,
                    torch.zeros(cur - cached, device=self.cumulative_scores.device,
                                dtype=self.cumulative_scores.dtype)])
            self.cumulative_scores[:cur] += position_scores
        self.total_queries += attention_weights.shape[2]

    def add_scores(self, position_scores: torch.Tensor, n_queries: int = 1):
        """Adds per-position totals already summed over queries (for example
        the key totals of ``flash_attention_with_cumulative_scores``, summed
        over batch and heads)."""
        self.update(position_scores.reshape(1, 1, 1, -1))
        self.total_queries += n_queries - 1

    def get_top_k_indices(self, k: int, exclude_indices: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The k highest-scoring positions, highest first (equal scores in
        position order), or an empty tensor before any update."""
        if self.cumulative_scores is None:
            return torch.arange(0, 0, device=self.device)
        scores = self.cumulative_scores
        if exclude_indices is not None and len(exclude_indices) > 0:
            scores = scores.clone()
            scores[exclude_indices] = -float("inf")
        n = scores.numel()
        k = min(k, n)
        keep, _, _, _ = select_positions(n, scores, 0, k, 0, False, BRIDGE_NONE, scores.device)
        vals = scores[keep]
        nan = torch.isnan(vals)
        order = torch.sort(torch.where(nan, torch.full_like(vals, float("inf")), vals), stable=True,
                           descending=True).indices
        order = order[torch.sort(nan[order].to(torch.uint8), stable=True, descending=True).indices]
        return keep[order]

    def get_scores(self) -> Optional[torch.Tensor]:
        return self.cumulative_scores

    def prune(self, keep_indices: torch.Tensor):
        """Keeps the totals of the kept positions (in order)."""
        if self.cumulative_scores is not None:
            valid = keep_indices[keep_indices < self.cumulative_scores.numel()]
            self.cumulative_scores = self.cumulative_scores[valid] if valid.numel() > 0 else None

    def __len__(self) -> int:
        return 0 if self.cumulative_scores is None else self.cumulative_scores.numel()
