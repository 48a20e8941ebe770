"""Token-level FRC tracking for bridge detection (reference:
``cab_attention/scoring/frc.py`` :16-199). Same constructor, methods, update
interval and return values; the curvature runs in
``cab_token_frc_from_keys`` / ``cab_attention_symmetrize`` +
``cab_token_frc``, and the key-similarity graph of ``compute_from_keys`` is
never formed."""

from __future__ import annotations

from typing import Optional

import torch

from ..kernels.token_frc import compute_frc, frc_from_keys, symmetrize_attention


class FRCTracker:
    """Token FRC scores of the cached positions: lower = bridge (keep),
    higher = redundant."""

    def __init__(self, device: str = "cuda", use_triton: bool = True):
        self.device = device
        self.use_triton = use_triton  # accepted, ignored (HIP kernels only)
        self.frc_scores = None
        self.last_update_len = 0
        self.update_interval = 10  # recompute at most every 10 new positions

    def reset(self):
        self.frc_scores = None
        self.last_update_len = 0

    def compute_from_keys(self, keys: torch.Tensor, force_update: bool = False) -> torch.Tensor:
        """FRC ``[N]`` of the key-similarity graph of ``keys [B, H, N, D]``:
        the (b, h)-mean keys, L2-normalised, relu of their dot products,
        rows normalised to sum 1 (frc.py:68-89). Within ``update_interval``
        new positions of the last computation the cached scores are returned,
        extended with zeros (frc.py:53-66). Scores are in the keys' dtype."""
        N = keys.shape[2]
        if not force_update and self.frc_scores is not None:
            if N - self.last_update_len < self.update_interval:
                if N > len(self.frc_scores):
                    pad = torch.zeros(N - len(self.frc_scores), device=self.frc_scores.device,
                                      dtype=self.frc_scores.dtype)
                    self.frc_scores = torch.cat([self.frc_scores, pad])
                return self.frc_scores
        frc_scores = frc_from_keys(keys).to(keys.dtype)
        self.frc_scores = frc_scores
        self.last_update_len = N
        return frc_scores

    def compute_from_attention(self, attention: torch.Tensor) -> torch.Tensor:
        """FRC ``[N]`` of ``attention [N, N]``, or of ``(agg.T + agg) / 2`` with
        ``agg`` the (b, h)-mean of ``attention [B, H, N_q, N_kv]``
        (frc.py:110-130)."""
        if attention.dim() == 4:
            matrix = symmetrize_attention(attention).to(attention.dtype)
        else:
            matrix = attention
        matrix = matrix.to(self.device)
        frc_scores = compute_frc(matrix, use_triton=self.use_triton)
        self.frc_scores = frc_scores
        self.last_update_len = len(frc_scores)
        return frc_scores

    def get_bottom_k_indices(self, k: int, exclude_indices: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The k lowest-FRC positions, lowest first (equal scores in position
        order; NaN last), excluding ``exclude_indices`` (frc.py:138-170)."""
        if self.frc_scores is None:
            return torch.tensor([], dtype=torch.long, device=self.device)
        scores = self.frc_scores.clone()
        if exclude_indices is not None and len(exclude_indices) > 0:
            scores[exclude_indices] = float("inf")
        k = min(k, len(scores))
        if k == 0:
            return torch.tensor([], dtype=torch.long, device=self.device)
        return torch.sort(scores, stable=True).indices[:k]

    def get_scores(self) -> Optional[torch.Tensor]:
        return self.frc_scores

    def prune(self, keep_indices: torch.Tensor):
        """Keeps the scores of the kept positions (frc.py:176-195)."""
        if self.frc_scores is not None:
            valid = keep_indices[keep_indices < len(self.frc_scores)]
            if len(valid) > 0:
                self.frc_scores = self.frc_scores[valid]
                self.last_update_len = len(self.frc_scores)
            else:
                self.frc_scores = None
                self.last_update_len = 0

    def __len__(self) -> int:
        return 0 if self.frc_scores is None else len(self.frc_scores)
