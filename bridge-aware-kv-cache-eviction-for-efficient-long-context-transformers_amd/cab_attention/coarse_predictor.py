"""CoarseCurvaturePredictor: Q, K -> block mask (coarsen -> FRC -> top-k).

Same class, constructor arguments, attributes and forward contract as the
reference's ``cab_attention/coarse_predictor.py`` (absent from the reference
tree; contract: README.md:116-129, examples/demo_cab_attention.py:76-115,
:192-207, benchmarks/benchmark_predictor.py:59-63, :94, :114-130). All three
stages run as HIP kernels on the GPU.
"""

from __future__ import annotations

import torch
from torch import nn

from .kernels.coarsening import coarsen_qk_max_l2
from .kernels.frc_kernel import compute_block_frc, generate_block_index, keep_count


class CoarseCurvaturePredictor(nn.Module):
    """Predicts which key blocks each query block attends to.

    Args:
        block_size: tokens per block (README.md:83).
        sparsity: fraction of blocks pruned per row (0.95 keeps 5%).
        lambda_redundancy: weight of the 2-hop redundancy term (README.md:122).
        use_triton: accepted for signature compatibility
            (benchmark_predictor.py:62) and ignored: the kernels are HIP.
        formula: ``additive`` (default), ``multiplicative`` or ``augmented``.
        normalization: ``minmax`` (default) or ``none``.
        temperature: affinity temperature.
        select_high: keep the highest FRC instead of the lowest.
        keep_diagonal: always keep block i in row i.
        causal: candidates restricted to j <= i.
    """

    def __init__(self, block_size: int = 64, sparsity: float = 0.95,
                 lambda_redundancy: float = 0.5, use_triton=None, formula: str = "additive",
                 normalization: str = "minmax", temperature: float = 1.0,
                 select_high: bool = False, keep_diagonal: bool = True, causal: bool = False):
        super().__init__()
        if int(block_size) < 1:
            raise ValueError(f"block_size must be >= 1, got {block_size}")
        if not 0.0 <= float(sparsity) <= 1.0:
            raise ValueError(f"sparsity must be in [0, 1], got {sparsity}")
        self.block_size = int(block_size)
        self.sparsity = float(sparsity)
        self.lambda_redundancy = float(lambda_redundancy)
        self.use_triton = use_triton
        self.formula = formula
        self.normalization = normalization
        self.temperature = float(temperature)
        self.select_high = bool(select_high)
        self.keep_diagonal = bool(keep_diagonal)
        self.causal = bool(causal)

    def extra_repr(self) -> str:
        return (f"block_size={self.block_size}, sparsity={self.sparsity}, "
                f"lambda_redundancy={self.lambda_redundancy}, formula={self.formula!r}, "
                f"normalization={self.normalization!r}, causal={self.causal}")

    def _scores(self, q: torch.Tensor, k: torch.Tensor, diagnostics: bool):
        qc, kc = coarsen_qk_max_l2(q, k, self.block_size)
        return compute_block_frc(qc, kc, temperature=self.temperature,
                                 lambda_redundancy=self.lambda_redundancy, formula=self.formula,
                                 normalization=self.normalization, diagnostics=diagnostics)

    def predict_index(self, q: torch.Tensor, k: torch.Tensor, return_diagnostics: bool = False,
                      dense: bool = False):
        """Compact prediction for the sparse executor: ``(kv_idx, kv_cnt)``
        (plus the dense mask when ``dense``; plus the diagnostics dict when
        ``return_diagnostics``)."""
        frc, aff, tri = self._scores(q, k, return_diagnostics)
        kv_idx, kv_cnt, mask = generate_block_index(
            frc, self.sparsity, select_high=self.select_high, keep_diagonal=self.keep_diagonal,
            causal=self.causal, dense=dense or return_diagnostics)
        out = (kv_idx, kv_cnt) + ((mask,) if dense else ())
        if return_diagnostics:
            return out + (self._diagnostics(kv_cnt, frc, aff, tri),)
        return out

    def _diagnostics(self, kv_cnt, frc, aff, tri) -> dict:
        B, H, M = kv_cnt.shape
        kept = float(kv_cnt.sum().item())
        return {
            "effective_sparsity": 1.0 - kept / float(B * H * M * M) if M else 0.0,
            "num_blocks": M,
            "frc_scores": frc,
            "affinity": aff,
            "triangles": tri,
        }

    def forward(self, q: torch.Tensor, k: torch.Tensor, return_diagnostics: bool = False):
        """``q, k [B, H, N, D]`` -> bool block mask ``[B, H, M, M]``; with
        ``return_diagnostics`` also ``{'effective_sparsity', 'num_blocks',
        'frc_scores', 'affinity', 'triangles'}`` (demo:56-57, :109-115)."""
        frc, aff, tri = self._scores(q, k, return_diagnostics)
        kv_idx, kv_cnt, mask = generate_block_index(
            frc, self.sparsity, select_high=self.select_high, keep_diagonal=self.keep_diagonal,
            causal=self.causal, dense=True)
        if return_diagnostics:
            return mask, self._diagnostics(kv_cnt, frc, aff, tri)
        return mask

    def keep_per_row(self, seq_len: int) -> int:
        """Blocks kept per (non-causal) row for a sequence of ``seq_len`` tokens."""
        m = (seq_len + self.block_size - 1) // self.block_size
        return keep_count(m, self.sparsity)

    def estimate_flops(self, N: int, D: int) -> dict:
        """Per-(b, h) operation counts: ``coarsening = 2 N D``,
        ``matmul = 2 M^2 D`` (affinity), ``triangles = 2 M^3`` (T = A @ A:
        M^3 multiply-adds, the demo's "M^3 ops", demo:209-210) and ``total``."""
        m = (int(N) + self.block_size - 1) // self.block_size
        c = 2 * int(N) * int(D)
        a = 2 * m * m * int(D)
        t = 2 * m ** 3
        return {"M": m, "coarsening": c, "matmul": a, "triangles": t, "total": c + a + t}
