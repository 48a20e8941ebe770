"""CABAttention: multi-head attention whose key blocks are chosen by the
coarse curvature predictor and executed by the block-sparse HIP kernel.

Same class, constructor and forward contract as the reference's
``cab_attention/cab_attention.py`` (absent from the reference tree; contract:
README.md:75-112, examples/demo_cab_attention.py:36-63). The QKV and output
projections are torch ``nn.Linear`` layers (hipBLASLt GEMMs); the predictor
and the sparse executor are this package's HIP kernels.
"""

from __future__ import annotations

import torch
from torch import nn

from .coarse_predictor import CoarseCurvaturePredictor
from .kernels.sparse_attention import (SUPPORTED_BLOCK_SIZES, SUPPORTED_HEAD_DIMS,
                                       block_sparse_attention)


class CABAttention(nn.Module):
    """Curvature-aware block-sparse multi-head self-attention.

    Args:
        dim: model width; ``dim % num_heads == 0`` and ``dim / num_heads``
            (the head dim) 64 or 128.
        num_heads: attention heads.
        block_size: tokens per block (predictor and executor); 64.
        sparsity: fraction of key blocks pruned per query block.
        lambda_redundancy: FRC redundancy weight.
        causal: token-causal attention (the predictor keeps only j <= i).
        qkv_bias: bias of the QKV projection.
        predictor_kwargs: forwarded to :class:`CoarseCurvaturePredictor`.
    """

    def __init__(self, dim: int, num_heads: int, block_size: int = 64, sparsity: float = 0.95,
                 lambda_redundancy: float = 0.5, causal: bool = False, qkv_bias: bool = False,
                 **predictor_kwargs):
        super().__init__()
        if dim % num_heads:
            raise ValueError(f"dim={dim} is not divisible by num_heads={num_heads}")
        if dim // num_heads not in SUPPORTED_HEAD_DIMS:
            raise ValueError(f"head_dim = dim / num_heads = {dim // num_heads} is not supported by "
                             f"the block-sparse executor (head_dim in {SUPPORTED_HEAD_DIMS})")
        if int(block_size) not in SUPPORTED_BLOCK_SIZES:
            raise ValueError(f"block_size={block_size} is not supported by the block-sparse "
                             f"executor (block_size in {SUPPORTED_BLOCK_SIZES}); "
                             "CoarseCurvaturePredictor alone accepts any block size")
        self.dim = dim
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.causal = bool(causal)
        self.qkv = nn.Linear(dim, 3 * dim, bias=qkv_bias)
        self.proj = nn.Linear(dim, dim)
        self.predictor = CoarseCurvaturePredictor(block_size=block_size, sparsity=sparsity,
                                                  lambda_redundancy=lambda_redundancy,
                                                  causal=causal, **predictor_kwargs)

    def attend(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
               return_diagnostics: bool = False, out: torch.Tensor | None = None):
        """Predictor + sparse executor on ``[B, H, N, D]`` q, k, v."""
        pred = self.predictor.predict_index(q, k, return_diagnostics=return_diagnostics)
        kv_idx, kv_cnt = pred[0], pred[1]
        o = block_sparse_attention(q, k, v, kv_idx, kv_cnt, block_size=self.predictor.block_size,
                                   causal=self.causal, out=out)
        return (o, pred[2]) if return_diagnostics else o

    def forward(self, x: torch.Tensor, return_diagnostics: bool = False):
        """``x [B, N, dim]`` -> ``[B, N, dim]`` (and the predictor's
        diagnostics dict with ``return_diagnostics``)."""
        B, N, C = x.shape
        H, Dh = self.num_heads, self.head_dim
        qkv = self.qkv(x).view(B, N, 3, H, Dh)
        q = qkv[:, :, 0].transpose(1, 2)  # [B, H, N, Dh] views, last dim contiguous
        k = qkv[:, :, 1].transpose(1, 2)
        v = qkv[:, :, 2].transpose(1, 2)
        o = torch.empty((B, N, H, Dh), dtype=x.dtype, device=x.device)
        res = self.attend(q, k, v, return_diagnostics=return_diagnostics, out=o.transpose(1, 2))
        y = self.proj(o.view(B, N, C))
        return (y, res[1]) if return_diagnostics else y
