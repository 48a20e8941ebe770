"""Max-L2 coarsening of Q and K (HIP kernel ``cab_coarsen_maxl2``).

Same names and call contract as the reference's
``cab_attention/kernels/coarsening.py`` (absent from the reference tree; its
callers are benchmarks/kernel_benchmark.py:23, :82-85,
benchmarks/quick_kernel_test.py:54-61, experiments/longbench_qa/methods.py:303,
:424 and CAB_Attention_Colab.ipynb:109-141): ``coarsen_qk_max_l2(q, k,
block_size) -> (q_coarse, k_coarse)`` with ``q, k [B, H, N, D]`` and outputs
``[B, H, M, D]``, ``M = ceil(N / block_size)``, in the input dtype.
"""

from __future__ import annotations

import torch

from .. import _native as nat


def coarsen_qk_max_l2(q: torch.Tensor, k: torch.Tensor, block_size: int = 64,
                      return_indices: bool = False):
    """Max-L2 pooling: per block, the token with the largest L2 norm.

    For each (b, h, block) of q and of k separately, the representative is
    the token whose squared norm is largest (float64, fixed summation order,
    first token on ties, NaN counts as largest; a ragged last block looks at
    its valid tokens only) and its row is copied bit for bit
    (README.md:30-33). With ``return_indices`` the absolute token indices
    ``(q_idx, k_idx)`` (int32 ``[B, H, M]``) are returned as well.
    """
    if q.dim() != 4 or k.dim() != 4:
        raise ValueError(f"q and k must be [B, H, N, D]; got {tuple(q.shape)} and {tuple(k.shape)}")
    if q.shape != k.shape:
        raise ValueError(f"q and k shapes differ: {tuple(q.shape)} vs {tuple(k.shape)}")
    if q.dtype != k.dtype:
        raise TypeError(f"q and k dtypes differ: {q.dtype} vs {k.dtype}")
    block_size = int(block_size)
    if block_size < 1:
        raise ValueError(f"block_size must be >= 1, got {block_size}")
    dev = nat.require_device(q, k)
    lib = nat.load()
    dt = nat.dtype_code(q)
    B, H, N, D = q.shape
    M = (N + block_size - 1) // block_size
    q = nat.aligned_rows(q)
    k = nat.aligned_rows(k)
    qc = torch.empty((B, H, M, D), dtype=q.dtype, device=dev)
    kc = torch.empty((B, H, M, D), dtype=k.dtype, device=dev)
    qi = torch.empty((B, H, M), dtype=torch.int32, device=dev) if return_indices else None
    ki = torch.empty((B, H, M), dtype=torch.int32, device=dev) if return_indices else None
    with torch.cuda.device(dev):
        st = lib.cab_coarsen_maxl2(q.data_ptr(), k.data_ptr(), dt, B, H, N, D,
                                   nat.strides4(q), nat.strides4(k), block_size,
                                   qc.data_ptr(), kc.data_ptr(), nat.ptr(qi), nat.ptr(ki),
                                   nat.stream_ptr(dev))
    nat.check("cab_coarsen_maxl2", st)
    if return_indices:
        return qc, kc, qi, ki
    return qc, kc


def coarsen_qk_max_l2_pytorch(q: torch.Tensor, k: torch.Tensor, block_size: int = 64):
    """Name kept for the reference's callers (methods.py:303, :424;
    kernel_benchmark.py:85). The reference had a torch-composed variant to
    compare its Triton kernel against; this framework has one implementation,
    so this runs the same HIP kernel as :func:`coarsen_qk_max_l2`."""
    return coarsen_qk_max_l2(q, k, block_size)
