"""CAB-Attention on MI355X (gfx950): curvature-aware block-sparse attention.

Public surface (same names as the reference package ``cab_attention``):
``CABAttention``, ``CoarseCurvaturePredictor`` and, in ``cab_attention.kernels``,
``coarsen_qk_max_l2``, ``compute_block_frc``, ``generate_block_mask``,
``block_sparse_attention``. Every stage is a hand-written HIP kernel in
``libcab_hip.so``; there is no CPU or Triton path.
"""

from .cab_attention import CABAttention
from .coarse_predictor import CoarseCurvaturePredictor

__version__ = "0.1.0"
__all__ = ["CABAttention", "CoarseCurvaturePredictor", "__version__"]
