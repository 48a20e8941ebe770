"""HIP kernel entry points (ctypes over libcab_hip.so)."""

from .coarsening import coarsen_qk_max_l2, coarsen_qk_max_l2_pytorch
from .frc_kernel import (compute_block_frc, generate_block_index, generate_block_mask,
                         keep_count, magnitude_quota, visualize_frc_statistics)
from .sparse_attention import (block_sparse_attention, block_sparse_attention_packed,
                               kept_tile_flops, pack_v)
from .flash_attention_accumulate import (FlashAttentionWithAccumulation, flash_attention,
                                         flash_attention_with_cumulative_scores,
                                         get_all_cumulative_scores, key_scores, repeat_kv)
from .token_frc import (compute_frc, compute_frc_pytorch, compute_frc_triton,
                        compute_node_strengths_triton, compute_triangles_triton, frc_from_keys,
                        symmetrize_attention, token_frc)

__all__ = [
    "coarsen_qk_max_l2", "coarsen_qk_max_l2_pytorch", "compute_block_frc", "generate_block_mask",
    "generate_block_index", "keep_count", "magnitude_quota", "visualize_frc_statistics", "block_sparse_attention",
    "block_sparse_attention_packed", "pack_v", "kept_tile_flops", "flash_attention",
    "key_scores", "flash_attention_with_cumulative_scores", "FlashAttentionWithAccumulation",
    "get_all_cumulative_scores", "repeat_kv", "compute_frc", "compute_frc_triton",
    "compute_frc_pytorch", "compute_node_strengths_triton", "compute_triangles_triton",
    "token_frc", "frc_from_keys", "symmetrize_attention",
]
