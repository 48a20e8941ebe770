"""Coarse FRC scores and block masks (HIP kernels ``cab_block_frc``,
``cab_block_topk``).

Same names and call contract as the reference's
``cab_attention/kernels/frc_kernel.py`` (absent from the reference tree; its
callers are experiments/longbench_qa/methods.py:330-345, :449-473,
benchmarks/kernel_benchmark.py:24, :149, :197-205, :252-254,
benchmarks/quick_kernel_test.py:61-84, examples/demo_cab_attention.py:22 and
README.md:106-111).
"""

from __future__ import annotations

import math

import torch

from .. import _native as nat


def keep_count(num_blocks: int, sparsity: float) -> int:
    """Blocks kept per row: ``max(1, int(M * (1 - sparsity)))``, at most M
    (the notebook's k_keep, CAB_Attention_Colab.ipynb:372, applied per row)."""
    if not 0.0 <= float(sparsity) <= 1.0:
        raise ValueError(f"sparsity must be in [0, 1], got {sparsity}")
    return min(num_blocks, max(1, int(num_blocks * (1.0 - float(sparsity)))))


def compute_block_frc(q_coarse: torch.Tensor, k_coarse: torch.Tensor, temperature: float = 1.0,
                      lambda_redundancy: float = 0.5, formula: str = "additive",
                      normalization: str = "minmax", diagnostics: bool = True):
    """Block-level Forman-Ricci curvature of the coarse attention graph.

    ``A = Qc Kc^T / sqrt(D) / temperature`` (fp32 accumulate on MFMA),
    ``Ahat = minmax(A)`` per (b, h) (``none`` keeps A),
    ``T = Ahat @ Ahat`` (the 2-hop redundancy, README.md:36) and
    ``F = Ahat - lambda T`` (``additive``, README.md:37) or
    ``Ahat / (1 + lambda T / (Ahat + 1e-8))`` (``multiplicative``,
    CAB_Attention_Colab.ipynb:249 cell 11); non-finite F becomes 0.
    ``augmented`` is test.ipynb's graph curvature ``4 Ahat - S_i - S_j + 3 T``
    on edges (Ahat > 0) and 1000 elsewhere.

    Returns ``(frc, affinity, redundancy)``, fp32 ``[B, H, M, M]``; affinity is
    the normalised Ahat. With ``diagnostics=False`` only frc is computed and
    the other two are ``None`` (saves two M^2 writes per head).
    """
    if q_coarse.dim() != 4 or k_coarse.dim() != 4 or q_coarse.shape != k_coarse.shape:
        raise ValueError("q_coarse and k_coarse must both be [B, H, M, D] of the same shape; got "
                         f"{tuple(q_coarse.shape)} and {tuple(k_coarse.shape)}")
    if q_coarse.dtype != k_coarse.dtype:
        raise TypeError(f"dtype mismatch: {q_coarse.dtype} vs {k_coarse.dtype}")
    if normalization not in nat.NORMALIZATIONS:
        raise ValueError(f"normalization must be one of {sorted(nat.NORMALIZATIONS)}, "
                         f"got {normalization!r}")
    if formula not in nat.FORMULAS:
        raise ValueError(f"formula must be one of {sorted(nat.FORMULAS)}, got {formula!r}")
    dev = nat.require_device(q_coarse, k_coarse)
    lib = nat.load()
    dt = nat.dtype_code(q_coarse)
    B, H, M, D = q_coarse.shape
    qc = q_coarse.contiguous()
    kc = k_coarse.contiguous()
    shape = (B, H, M, M)
    frc = torch.empty(shape, dtype=torch.float32, device=dev)
    aff = torch.empty(shape, dtype=torch.float32, device=dev) if diagnostics else None
    tri = torch.empty(shape, dtype=torch.float32, device=dev) if diagnostics else None
    norm = nat.NORMALIZATIONS[normalization]
    form = nat.FORMULAS[formula]
    wbytes = lib.cab_block_frc_workspace_bytes(B, H, M, D, norm, form)
    ws = torch.empty(max(int(wbytes), 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = lib.cab_block_frc(qc.data_ptr(), kc.data_ptr(), dt, B, H, M, D,
                               1.0 / math.sqrt(D), float(temperature), float(lambda_redundancy),
                               norm, form, frc.data_ptr(), nat.ptr(aff), nat.ptr(tri),
                               ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    nat.check("cab_block_frc", st)
    return frc, aff, tri


def magnitude_quota(k: int, magnitude_ratio: float) -> int:
    """Blocks per row reserved for the magnitude ranking of the hybrid mask:
    ``int(k * magnitude_ratio)`` in ``[0, k]`` ("reserve X% of budget for
    top-magnitude blocks", methods.py:404-418)."""
    if not 0.0 <= float(magnitude_ratio) <= 1.0:
        raise ValueError(f"magnitude_ratio must be in [0, 1], got {magnitude_ratio}")
    return min(k, max(0, int(k * float(magnitude_ratio))))


def _select(frc: torch.Tensor, sparsity: float, select_high: bool, keep_diagonal: bool,
            causal: bool, dense: bool, magnitude_scores: torch.Tensor | None = None,
            magnitude_ratio: float = 0.5):
    if frc.dim() != 4 or frc.shape[-1] != frc.shape[-2]:
        raise ValueError(f"frc must be [B, H, M, M]; got {tuple(frc.shape)}")
    if magnitude_scores is not None and tuple(magnitude_scores.shape) != tuple(frc.shape):
        raise ValueError(f"magnitude_scores must match frc's shape {tuple(frc.shape)}; got "
                         f"{tuple(magnitude_scores.shape)}")
    tensors = (frc,) if magnitude_scores is None else (frc, magnitude_scores)
    dev = nat.require_device(*tensors)
    lib = nat.load()
    B, H, M, _ = frc.shape
    k = keep_count(M, sparsity) if M > 0 else 1
    f = frc.to(torch.float32).contiguous()
    kv_idx = torch.empty((B, H, M, k), dtype=torch.int32, device=dev)
    kv_cnt = torch.empty((B, H, M), dtype=torch.int32, device=dev)
    mask = torch.empty((B, H, M, M), dtype=torch.bool, device=dev) if dense else None
    flags = (int(bool(select_high)), int(bool(keep_diagonal)), int(bool(causal)))
    with torch.cuda.device(dev):
        if magnitude_scores is None:
            name = "cab_block_topk"
            st = lib.cab_block_topk(f.data_ptr(), B, H, M, k, *flags, kv_idx.data_ptr(),
                                    kv_cnt.data_ptr(), nat.ptr(mask), nat.stream_ptr(dev))
        else:
            name = "cab_block_topk_hybrid"
            mg = magnitude_scores.to(torch.float32).contiguous()
            st = lib.cab_block_topk_hybrid(f.data_ptr(), mg.data_ptr(), B, H, M, k,
                                           magnitude_quota(k, magnitude_ratio), *flags,
                                           kv_idx.data_ptr(), kv_cnt.data_ptr(), nat.ptr(mask),
                                           nat.stream_ptr(dev))
    nat.check(name, st)
    return kv_idx, kv_cnt, mask


def generate_block_mask(frc_scores: torch.Tensor, sparsity: float = 0.95, select_high: bool = False,
                        keep_diagonal: bool = True, causal: bool = False,
                        magnitude_scores: torch.Tensor | None = None,
                        magnitude_ratio: float = 0.5) -> torch.Tensor:
    """Block mask ``[B, H, M, M]`` (True = keep).

    Row i keeps ``k = max(1, int(M (1 - sparsity)))`` blocks (``min(k, i+1)``
    when causal, candidates ``j <= i``), lowest FRC first (highest with
    ``select_high``, as methods.py:342 passes), ties to the lower block index.
    ``keep_diagonal`` forces block ``i`` in; it counts toward k.

    Hybrid (CAB V4, methods.py:465-473): with ``magnitude_scores``
    ``[B, H, M, M]`` the first ``int(k * magnitude_ratio)`` of a row's blocks
    after the diagonal (fewer if the row has fewer) are those with the
    highest magnitude; FRC order fills the rest.
    """
    _, _, mask = _select(frc_scores, sparsity, select_high, keep_diagonal, causal, dense=True,
                         magnitude_scores=magnitude_scores, magnitude_ratio=magnitude_ratio)
    return mask


def generate_block_index(frc_scores: torch.Tensor, sparsity: float = 0.95,
                         select_high: bool = False, keep_diagonal: bool = True,
                         causal: bool = False, dense: bool = False,
                         magnitude_scores: torch.Tensor | None = None,
                         magnitude_ratio: float = 0.5):
    """Compact form of :func:`generate_block_mask` for the sparse executor.

    Returns ``(kv_idx int32 [B, H, M, k] ascending with -1 padding,
    kv_cnt int32 [B, H, M], mask or None)``.
    """
    return _select(frc_scores, sparsity, select_high, keep_diagonal, causal, dense,
                   magnitude_scores, magnitude_ratio)


def visualize_frc_statistics(frc_scores: torch.Tensor, affinity: torch.Tensor,
                             triangles: torch.Tensor, save_path: str | None = None):
    """Summary statistics of the curvature diagnostics (README.md:106-111).

    Returns a dict of host floats; when matplotlib is importable it also
    draws histograms of F, Ahat and T (saved to ``save_path`` if given).
    """
    f = frc_scores.detach().float().cpu()
    a = affinity.detach().float().cpu()
    t = triangles.detach().float().cpu()
    stats = {
        "frc_mean": float(f.mean()), "frc_std": float(f.std()),
        "frc_min": float(f.min()), "frc_max": float(f.max()),
        "frc_negative_fraction": float((f < 0).float().mean()),
        "affinity_mean": float(a.mean()), "triangles_mean": float(t.mean()),
    }
    try:
        import matplotlib
        matplotlib.use("Agg")
        import matplotlib.pyplot as plt
    except ImportError:
        return stats
    fig, axes = plt.subplots(1, 3, figsize=(15, 4))
    for ax, x, name in zip(axes, (f, a, t), ("FRC", "Affinity", "Triangles")):
        ax.hist(x.flatten().numpy(), bins=100)
        ax.set_title(name)
    fig.tight_layout()
    if save_path:
        fig.savefig(save_path, dpi=120)
    plt.close(fig)
    return stats
