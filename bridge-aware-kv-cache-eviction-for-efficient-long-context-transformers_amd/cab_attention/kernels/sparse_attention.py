"""Block-sparse attention executor (HIP kernel ``cab_block_sparse_attn_fwd``).

Replaces the executor inside the reference's ``CABAttention`` (absent from
the reference tree): FlexAttention over the predictor's BlockMask, or the
manual masked softmax of CAB_Attention_Colab.ipynb:376-382 and
experiments/longbench_qa/methods.py:103-119 (README.md:44-46). The kernel
walks only the kept key blocks of each query block.
"""

from __future__ import annotations

import math

import torch

from .. import _native as nat

# What the executor kernel is built for; anything else is rejected by the
# C ABI (CAB_ESHAPE) rather than computed approximately.
SUPPORTED_HEAD_DIMS = (64, 128)
# 64, its multiples 128 and 256 (lists expanded to 64-token tiles), and 8,
# 16, 32 (64-token tiles with sub-tile masks); the packed-V path takes 64.
SUPPORTED_BLOCK_SIZES = (8, 16, 32, 64, 128, 256)


def _check_lists(kv_idx, kv_cnt, B, H, M):
    if kv_idx.dim() != 4 or tuple(kv_idx.shape[:3]) != (B, H, M):
        raise ValueError(f"kv_idx must be [B, H, M={M}, kmax]; got {tuple(kv_idx.shape)}")
    if tuple(kv_cnt.shape) != (B, H, M):
        raise ValueError(f"kv_cnt must be [B, H, M={M}]; got {tuple(kv_cnt.shape)}")
    if kv_idx.dtype != torch.int32 or kv_cnt.dtype != torch.int32:
        raise TypeError("kv_idx and kv_cnt must be int32")
    return kv_idx.contiguous(), kv_cnt.contiguous()


def _outputs(q, out, return_lse, dev):
    B, H, N, D = q.shape
    if out is None:
        out = torch.empty((B, H, N, D), dtype=q.dtype, device=dev)
    elif tuple(out.shape) != (B, H, N, D) or out.dtype != q.dtype:
        raise ValueError("out must match q's shape and dtype")
    lse = torch.empty((B, H, N), dtype=torch.float32, device=dev) if return_lse else None
    return out, lse


def block_sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           kv_idx: torch.Tensor, kv_cnt: torch.Tensor, block_size: int = 64,
                           causal: bool = False, scale: float | None = None,
                           out: torch.Tensor | None = None, return_lse: bool = False):
    """``out[t] = softmax_s(q_t . k_s * scale) v_s`` over the key blocks
    ``kv_idx[b, h, i, :kv_cnt[b, h, i]]`` of the query block i holding t.

    q, k, v: ``[B, H, N, D]`` bf16, fp16 or fp32 (D = 64 or 128, block_size in
    ``SUPPORTED_BLOCK_SIZES``;
    fp32 runs on split bf16 hi + lo operands, three MFMA products each); causal
    drops keys s > t; a query with no key gets 0; ``scale`` (> 0) defaults to
    ``1/sqrt(D)``. Index entries outside ``[0, M)`` are skipped. ``out`` may be
    a preallocated ``[B, H, N, D]`` view (any strides with a contiguous last
    dim), e.g. a transposed view of a ``[B, N, H, D]`` buffer. With
    ``return_lse`` the fp32 natural-log log-sum-exp ``[B, H, N]`` is returned
    too.
    """
    if q.dim() != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q, k, v must share one [B, H, N, D] shape; got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v dtypes differ")
    dev = nat.require_device(q, k, v, kv_idx, kv_cnt)
    lib = nat.load()
    dt = nat.dtype_code(q)
    B, H, N, D = q.shape
    M = (N + block_size - 1) // block_size
    kv_idx, kv_cnt = _check_lists(kv_idx, kv_cnt, B, H, M)
    q = nat.aligned_rows(q)
    k = nat.aligned_rows(k)
    v = nat.aligned_rows(v)
    out, lse = _outputs(q, out, return_lse, dev)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    wbytes = lib.cab_block_sparse_attn_workspace_bytes_k(dt, B, H, N, D, int(block_size),
                                                         int(kv_idx.shape[-1]))
    ws = torch.empty(max(int(wbytes), 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = lib.cab_block_sparse_attn_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, B, H, N, D, nat.strides4(q),
            nat.strides4(k), nat.strides4(v), nat.strides4(out), int(block_size),
            kv_idx.data_ptr(), kv_cnt.data_ptr(), int(kv_idx.shape[-1]), float(scale),
            int(bool(causal)), out.data_ptr(), nat.ptr(lse), ws.data_ptr(), ws.numel(),
            nat.stream_ptr(dev))
    nat.check("cab_block_sparse_attn_fwd", st)
    return (out, lse) if return_lse else out


def pack_v(v: torch.Tensor, block_size: int = 64) -> torch.Tensor:
    """V ``[B, H, N, D]`` -> its packed V^T tiles (uint8, 16 KB per (b, h, key
    block)) for :func:`block_sparse_attention_packed`; reusable while V is
    unchanged. bf16 / fp16 only."""
    if v.dim() != 4:
        raise ValueError(f"v must be [B, H, N, D]; got {tuple(v.shape)}")
    dev = nat.require_device(v)
    lib = nat.load()
    dt = nat.dtype_code(v)
    B, H, N, D = v.shape
    v = nat.aligned_rows(v)
    wbytes = lib.cab_block_sparse_attn_workspace_bytes(dt, B, H, N, D, int(block_size))
    vt = torch.empty(max(int(wbytes), 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = lib.cab_block_sparse_attn_pack_v(v.data_ptr(), dt, B, H, N, D, nat.strides4(v),
                                              int(block_size), vt.data_ptr(), vt.numel(),
                                              nat.stream_ptr(dev))
    nat.check("cab_block_sparse_attn_pack_v", st)
    return vt


def block_sparse_attention_packed(q: torch.Tensor, k: torch.Tensor, vt: torch.Tensor,
                                  kv_idx: torch.Tensor, kv_cnt: torch.Tensor,
                                  block_size: int = 64, causal: bool = False,
                                  scale: float | None = None, out: torch.Tensor | None = None,
                                  return_lse: bool = False):
    """:func:`block_sparse_attention` with V given as :func:`pack_v`'s tiles."""
    if q.dim() != 4 or q.shape != k.shape:
        raise ValueError(f"q, k must share one [B, H, N, D] shape; got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}")
    if q.dtype != k.dtype:
        raise TypeError("q, k dtypes differ")
    if vt.dtype != torch.uint8 or not vt.is_contiguous():
        raise TypeError("vt must be the contiguous uint8 tensor pack_v returned")
    dev = nat.require_device(q, k, vt, kv_idx, kv_cnt)
    lib = nat.load()
    dt = nat.dtype_code(q)
    B, H, N, D = q.shape
    M = (N + block_size - 1) // block_size
    kv_idx, kv_cnt = _check_lists(kv_idx, kv_cnt, B, H, M)
    q = nat.aligned_rows(q)
    k = nat.aligned_rows(k)
    out, lse = _outputs(q, out, return_lse, dev)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    with torch.cuda.device(dev):
        st = lib.cab_block_sparse_attn_fwd_packed(
            q.data_ptr(), k.data_ptr(), vt.data_ptr(), dt, B, H, N, D, nat.strides4(q),
            nat.strides4(k), nat.strides4(out), int(block_size), kv_idx.data_ptr(),
            kv_cnt.data_ptr(), int(kv_idx.shape[-1]), float(scale), int(bool(causal)),
            out.data_ptr(), nat.ptr(lse), vt.numel(), nat.stream_ptr(dev))
    nat.check("cab_block_sparse_attn_fwd_packed", st)
    return (out, lse) if return_lse else out


def kept_tile_flops(kv_idx: torch.Tensor, kv_cnt: torch.Tensor, block_size: int, head_dim: int,
                    seq_len: int, causal: bool) -> int:
    """Useful flops of one executor call: ``4 * bs * bs * D`` per kept tile
    (QK^T and PV), ``2 * bs * (bs + 1) * D`` for a causal diagonal tile,
    with ragged edge blocks counted at their valid sizes."""
    idx = kv_idx.long()
    cnt = kv_cnt.long()
    kmax = idx.shape[-1]
    valid = (torch.arange(kmax, device=idx.device) < cnt[..., None]) & (idx >= 0)
    M = (seq_len + block_size - 1) // block_size
    sizes = torch.full((M,), block_size, dtype=torch.long, device=idx.device)
    sizes[-1] = seq_len - (M - 1) * block_size
    qsize = sizes.view(1, 1, M, 1)
    ksize = sizes[idx.clamp(0, M - 1)]
    pairs = qsize * ksize
    if causal:
        rows = torch.arange(M, device=idx.device).view(1, 1, M, 1)
        diag = idx == rows
        pairs = torch.where(diag, qsize * (qsize + 1) // 2, pairs)
    return int((pairs * valid).sum().item()) * 4 * head_dim
