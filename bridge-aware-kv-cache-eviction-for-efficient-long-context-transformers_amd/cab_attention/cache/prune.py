"""Row gathers over cache tensors through ``cab_kv_gather``: every layer's K
and V pruned to the kept positions in one launch per 32 tensors, in place of
the per-layer ``cache[:, :, keep_indices, :]`` of the reference caches
(cab_cache.py:207-210, h2o_cache.py:146-149)."""

from __future__ import annotations

import ctypes
from typing import List, Sequence

import torch

from .. import _native as nat

def _rows_aligned(t: torch.Tensor) -> bool:
    es = t.element_size()
    return (t.stride(3) == 1 and t.data_ptr() % 16 == 0 and (t.shape[3] * es) % 16 == 0
            and all((s * es) % 16 == 0 for s in t.stride()[:3]))


def gather_into(srcs: Sequence[torch.Tensor], dsts: Sequence[torch.Tensor],
                keep_indices: torch.Tensor, n_src: int, validate: bool = True) -> None:
    """``dst[:, :, t, :] = src[:, :, keep[t], :]`` for pairs of ``[B, H, *, D]``
    views that share B, H, D, dtype and one stride set per side (rows 16-byte
    aligned). ``keep`` is int64 on the tensors' device; positions outside
    ``[0, n_src)`` give zero rows. ``validate=False`` skips the per-tensor
    checks for callers whose buffers hold these properties by construction."""
    srcs, dsts = list(srcs), list(dsts)
    if not srcs:
        return
    ref = srcs[0]
    B, H, _, D = ref.shape
    n_keep = keep_indices.numel()
    if n_keep == 0 or B == 0 or H == 0:
        return
    es = ref.element_size()
    sstr, dstr = ref.stride(), dsts[0].stride()
    if validate:
        for s, d in zip(srcs, dsts):
            if (s.stride() != sstr or d.stride() != dstr or s.dtype != ref.dtype
                    or d.dtype != ref.dtype or s.shape[:2] != ref.shape[:2] or s.shape[3] != D
                    or d.shape[3] != D or d.shape[2] < n_keep
                    or not _rows_aligned(s) or not _rows_aligned(d)):
                raise ValueError("gather_into: tensors must share shape, dtype, strides and "
                                 "16-byte rows")
    dev = ref.device
    ss = (ctypes.c_int64 * 4)(sstr[0] * es, sstr[1] * es, sstr[2] * es, 0)
    ds = (ctypes.c_int64 * 4)(dstr[0] * es, dstr[1] * es, dstr[2] * es, 0)
    lib = nat.load()
    src_arr = (ctypes.c_void_p * len(srcs))(*[s.data_ptr() for s in srcs])
    dst_arr = (ctypes.c_void_p * len(dsts))(*[d.data_ptr() for d in dsts])
    with torch.cuda.device(dev):  # the library launches one kernel per 32 tensors
        st = lib.cab_kv_gather(src_arr, dst_arr, len(srcs), B, H, n_src, D * es, ss, ds,
                               keep_indices.data_ptr(), n_keep, nat.stream_ptr(dev))
    nat.check("cab_kv_gather", st)


def gather_positions(tensors: Sequence[torch.Tensor], keep_indices: torch.Tensor) -> List[torch.Tensor]:
    """``[t[:, :, keep_indices, :] for t in tensors]`` for ``[B, H, N, D]``
    tensors of one shape and dtype, into new contiguous tensors. Positions
    outside ``[0, N)`` give zero rows."""
    tensors = list(tensors)
    if not tensors:
        return []
    ref = tensors[0]
    if ref.dim() != 4:
        raise ValueError("cache tensors must be [B, H, N, D]")
    for t in tensors:
        if t.shape != ref.shape or t.dtype != ref.dtype:
            raise ValueError("all cache tensors must share one shape and dtype")
    dev = nat.require_device(*tensors, keep_indices)
    B, H, N, D = ref.shape
    if (D * ref.element_size()) % 16 != 0:
        raise ValueError("cab_kv_gather moves whole 16-byte row chunks: D * element size "
                         f"must be a multiple of 16 (got {D} x {ref.element_size()})")
    idx = keep_indices.detach().reshape(-1).to(torch.int64).contiguous()
    srcs = [t if _rows_aligned(t) else t.contiguous() for t in tensors]
    if any(s.stride() != srcs[0].stride() for s in srcs):
        srcs = [s.contiguous() for s in srcs]
    outs = [torch.empty((B, H, idx.numel(), D), dtype=ref.dtype, device=dev) for _ in tensors]
    gather_into(srcs, outs, idx, N, validate=False)  # normalised above; outputs are fresh
    return outs


def prune_layers(key_cache: list, value_cache: list, keep_indices: torch.Tensor):
    """Replaces the non-None entries of both per-layer lists by their rows at
    ``keep_indices`` (new tensors; layers of one shape share launches)."""
    groups = {}
    for i, k in enumerate(key_cache):
        if k is not None:
            groups.setdefault((tuple(k.shape), k.dtype), []).append(i)
    for ids in groups.values():
        outs = gather_positions([key_cache[i] for i in ids] + [value_cache[i] for i in ids],
                                keep_indices)
        for n, i in enumerate(ids):
            key_cache[i] = outs[n]
            value_cache[i] = outs[len(ids) + n]
