"""One-launch pruning of every layer's K and V to the kept positions
(``cab_kv_gather``), replacing the reference caches' per-layer
``cache[:, :, keep_indices, :]`` (cab_cache.py:207-210, h2o_cache.py:146-149)."""

from __future__ import annotations

import ctypes
from typing import List, Sequence

import torch

from .. import _native as nat


def gather_positions(tensors: Sequence[torch.Tensor], keep_indices: torch.Tensor) -> List[torch.Tensor]:
    """``[t[:, :, keep_indices, :] for t in tensors]`` for ``[B, H, N, D]``
    tensors of one shape and dtype, written by one kernel per 32 tensors.
    Positions outside [0, N) give zero rows."""
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
    idx = keep_indices.detach().reshape(-1).to(torch.int64).contiguous()
    n_keep = idx.numel()
    row_bytes = D * ref.element_size()
    srcs = []
    for t in tensors:
        ok = (t.stride(3) == 1 and t.data_ptr() % 16 == 0 and row_bytes % 16 == 0
              and all((s * t.element_size()) % 16 == 0 for s in t.stride()[:3]))
        srcs.append(t if ok else t.contiguous())
    outs = [torch.empty((B, H, n_keep, D), dtype=ref.dtype, device=dev) for _ in tensors]
    if n_keep == 0 or B == 0 or H == 0:
        return outs
    es = ref.element_size()
    sstr = srcs[0].stride()
    if any(s.stride() != sstr for s in srcs):
        srcs = [s.contiguous() for s in srcs]
        sstr = srcs[0].stride()
    src_arr = (ctypes.c_void_p * len(srcs))(*[s.data_ptr() for s in srcs])
    dst_arr = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    ss = (ctypes.c_int64 * 4)(sstr[0] * es, sstr[1] * es, sstr[2] * es, 0)
    ds_ = outs[0].stride()
    ds = (ctypes.c_int64 * 4)(ds_[0] * es, ds_[1] * es, ds_[2] * es, 0)
    lib = nat.load()
    with torch.cuda.device(dev):
        st = lib.cab_kv_gather(src_arr, dst_arr, len(srcs), B, H, N, row_bytes, ss, ds,
                               idx.data_ptr(), n_keep, nat.stream_ptr(dev))
    nat.check("cab_kv_gather", st)
    return outs


def prune_layers(key_cache: list, value_cache: list, keep_indices: torch.Tensor):
    """Prunes the non-None layers of both lists in place (new tensors)."""
    layers = [i for i, k in enumerate(key_cache) if k is not None]
    if not layers:
        return
    groups = {}
    for i in layers:
        k, v = key_cache[i], value_cache[i]
        groups.setdefault((tuple(k.shape), k.dtype), []).append(i)
    for (_, _), ids in groups.items():
        outs = gather_positions([key_cache[i] for i in ids] + [value_cache[i] for i in ids],
                                keep_indices)
        for n, i in enumerate(ids):
            key_cache[i] = outs[n]
            value_cache[i] = outs[len(ids) + n]
