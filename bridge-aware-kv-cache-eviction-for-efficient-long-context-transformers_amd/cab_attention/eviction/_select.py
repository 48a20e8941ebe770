"""Device selection of the positions a KV cache keeps (``cab_evict_select``)
and the bridge scores of the attention-matrix mode
(``cab_evict_connectivity``)."""

from __future__ import annotations

import torch

from .. import _native as nat

BRIDGE_NONE, BRIDGE_MEDIAN, BRIDGE_SCORES, BRIDGE_POSITIONAL = 0, 1, 2, 3
MULTI_MIN = 1 << 15  # cache_len from which cab_evict_select needs its workspace


def planned_counts(cache_len: int, local: int, imp: int, bridge: int, has_scores: bool,
                   fallback: bool, mode: int):
    """(local, importance, bridge) counts the kernel will report: known on the
    host from the budgets alone, so callers need no device round trip."""
    free0 = cache_len - local
    if has_scores:
        n_imp = min(imp, free0)
    elif fallback and imp > 0:
        n_imp = free0 - max(0, cache_len - local - imp)
    else:
        n_imp = 0
    free1 = free0 - n_imp
    if mode == BRIDGE_SCORES and n_imp == 0:
        mode = BRIDGE_MEDIAN if has_scores else BRIDGE_POSITIONAL
    if mode == BRIDGE_MEDIAN and not has_scores:
        mode = BRIDGE_POSITIONAL
    n_br = min(bridge, free1) if (bridge > 0 and free1 > 0 and mode != BRIDGE_NONE) else 0
    if mode == BRIDGE_POSITIONAL:
        n_br = min(n_br, free1 - free1 // 3)  # remaining[free1 // 3:][:budget]
    return local, n_imp, n_br


def select_positions(cache_len: int, scores: torch.Tensor | None, local: int, imp: int,
                     bridge: int, fallback: bool, mode: int, device,
                     bridge_scores: torch.Tensor | None = None, category: bool = False):
    """Runs ``cab_evict_select``; returns (ascending kept positions [int64],
    (local, importance, bridge) counts, category [uint8] or None)."""
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("CAB-Attention kernels run on the GPU only (HIP, gfx950); "
                           f"got device {dev}")
    lib = nat.load()
    if scores is not None:
        nat.require_device(scores)
        scores = scores.detach().reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
    if bridge_scores is not None:
        bridge_scores = bridge_scores.detach().reshape(-1).to(device=dev,
                                                               dtype=torch.float32).contiguous()
    keep = torch.empty(max(cache_len, 1), dtype=torch.int64, device=dev)
    counts = torch.empty(4, dtype=torch.int32, device=dev)
    cat = torch.empty(max(cache_len, 1), dtype=torch.uint8, device=dev) if category else None
    # Large caches run one workgroup per segment with a workspace.
    wbytes = int(lib.cab_evict_select_workspace_bytes(cache_len)) if cache_len >= MULTI_MIN else 0
    ws = torch.empty(wbytes, dtype=torch.uint8, device=dev) if wbytes else None
    with torch.cuda.device(dev):
        st = lib.cab_evict_select(nat.ptr(scores), 0 if scores is None else scores.numel(),
                                  nat.ptr(bridge_scores), cache_len, local, imp, bridge,
                                  int(bool(fallback)), mode, keep.data_ptr(), counts.data_ptr(),
                                  nat.ptr(cat), nat.ptr(ws), wbytes, nat.stream_ptr(dev))
    nat.check("cab_evict_select", st)
    n_loc, n_imp, n_br = planned_counts(cache_len, local, imp, bridge, scores is not None,
                                        fallback, mode)
    keep = keep[:n_loc + n_imp + n_br]
    return keep, (n_loc, n_imp, n_br), (cat[:cache_len] if cat is not None else None), counts


def connectivity(attention: torch.Tensor, category: torch.Tensor) -> torch.Tensor:
    """``(A[imp, :].sum(0)) * (A[:, imp].sum(1))`` with imp = category == 2
    (``cab_evict_connectivity``); A is [cache_len, cache_len]."""
    n = category.numel()
    if attention.dim() != 2 or tuple(attention.shape) != (n, n):
        raise ValueError(f"attention_matrix must be [{n}, {n}]; got {tuple(attention.shape)}")
    dev = nat.require_device(attention, category)
    a = attention.detach().to(torch.float32)
    if a.stride(1) != 1:
        a = a.contiguous()
    out = torch.empty(max(n, 1), dtype=torch.float32, device=dev)
    lib = nat.load()
    with torch.cuda.device(dev):
        st = lib.cab_evict_connectivity(a.data_ptr(), n, a.stride(0), category.data_ptr(),
                                        out.data_ptr(), nat.stream_ptr(dev))
    nat.check("cab_evict_connectivity", st)
    return out[:n]
