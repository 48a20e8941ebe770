"""Device-resident layered K/V store and the eviction core the CAB and H2O
caches share.

``LayeredKV`` keeps each layer's K and V rows in two preallocated buffers
``[B, H, capacity, D]`` (an active and a spare one). A decode step copies its
new rows after the active rows, so appending costs the new rows only, not a
copy of the whole cache per token. A prune gathers the kept rows of every
layer from the active buffers into the spares (``cab_kv_gather``: one launch
per 32 tensors of one geometry) and swaps the two. Capacity doubles only when
an append would overflow it, and a prune that leaves a layer with less than
half of its capacity in use (kept rows plus the caller's headroom) moves it
into buffers of that size and releases the large ones: after a long prefill
the cache holds about twice the kept rows plus headroom per layer, not the
prefill's length.

The tensors a layer hands out are views of its active buffer, valid until
the next append or prune of that layer: a prune writes into the former
active buffer, so a view kept across it changes. Callers that keep K or V
across updates copy them.

``EvictingCache`` is the decision layer: it counts update calls, asks its
``selector`` for the positions to keep when an eviction is due, prunes the
store and the importance tracker with them and keeps the statistics. The
CAB and H2O caches differ only in their selector and in the length at or
below which they never evict.
"""

from __future__ import annotations

from typing import Any, Callable, Dict, List, Optional, Tuple

import torch

from ..scoring import ImportanceTracker
from .prune import gather_into

_GRAIN = 16  # bytes: rows are padded to whole 16-byte chunks for the gather kernel


class _Layer:
    __slots__ = ("k", "v", "k_spare", "v_spare", "length", "width")

    def __init__(self, k, v, width):
        self.k, self.v = k, v
        self.k_spare = self.v_spare = None
        self.length = 0
        self.width = width  # the caller's D (buffers may be wider)


class LayeredKV:
    """Per-layer K/V rows in preallocated double buffers (see module doc)."""

    def __init__(self, initial_capacity: int = 256):
        self.initial_capacity = max(1, int(initial_capacity))
        self.layers: List[Optional[_Layer]] = []

    # -- geometry ---------------------------------------------------------
    @staticmethod
    def _padded(d: int, element_size: int) -> int:
        per = _GRAIN // element_size if _GRAIN % element_size == 0 else 1
        return -(-d // per) * per

    def _alloc(self, like: torch.Tensor, capacity: int, width: int) -> torch.Tensor:
        B, H = like.shape[0], like.shape[1]
        return torch.zeros((B, H, capacity, width), dtype=like.dtype, device=like.device)

    # -- rows -------------------------------------------------------------
    def length(self, layer: int) -> int:
        if layer >= len(self.layers) or self.layers[layer] is None:
            return 0
        return self.layers[layer].length

    def view(self, layer: int) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        if layer >= len(self.layers) or self.layers[layer] is None:
            return None, None
        L = self.layers[layer]
        return L.k[:, :, :L.length, :L.width], L.v[:, :, :L.length, :L.width]

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor):
        if k.dim() != 4 or v.shape != k.shape or v.dtype != k.dtype:
            raise ValueError("key/value states must be two [B, H, n, D] tensors of one dtype")
        while len(self.layers) <= layer:
            self.layers.append(None)
        n = k.shape[2]
        L = self.layers[layer]
        if L is None:
            width = self._padded(k.shape[3], k.element_size())
            cap = max(self.initial_capacity, n)
            L = _Layer(self._alloc(k, cap, width), self._alloc(k, cap, width), k.shape[3])
            self.layers[layer] = L
        elif (k.shape[0], k.shape[1], k.shape[3]) != (L.k.shape[0], L.k.shape[1], L.width) \
                or k.dtype != L.k.dtype or k.device != L.k.device:
            raise ValueError(f"layer {layer}: new states {tuple(k.shape)} {k.dtype} do not match "
                             f"the cached [B, H, *, D] = {tuple(L.k.shape[:2])} x {L.width} {L.k.dtype}")
        need = L.length + n
        if need > L.k.shape[2]:
            cap = max(need, 2 * L.k.shape[2])
            nk, nv = self._alloc(k, cap, L.k.shape[3]), self._alloc(k, cap, L.k.shape[3])
            nk[:, :, :L.length].copy_(L.k[:, :, :L.length])
            nv[:, :, :L.length].copy_(L.v[:, :, :L.length])
            L.k, L.v = nk, nv
            L.k_spare = L.v_spare = None  # reallocated at the next prune
        L.k[:, :, L.length:need, :L.width].copy_(k)
        L.v[:, :, L.length:need, :L.width].copy_(v)
        L.length = need

    def capacity(self, layer: int) -> int:
        """Rows the layer's active buffer holds (0 for an absent layer)."""
        if layer >= len(self.layers) or self.layers[layer] is None:
            return 0
        return self.layers[layer].k.shape[2]

    def prune(self, keep: torch.Tensor, headroom: int = 0):
        """Every present layer keeps its rows at ``keep`` (ascending int64
        positions), in that order. ``headroom``: rows the caller expects to
        append before the next prune. A layer whose capacity exceeds twice
        ``len(keep) + headroom`` (and the initial capacity) moves into new
        buffers of that many rows; its old buffers are released."""
        n_keep = keep.numel()
        target = max(self.initial_capacity, n_keep + max(0, int(headroom)))
        groups: Dict[tuple, List[_Layer]] = {}
        shrunk = set()
        for L in self.layers:
            if L is None:
                continue
            if L.k.shape[2] > 2 * target:
                B, H, _, W = L.k.shape
                L.k_spare = L.k.new_empty((B, H, target, W))
                L.v_spare = L.v.new_empty((B, H, target, W))
                shrunk.add(id(L))
            elif L.k_spare is None or L.k_spare.shape != L.k.shape:
                L.k_spare, L.v_spare = torch.empty_like(L.k), torch.empty_like(L.v)
            key = (tuple(L.k.shape), tuple(L.k_spare.shape), L.k.dtype, L.k.device, L.length)
            groups.setdefault(key, []).append(L)
        idx = None
        for (_, _, _, dev, length), members in groups.items():
            if idx is None or idx.device != dev:
                idx = keep.detach().reshape(-1).to(device=dev, dtype=torch.int64).contiguous()
            srcs = [L.k for L in members] + [L.v for L in members]
            dsts = [L.k_spare for L in members] + [L.v_spare for L in members]
            gather_into(srcs, dsts, idx, length, validate=False)  # own buffers: aligned
        for L in self.layers:
            if L is None:
                continue
            L.k, L.k_spare = L.k_spare, L.k
            L.v, L.v_spare = L.v_spare, L.v
            if id(L) in shrunk:
                L.k_spare = L.v_spare = None  # the large buffers are released
            L.length = n_keep

    def clear(self):
        self.layers = []


Selector = Callable[[int, int], torch.Tensor]


class EvictingCache:
    """Update / evict control shared by the CAB and H2O caches.

    Per ``update`` call (one layer's new rows): the rows are appended, layer
    0's attention weights (when given) feed the importance tracker, and an
    eviction is due once the layer holds more than ``int(1.1 *
    max_cache_size)`` rows or ``eviction_interval`` calls have passed since
    the last one, provided the layer holds more than ``floor`` rows. An
    eviction keeps ``int(max_cache_size * (1 - sparsity) * 0.9)`` positions
    chosen by the selector among the first ``cache_len`` (the shortest
    layer's length) and prunes every layer and the tracker to them.
    """

    def __init__(self, max_cache_size: int, sparsity: float, eviction_interval: int, device: str,
                 floor: float, selector: Selector):
        self.max_cache_size = max_cache_size
        self.sparsity = sparsity
        self.eviction_interval = eviction_interval
        self.device = device
        self._floor = floor
        self._selector = selector
        # Kept rows plus the rows the update calls between two evictions
        # append; larger appends (a prefill) grow a layer until its next prune.
        self._headroom = max(1, eviction_interval) + 1
        self._store = LayeredKV(initial_capacity=max(self.keep_size + self._headroom, 16))
        self.importance_tracker = ImportanceTracker(device=device)
        self.tokens_since_last_eviction = 0
        self.total_evictions = 0
        self.stats: Dict[str, Any] = {"total_tokens_processed": 0, "total_evictions": 0,
                                      "total_tokens_evicted": 0}

    # The per-layer tensors as read-only tuples of views (None for a layer
    # never updated): assigning an entry raises TypeError instead of being
    # silently lost, and the views follow the store's lifetime rule (valid
    # until the layer's next update or eviction).
    @property
    def key_cache(self) -> Tuple[Optional[torch.Tensor], ...]:
        return tuple(self._store.view(i)[0] for i in range(len(self._store.layers)))

    @property
    def value_cache(self) -> Tuple[Optional[torch.Tensor], ...]:
        return tuple(self._store.view(i)[1] for i in range(len(self._store.layers)))

    @property
    def keep_size(self) -> int:
        return int(self.max_cache_size * (1.0 - self.sparsity) * 0.9)

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               attention_weights: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """Appends one layer's new K/V ``[B, H, n, D]`` (attention weights
        ``[B, H, n, N]`` optional, read on layer 0) and returns the layer's
        cached K and V after any eviction."""
        self._store.append(layer_idx, key_states, value_states)
        if layer_idx == 0 and attention_weights is not None:
            self.importance_tracker.update(attention_weights)
        self.stats["total_tokens_processed"] += 1
        self.tokens_since_last_eviction += 1
        n = self._store.length(layer_idx)
        due = (n > int(self.max_cache_size * 1.1)
               or self.tokens_since_last_eviction >= self.eviction_interval)
        if due and n > self._floor:
            self._evict()
        return self._store.view(layer_idx)

    def _evict(self):
        lengths = [L.length for L in self._store.layers if L is not None]
        if not lengths or self._store.layers[0] is None:
            return
        cache_len = min(lengths)
        if cache_len <= self.keep_size:
            return
        keep = self._selector(cache_len, self.keep_size)
        self._store.prune(keep, headroom=self._headroom)
        self.importance_tracker.prune(keep)
        self.tokens_since_last_eviction = 0
        self.total_evictions += 1
        self._on_evicted(cache_len, keep.numel())

    def _on_evicted(self, cache_len: int, kept: int):
        self.stats["total_evictions"] += 1
        self.stats["total_tokens_evicted"] += cache_len - kept

    # HF-style queries.
    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._store.length(layer_idx)

    def get_max_length(self) -> int:
        return self.max_cache_size

    def reset(self):
        """Empties the cache and the tracker (the cumulative statistics stay)."""
        self._store.clear()
        self.importance_tracker.reset()
        self.tokens_since_last_eviction = 0
        self.total_evictions = 0

    def get_stats(self) -> Dict[str, Any]:
        out = dict(self.stats)
        out["current_cache_size"] = self.get_seq_length(0)
        out["max_cache_size"] = self.max_cache_size
        return out

    def __len__(self) -> int:
        return self.get_seq_length(0)

    def __repr__(self) -> str:
        return (f"{type(self).__name__}[{self.get_seq_length(0)} of {self.max_cache_size} rows, "
                f"keep {1.0 - self.sparsity:.1%} per eviction, {self.total_evictions} evictions]")
