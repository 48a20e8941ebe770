"""Host logic of the KV caches' shared core (cab_attention/cache/store.py), on
the CPU: the device gather (cab_kv_gather) is replaced by torch indexing and
the selector by a fixed rule, so the test checks the bookkeeping only -- the
append path, capacity growth, row padding, the double-buffer swap, the
eviction triggers and the statistics -- against a plain list model of the
reference caches' documented rules (cab_cache.py:122-226,
h2o_cache.py:65-160). The GPU tests run the same caches on the kernels."""

import pytest
import torch

from cab_attention.cache import store as S
from cab_attention.cache.cab_cache import CABCache
from cab_attention.cache.h2o_cache import H2OCache


def torch_gather_into(srcs, dsts, keep, n_src, validate=True):
    for s, d in zip(srcs, dsts):
        rows = torch.zeros((s.shape[0], s.shape[1], keep.numel(), s.shape[3]), dtype=s.dtype)
        ok = (keep >= 0) & (keep < n_src)
        rows[:, :, ok] = s[:, :, keep[ok]]
        d[:, :, :keep.numel()] = rows


def every_other_newest(cache_len, keep_size):
    """A fixed selector: the keep_size newest positions of even parity first."""
    cand = [p for p in range(cache_len - 1, -1, -1) if p % 2 == 0]
    cand += [p for p in range(cache_len - 1, -1, -1) if p % 2 == 1]
    return torch.tensor(sorted(cand[:keep_size]), dtype=torch.int64)


class Model:
    """The reference caches' rules on lists of token ids."""

    def __init__(self, max_size, sparsity, interval, floor):
        self.max, self.sp, self.iv, self.floor = max_size, sparsity, interval, floor
        self.layers, self.since, self.evictions, self.evicted, self.calls = [], 0, 0, 0, 0

    def update(self, layer, ids):
        while len(self.layers) <= layer:
            self.layers.append(None)
        self.layers[layer] = (self.layers[layer] or []) + ids
        self.calls += 1
        self.since += 1
        n = len(self.layers[layer])
        if (n > int(self.max * 1.1) or self.since >= self.iv) and n > self.floor:
            cache_len = min(len(x) for x in self.layers if x is not None)
            keep_size = int(self.max * (1 - self.sp) * 0.9)
            if cache_len > keep_size:
                keep = every_other_newest(cache_len, keep_size).tolist()
                self.layers = [None if x is None else [x[p] for p in keep] for x in self.layers]
                self.since = 0
                self.evictions += 1
                self.evicted += cache_len - len(keep)


@pytest.mark.parametrize("kind", ["cab", "h2o"])
@pytest.mark.parametrize("D,dtype", [(8, torch.float32), (3, torch.float32), (5, torch.bfloat16)])
def test_cache_core_matches_the_reference_rules(monkeypatch, kind, D, dtype):
    monkeypatch.setattr(S, "gather_into", torch_gather_into)
    if kind == "cab":
        cache = CABCache(max_cache_size=40, sparsity=0.5, eviction_interval=7, device="cpu")
        floor = 40 * 0.5
    else:
        cache = H2OCache(max_cache_size=40, sparsity=0.5, eviction_interval=7, device="cpu")
        floor = float("-inf")
    cache._selector = every_other_newest
    model = Model(40, 0.5, 7, floor)
    B, H, layers = 1, 2, 3
    tok = 0
    steps = [5] + [1] * 60 + [70] + [1] * 30  # a prefill, decode steps, a long chunk, decode
    for n in steps:
        for layer in range(layers):
            ids = list(range(tok, tok + n))
            tok += n
            x = torch.tensor(ids, dtype=torch.float32).view(1, 1, n, 1).expand(B, H, n, D)
            k, v = x.to(dtype), (x + 0.5).to(dtype)
            got_k, got_v = cache.update(k, v, layer, None)
            model.update(layer, ids)
            assert got_k.shape == (B, H, len(model.layers[layer]), D)
            for l2 in range(layers):
                want = model.layers[l2] if l2 < len(model.layers) else None
                have = cache.key_cache[l2] if l2 < len(cache.key_cache) else None
                if want is None:
                    assert have is None
                    continue
                ids_t = torch.tensor(want, dtype=torch.float32)
                assert torch.equal(have[0, 1, :, D - 1], ids_t.to(dtype))
                assert torch.equal(cache.value_cache[l2][0, 1, :, 0], (ids_t + 0.5).to(dtype))
    assert cache.total_evictions == model.evictions > 5
    st = cache.get_stats()
    assert st["total_evictions"] == model.evictions
    assert st["total_tokens_evicted"] == model.evicted
    assert st["total_tokens_processed"] == model.calls
    assert len(cache) == len(model.layers[0])
    if kind == "cab":
        assert 0 < st["avg_cache_size"] <= int(40 * 0.5 * 0.9)
        assert st["effective_sparsity"] == pytest.approx(1 - len(model.layers[0]) / 40)
    cache.reset()
    assert len(cache) == 0 and cache.key_cache == () and cache.get_seq_length(2) == 0


def test_store_grows_and_pads_rows(monkeypatch):
    """Appends beyond the capacity double it and keep the rows; rows are
    padded to whole 16-byte chunks internally and handed out unpadded."""
    monkeypatch.setattr(S, "gather_into", torch_gather_into)
    st = S.LayeredKV(initial_capacity=4)
    x = torch.arange(3 * 2 * 5 * 3, dtype=torch.float32).view(3, 2, 5, 3)
    st.append(0, x, -x)
    assert st.layers[0].k.shape == (3, 2, 5, 4)  # 12-byte rows padded to 16
    y = torch.ones(3, 2, 6, 3)
    st.append(0, y, y)
    assert st.layers[0].k.shape[2] == 11 and st.length(0) == 11
    k, v = st.view(0)
    assert torch.equal(k[:, :, :5], x) and torch.equal(v[:, :, :5], -x) and torch.equal(k[:, :, 5:], y)
    st.prune(torch.tensor([1, 4, 10]))
    k, v = st.view(0)
    assert torch.equal(k[:, :, 0], x[:, :, 1]) and torch.equal(k[:, :, 1], x[:, :, 4])
    assert torch.equal(k[:, :, 2], y[:, :, 0]) and st.length(0) == 3
    with pytest.raises(ValueError):
        st.append(0, torch.ones(3, 2, 1, 4), torch.ones(3, 2, 1, 4))


@pytest.mark.parametrize("kind", ["cab", "h2o"])
def test_capacity_stays_bounded_after_a_long_prefill(monkeypatch, kind):
    """A prefill far longer than the cache grows each layer to its length;
    the first eviction moves every layer into buffers of about the kept rows
    plus the eviction interval, and decode steps keep it there."""
    monkeypatch.setattr(S, "gather_into", torch_gather_into)
    cls = CABCache if kind == "cab" else H2OCache
    cache = cls(max_cache_size=256, sparsity=0.5, eviction_interval=8, device="cpu")
    cache._selector = every_other_newest
    bound = 2 * (cache.keep_size + 8 + 1)
    B, H, D, layers = 1, 2, 4, 3
    for layer in range(layers):
        x = torch.randn(B, H, 5000, D)
        cache.update(x, x, layer, None)
    for _ in range(40):
        for layer in range(layers):
            x = torch.randn(B, H, 1, D)
            cache.update(x, x, layer, None)
    assert cache.total_evictions >= 2
    for layer in range(layers):
        L = cache._store.layers[layer]
        assert cache._store.capacity(layer) <= bound
        assert L.k_spare is None or L.k_spare.shape[2] <= bound
        assert cache.get_seq_length(layer) <= cache._store.capacity(layer)


def test_cache_views_are_read_only_and_alias_the_store(monkeypatch):
    """key_cache / value_cache are tuples (item assignment raises), and a view
    kept across an eviction is overwritten by the next prune: the documented
    lifetime (copy to keep)."""
    monkeypatch.setattr(S, "gather_into", torch_gather_into)
    cache = H2OCache(max_cache_size=40, sparsity=0.5, eviction_interval=3, device="cpu")
    cache._selector = every_other_newest
    # 20 rows fit the initial capacity (18 kept + 4 headroom), so no append
    # reallocates and the view stays on one of the two store buffers
    x = torch.arange(20, dtype=torch.float32).view(1, 1, 20, 1).expand(1, 2, 20, 4).contiguous()
    cache.update(x, x, 0, None)
    assert cache._store.capacity(0) == 22
    with pytest.raises(TypeError):
        cache.key_cache[0] = x
    with pytest.raises(TypeError):
        cache.value_cache[0] = x
    kept = cache.key_cache[0]
    snapshot = kept.clone()
    for _ in range(6):
        y = torch.full((1, 2, 1, 4), -1.0)
        cache.update(y, y, 0, None)
    assert cache.total_evictions >= 2
    assert not torch.equal(kept, snapshot)  # the old view now shows a later prune's rows
