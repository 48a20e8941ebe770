"""GPU parity of the KV-cache eviction kernels through the C ABI:
cab_evict_select (bit-exact positions, counts and categories against the
oracle), cab_evict_connectivity, cab_kv_gather, and the policy / cache
layers built on them."""

import numpy as np
import pytest
import torch

from oracle import cab_oracle as O

pytestmark = pytest.mark.gpu


def run_select(cuda, scores, n, local, imp, br, fallback, mode, bridge_scores=None):
    from cab_attention.eviction._select import select_positions
    sc = None if scores is None else torch.from_numpy(np.asarray(scores, np.float32)).to(cuda)
    bs = None if bridge_scores is None else torch.from_numpy(np.asarray(bridge_scores, np.float32)).to(cuda)
    keep, counts, cat, dev_counts = select_positions(n, sc, local, imp, br, fallback, mode, cuda,
                                                     bridge_scores=bs, category=True)
    return keep.cpu().numpy(), counts, cat.cpu().numpy(), dev_counts.cpu().numpy()


def score_cases(rng, n):
    yield "normal", (rng.standard_normal(n) * 3).astype(np.float32)
    yield "ties", rng.integers(0, 7, n).astype(np.float32)
    s = rng.integers(-3, 4, n).astype(np.float32)
    idx = rng.choice(n, size=min(n, 12), replace=False)
    s[idx[:3]] = np.nan
    s[idx[3:6]] = np.inf
    s[idx[6:9]] = -np.inf
    s[idx[9:]] = -0.0
    yield "special", s


@pytest.mark.parametrize("n", [1, 7, 100, 1000, 65537])
@pytest.mark.parametrize("mode", [0, 1, 3])
def test_evict_select_bit_exact(cuda, n, mode):
    rng = np.random.default_rng(n * 10 + mode)
    budgets = [(n // 10, n // 4, n // 5), (0, n, 0), (n, 3, 3), (min(5, n), n // 3, n)]
    for name, s in score_cases(rng, n):
        for local, imp, br in budgets:
            for short in (False, True):
                sc = s[: max(1, n // 2)] if short else s
                keep, cnt, cat, dc = run_select(cuda, sc, n, local, imp, br, True, mode)
                wk, wc, wcat = O.evict_select(sc, n, local, imp, br, True, mode)
                tag = f"{name} n={n} budgets={(local, imp, br)} short={short}"
                assert tuple(cnt) == tuple(wc) and tuple(dc[:3]) == tuple(wc), tag
                assert dc[3] == wk.size, tag
                assert np.array_equal(keep, wk), tag
                assert np.array_equal(cat, wcat), tag


def test_evict_select_without_scores_and_given_bridge_scores(cuda):
    rng = np.random.default_rng(5)
    n = 3000
    for local, imp, br, fb, mode in [(100, 200, 50, True, 1), (100, 200, 50, True, 3),
                                     (10, 0, 40, True, 2), (100, 200, 0, False, 0)]:
        keep, cnt, cat, _ = run_select(cuda, None, n, local, imp, br, fb, mode,
                                       bridge_scores=rng.random(n).astype(np.float32))
        wk, wc, wcat = O.evict_select(None, n, local, imp, br, fb, mode)
        assert tuple(cnt) == tuple(wc) and np.array_equal(keep, wk) and np.array_equal(cat, wcat)
    s = rng.integers(0, 50, n).astype(np.float32)
    b = rng.integers(0, 9, n).astype(np.float32)  # many tied bridge scores
    keep, cnt, cat, _ = run_select(cuda, s, n, 100, 300, 200, True, 2, bridge_scores=b)
    wk, wc, wcat = O.evict_select(s, n, 100, 300, 200, True, 2, bridge_scores=b)
    assert tuple(cnt) == tuple(wc) and np.array_equal(keep, wk) and np.array_equal(cat, wcat)


def test_evict_select_largest_cache(cuda):
    rng = np.random.default_rng(7)
    n = 1 << 20
    s = rng.integers(0, 1000, n).astype(np.float32)
    keep, cnt, cat, _ = run_select(cuda, s, n, 4096, 40000, 20000, True, 1)
    wk, wc, wcat = O.evict_select(s, n, 4096, 40000, 20000, True, 1)
    assert tuple(cnt) == tuple(wc) and np.array_equal(keep, wk) and np.array_equal(cat, wcat)


def test_connectivity_and_matrix_mode_policy(cuda):
    """Attention-matrix bridges: connectivity vs the float64 oracle, and the
    policy's two-call flow against the oracle on well-separated scores."""
    from cab_attention.eviction import EvictionConfig, ThreeComponentEvictionPolicy
    from cab_attention.eviction._select import connectivity
    rng = np.random.default_rng(8)
    n = 600
    a = rng.random((n, n)).astype(np.float32)
    s = (rng.standard_normal(n) * 3).astype(np.float32)
    _, (loc, n_imp, _), cat = O.evict_select(s, n, 30, 60, 0, True, 0)
    got = connectivity(torch.from_numpy(a).to(cuda), torch.from_numpy(cat).to(cuda)).cpu().numpy()
    want = O.evict_connectivity(a, cat)
    np.testing.assert_allclose(got, want, rtol=1e-5)
    pol = ThreeComponentEvictionPolicy(EvictionConfig(0.25, 0.25, 0.5))
    keep, diag = pol.select_indices(n, 120, torch.from_numpy(s).to(cuda),
                                    attention_matrix=torch.from_numpy(a).to(cuda), device="cuda")
    wk, wc, _ = O.evict_select(s, n, 30, 60, 30, True, 2, bridge_scores=want.astype(np.float32))
    assert np.array_equal(keep.cpu().numpy(), wk)
    assert (diag["local_count"], diag["importance_count"], diag["bridge_count"]) == wc
    assert diag["keep_size"] == wk.size


def test_policy_and_h2o_wrappers(cuda):
    """The reference-named wrappers: budgets from keep_size and the ratios,
    sorted unique output, and the demo's planted heavy hitters kept."""
    from cab_attention.eviction import EvictionConfig, ThreeComponentEvictionPolicy, h2o_select_indices
    rng = np.random.default_rng(9)
    s = rng.random(1000).astype(np.float32)
    s[100], s[500] = 10.0, 15.0
    pol = ThreeComponentEvictionPolicy(EvictionConfig(0.3, 0.2, 0.5))
    keep, diag = pol.select_indices(1000, 100, torch.from_numpy(s).to(cuda), device="cuda")
    k = keep.cpu().numpy()
    assert 100 in k and 500 in k and set(range(970, 1000)) <= set(k)
    assert np.all(np.diff(k) > 0) and diag["keep_size"] == 100
    wk, _, _ = O.evict_select(s, 1000, 30, 50, 20, True, 1)
    assert np.array_equal(k, wk)
    keep, diag = h2o_select_indices(1000, 100, torch.from_numpy(s).to(cuda), local_ratio=0.2)
    wk, wc, _ = O.evict_select(s, 1000, 20, 80, 0, False, 0)
    assert np.array_equal(keep.cpu().numpy(), wk)
    assert diag["local_count"] == 20 and diag["important_count"] == 80 and diag["total_kept"] == 100
    keep, diag = h2o_select_indices(50, 10, None)
    assert keep.cpu().tolist() == [48, 49] and diag["important_count"] == 0


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_kv_gather_matches_indexing(cuda, dt):
    """One call over 70 tensors (three launches of up to 32), strided
    sources, repeated and out-of-range positions."""
    from cab_attention.cache import gather_positions
    g = torch.Generator().manual_seed(3)
    base = torch.randn(2, 70, 3, 300, 64, generator=g).to(dt).to(cuda)
    tensors = [base[:, i] for i in range(70)]  # [2, 3, 300, 64] views with a batch stride of 70 rows
    keep = torch.tensor([0, 5, 5, 299, 7, 150], dtype=torch.int64, device=cuda)
    outs = gather_positions(tensors, keep)
    for t, o in zip(tensors, outs):
        assert torch.equal(o, t[:, :, keep, :])
    bad = torch.tensor([1, 300, -1], dtype=torch.int64, device=cuda)
    o = gather_positions(tensors[:1], bad)[0]
    assert torch.equal(o[:, :, 0], tensors[0][:, :, 1]) and torch.all(o[:, :, 1:] == 0)


def test_caches_prune_to_the_selected_positions(cuda):
    """CABCache / H2OCache decode loop on one layer: every eviction keeps
    keep_size rows in position order (CABCache: always the newest local
    window), and the stored rows stay the original rows of those positions."""
    from cab_attention.cache import CABCache, H2OCache
    B, H, D = 1, 2, 64
    for cache in (CABCache(max_cache_size=100, sparsity=0.5, eviction_interval=5, device="cuda"),
                  H2OCache(max_cache_size=100, sparsity=0.5, eviction_interval=5, device="cuda")):
        keep_size = int(100 * 0.5 * 0.9)
        pos = []
        g = torch.Generator().manual_seed(11)
        for step in range(140):
            n_before = cache.get_seq_length(0)
            att = torch.rand(B, H, 1, n_before + 1, generator=g).to(cuda)
            kv = torch.full((B, H, 1, D), float(step), device=cuda)
            cache.update(kv, kv + 0.5, 0, att)
            pos.append(step)
            rows = cache.key_cache[0][0, 0, :, 0].round().long().cpu().tolist()
            if len(rows) != len(pos):  # evicted
                assert len(rows) == keep_size and rows == sorted(rows) and set(rows) <= set(pos)
                if isinstance(cache, CABCache):
                    assert rows[-13:] == pos[-13:]  # local window: int(45 * 0.3) newest
                pos = rows
            assert rows == pos
            assert torch.equal(cache.value_cache[0], cache.key_cache[0] + 0.5)
            assert len(cache.importance_tracker) in (len(pos), len(pos) - 1)
        assert cache.total_evictions > 3


def test_cab_cache_reference_demo_replay(cuda):
    """The reference's CABCache demo (cab_cache.py:270-327): 200 decode steps
    over 4 layers, max_cache_size 100, sparsity 0.9, eviction interval 5,
    random attention on layer 0. Every selection the cache makes is checked
    bit for bit against the oracle on the same fp32 importance scores; after
    every eviction each layer holds exactly its old rows at the kept
    positions; the statistics follow the evictions."""
    from cab_attention.cache import CABCache
    cache = CABCache(max_cache_size=100, sparsity=0.9, local_ratio=0.3, bridge_ratio=0.2,
                     importance_ratio=0.5, eviction_interval=5, device="cuda")
    calls = []
    policy = cache.eviction_policy
    inner = policy.select_indices

    def recording(cache_len, keep_size, importance_scores, attention_matrix=None, device="cuda"):
        keep, diag = inner(cache_len, keep_size, importance_scores, attention_matrix, device)
        sc = None if importance_scores is None else importance_scores.detach().float().cpu().numpy().copy()
        calls.append((cache_len, keep_size, sc, keep.cpu().numpy()))
        return keep, diag

    policy.select_indices = recording
    B, H, D, layers = 1, 8, 64, 4
    g = torch.Generator().manual_seed(5)
    ids = [[] for _ in range(layers)]  # token id of each stored row, per layer
    evicted_tokens = 0
    for step in range(200):
        for layer in range(layers):
            tok = float(step * 10 + layer)
            kv = torch.full((B, H, 1, D), tok, device=cuda)
            att = None
            if layer == 0 and cache.get_seq_length(0) > 0:
                n = cache.get_seq_length(0)
                att = torch.rand((B, H, 1, n), generator=g).to(cuda)
                att = att / att.sum(dim=-1, keepdim=True)
            before = len(calls)
            old = [list(x) for x in ids]
            ids[layer].append(tok)
            cache.update(kv, kv + 0.25, layer, att)
            if len(calls) > before:  # an eviction: every layer keeps the same positions
                cache_len, keep_size, sc, keep = calls[-1]
                local = int(keep_size * 0.3)
                bridge = int(keep_size * 0.2)
                imp = keep_size - local - bridge
                want, _, _ = O.evict_select(sc, cache_len, min(local, cache_len), imp,
                                            min(bridge, cache_len), True, 1 if sc is not None else 3)
                assert np.array_equal(keep, want), f"step {step} layer {layer}"
                evicted_tokens += cache_len - keep.size
                ids = [[row[int(k)] for k in keep] for row in (old[:layer] + [ids[layer]] + old[layer + 1:])]
            for l2 in range(layers):
                if l2 < len(cache.key_cache) and cache.key_cache[l2] is not None:
                    got = cache.key_cache[l2][0, 0, :, 0].cpu().tolist()
                    assert got == ids[l2], f"step {step} layer {l2}"
                    assert torch.equal(cache.value_cache[l2], cache.key_cache[l2] + 0.25)
    assert cache.total_evictions == len(calls) > 10
    st = cache.get_stats()
    assert st["total_evictions"] == len(calls)
    assert st["total_tokens_evicted"] == evicted_tokens
    assert st["total_tokens_processed"] == 200 * layers
    assert len(cache) == cache.get_seq_length(0) <= int(100 * 1.1) + 1


@pytest.mark.parametrize("n", [32768, 40001, 65536 + 123])
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_evict_select_multi_workgroup_path(cuda, n, mode):
    """Caches of 32768 positions and more run one workgroup per 4096-position
    segment (workspace bitmap and histograms); positions, counts and
    categories stay bit-exact against the oracle: normal, tie-heavy and
    NaN/inf/-0 scores, missing and short score vectors, with and without the
    fallback, and given bridge scores with ties across segments."""
    rng = np.random.default_rng(n + mode)
    budgets = [(n // 10, n // 4, n // 5), (5, n // 3, n), (0, 7, 3)]
    for name, s in score_cases(rng, n):
        for local, imp, br in budgets:
            bs = rng.integers(0, 5, n).astype(np.float32) if mode == 2 else None
            for fb in (True, False):
                keep, cnt, cat, dev = run_select(cuda, s, n, local, imp, br, fb, mode, bridge_scores=bs)
                wk, wc, wcat = O.evict_select(s, n, local, imp, br, fb, mode, bridge_scores=bs)
                msg = f"{name} n={n} budgets={(local, imp, br)} fb={fb}"
                assert tuple(cnt) == tuple(wc), msg
                assert np.array_equal(keep, wk), msg
                assert np.array_equal(cat, wcat), msg
                assert list(dev) == [wc[0], wc[1], wc[2], wk.size], msg
    for scores in (None, rng.standard_normal(n // 3).astype(np.float32)):
        for fb in (True, False):
            bs = rng.random(n).astype(np.float32)
            keep, cnt, cat, _ = run_select(cuda, scores, n, 100, n // 4, n // 6, fb, mode,
                                           bridge_scores=bs)
            wk, wc, wcat = O.evict_select(scores, n, 100, n // 4, n // 6, fb, mode, bridge_scores=bs)
            assert tuple(cnt) == tuple(wc) and np.array_equal(keep, wk) and np.array_equal(cat, wcat)
