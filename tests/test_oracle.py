"""Pins the CPU oracle against the reference's stored answers, closed forms,
invariants and brute force (CPU only)."""

import json
import math

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import cab_oracle as O


# ---------------------------------------------------------------------------
# canonical squared norm
# ---------------------------------------------------------------------------

def test_sqnorm_exact_on_small_integers():
    rng = np.random.default_rng(0)
    x = rng.integers(-8, 9, size=(5, 7, 128)).astype(np.float32)
    exact = (x.astype(np.int64) ** 2).sum(-1).astype(np.float64)
    np.testing.assert_array_equal(O.canonical_sqnorm(x), exact)


@pytest.mark.parametrize("d", [8, 64, 96, 128, 256])
def test_sqnorm_within_ulps_of_exactly_rounded_sum(d):
    rng = np.random.default_rng(d)
    x = (rng.standard_normal((50, d)) * rng.uniform(0.1, 100, (50, 1))).astype(np.float32)
    got = O.canonical_sqnorm(x)
    for r in range(50):
        ref = math.fsum(float(v) ** 2 for v in x[r].astype(np.float64))
        assert abs(got[r] - ref) <= 8 * np.spacing(ref)


def test_sqnorm_order_is_chunks_then_pairwise():
    # 2^54 has a float64 spacing of 4, so a lone +1 added to it is lost.
    # Chunk 0 = [2^27, 1 x 7] sums left to right to 2^54 (every 1 lost);
    # chunk 1 = [1 x 8] sums to 8; the pairwise step gives 2^54 + 8. A plain
    # left-to-right sum would give 2^54, the exactly rounded sum 2^54 + 16.
    x = np.ones(16, dtype=np.float32)
    x[0] = 2.0 ** 27
    assert O.canonical_sqnorm(x[None])[0] == 2.0 ** 54 + 8
    # Dropping the zero padding or reordering chunks must not change the value.
    x24 = np.concatenate([x, np.ones(8, np.float32)])
    x32 = np.concatenate([x24, np.zeros(8, np.float32)])
    assert O.canonical_sqnorm(x24[None])[0] == O.canonical_sqnorm(x32[None])[0]


def test_sqnorm_rejects_ragged_dim():
    with pytest.raises(ValueError):
        O.canonical_sqnorm(np.zeros((2, 12), np.float32))


# ---------------------------------------------------------------------------
# Max-L2 coarsening
# ---------------------------------------------------------------------------

def _brute_coarsen(x, bs):
    b, h, n, d = x.shape
    m = (n + bs - 1) // bs
    idx = np.zeros((b, h, m), np.int32)
    for bb in range(b):
        for hh in range(h):
            for mm in range(m):
                best, bt = -1.0, -1
                for t in range(mm * bs, min((mm + 1) * bs, n)):
                    v = math.fsum(float(e) ** 2 for e in x[bb, hh, t].astype(np.float64))
                    if v > best:
                        best, bt = v, t
                idx[bb, hh, mm] = bt
    return idx


@pytest.mark.parametrize("n,bs", [(64, 16), (100, 16), (37, 8)])
def test_coarsen_matches_brute_force(n, bs):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((2, 3, n, 16)).astype(np.float32)
    xc, idx = O.coarsen_max_l2(x, bs)
    np.testing.assert_array_equal(idx, _brute_coarsen(x, bs))
    for bb in range(2):
        for hh in range(3):
            np.testing.assert_array_equal(xc[bb, hh], x[bb, hh, idx[bb, hh]])
    m = (n + bs - 1) // bs
    blocks = idx // bs
    np.testing.assert_array_equal(blocks, np.broadcast_to(np.arange(m), blocks.shape))


def test_coarsen_planted_max_ties_and_nan():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 1, 64, 8)).astype(np.float32)
    x[0, 0, 5] *= 50                     # block 0: planted maximum
    x[0, 0, 20] = x[0, 0, 30] = 40.0     # block 1: exact tie -> lowest
    x[0, 0, 40] = np.nan                 # block 2: NaN wins
    x[0, 0, 41] = 1e6
    x[0, 0, 50] = x[0, 0, 60] = np.nan   # block 3: first NaN
    _, idx = O.coarsen_max_l2(x, 16)
    assert idx.ravel().tolist() == [5, 20, 40, 50]


def test_coarsen_identity_and_global():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 2, 10, 8)).astype(np.float32)
    xc, idx = O.coarsen_max_l2(x, 1)
    np.testing.assert_array_equal(xc, x)
    np.testing.assert_array_equal(idx[0, 0], np.arange(10))
    _, idx = O.coarsen_max_l2(x, 64)
    norms = (x.astype(np.float64) ** 2).sum(-1)
    np.testing.assert_array_equal(idx[..., 0], norms.argmax(-1))


# ---------------------------------------------------------------------------
# Coarse FRC
# ---------------------------------------------------------------------------

def _unit_scale_frc(qc, kc, **kw):
    d = qc.shape[-1]
    return O.compute_block_frc(qc, kc, temperature=1.0 / math.sqrt(d), **kw)


def test_bridge_known_answer():
    """test.ipynb:19-25: bridge FRC -85.71 and the retrieval flags."""
    adj = np.load(GOLDEN / "bridge_sbm_adj.npy")
    kat = json.loads((GOLDEN / "bridge_kat.json").read_text())
    n, d = adj.shape[0], 104
    qc = np.zeros((1, 1, n, d), np.float32)
    qc[0, 0, :, :n] = adj
    kc = np.zeros((1, 1, n, d), np.float32)
    kc[0, 0, :, :n] = np.eye(n, dtype=np.float32)
    f, ahat, t = _unit_scale_frc(qc, kc, normalization="none", formula="augmented")
    np.testing.assert_allclose(ahat[0, 0], adj, rtol=1e-12)
    u, v = kat["bridge"]
    assert round(float(f[0, 0, u, v]), 2) == kat["bridge_frc_2dp"]
    for sp, h2o, cab in zip(kat["sparsities"], kat["h2o_found"], kat["cab_found"]):
        assert bool(O.global_topk_mask(adj, sp, largest=True)[u, v]) == h2o
        assert bool(O.global_topk_mask(f[0, 0], sp, largest=False)[u, v]) == cab


def test_frc_identity_affinity():
    m, d, lam = 8, 16, 0.5
    eye = np.zeros((1, 1, m, d), np.float32)
    eye[0, 0, :, :m] = np.eye(m)
    f, ahat, t = _unit_scale_frc(eye, eye, normalization="none", lambda_redundancy=lam)
    np.testing.assert_allclose(t[0, 0], np.eye(m), atol=1e-12)
    np.testing.assert_allclose(f[0, 0], (1 - lam) * np.eye(m), atol=1e-12)
    fm, _, _ = _unit_scale_frc(eye, eye, normalization="none", formula="multiplicative",
                               lambda_redundancy=lam)
    np.testing.assert_allclose(np.diag(fm[0, 0]), 1 / (1 + lam / (1 + 1e-8)), rtol=1e-12)
    assert np.all(fm[0, 0][~np.eye(m, dtype=bool)] == 0)


def test_frc_all_ones_and_rank_one():
    m, d, lam = 6, 8, 0.3
    e1 = np.zeros((1, 1, m, d), np.float32)
    e1[..., 0] = 1
    f, ahat, t = _unit_scale_frc(e1, e1, normalization="none", lambda_redundancy=lam)
    np.testing.assert_allclose(t[0, 0], m * np.ones((m, m)), rtol=1e-12)
    np.testing.assert_allclose(f[0, 0], (1 - lam * m) * np.ones((m, m)), rtol=1e-12)
    rng = np.random.default_rng(3)
    uu = rng.uniform(0.5, 2, m).astype(np.float32)
    vv = rng.uniform(0.5, 2, m).astype(np.float32)
    qc = np.zeros((1, 1, m, d), np.float32)
    kc = np.zeros((1, 1, m, d), np.float32)
    qc[0, 0, :, 0] = uu
    kc[0, 0, :, 0] = vv
    _, _, t = _unit_scale_frc(qc, kc, normalization="none")
    u64, v64 = uu.astype(np.float64), vv.astype(np.float64)
    np.testing.assert_allclose(t[0, 0], np.dot(v64, u64) * np.outer(u64, v64), rtol=1e-12)


def test_frc_block_diagonal_and_permutation():
    rng = np.random.default_rng(4)
    m, d = 12, 16
    qc = np.zeros((1, 1, m, d), np.float32)
    kc = np.zeros((1, 1, m, d), np.float32)
    qc[0, 0, :6, :8] = rng.standard_normal((6, 8))
    qc[0, 0, 6:, 8:] = rng.standard_normal((6, 8))
    kc[0, 0, :6, :8] = rng.standard_normal((6, 8))
    kc[0, 0, 6:, 8:] = rng.standard_normal((6, 8))
    _, _, t = O.compute_block_frc(qc, kc, normalization="none")
    assert np.all(t[0, 0, :6, 6:] == 0) and np.all(t[0, 0, 6:, :6] == 0)
    f, _, _ = O.compute_block_frc(qc, kc)
    perm = rng.permutation(m)
    fp, _, _ = O.compute_block_frc(qc[:, :, perm], kc[:, :, perm])
    np.testing.assert_allclose(fp[0, 0], f[0, 0][np.ix_(perm, perm)], rtol=1e-10, atol=1e-12)


def test_frc_minmax_range_temperature_and_constant():
    rng = np.random.default_rng(5)
    qc = rng.standard_normal((2, 2, 20, 32)).astype(np.float32)
    kc = rng.standard_normal((2, 2, 20, 32)).astype(np.float32)
    f1, a1, _ = O.compute_block_frc(qc, kc, temperature=1.0)
    f2, a2, _ = O.compute_block_frc(qc, kc, temperature=3.0)
    assert a1.min() == 0 and np.all(a1.max(axis=(-2, -1)) <= 1) and np.all(a1.max(axis=(-2, -1)) > 1 - 1e-6)
    np.testing.assert_allclose(a1, a2, atol=1e-7)
    np.testing.assert_allclose(f1, f2, rtol=1e-6, atol=1e-6)
    const = np.ones((1, 1, 4, 8), np.float32)
    _, ac, _ = O.compute_block_frc(const, const)
    np.testing.assert_allclose(ac, 8 / math.sqrt(8))  # max == min: left unnormalised


# ---------------------------------------------------------------------------
# Block mask
# ---------------------------------------------------------------------------

def _brute_mask(f, k, select_high, keep_diag, causal):
    m = f.shape[0]
    rows = []
    for i in range(m):
        cand = list(range(i + 1 if causal else m))
        krow = min(k, len(cand))
        chosen = [i] if keep_diag else []
        rest = [j for j in cand if not (keep_diag and j == i)]
        sign = -1.0 if select_high else 1.0
        rest.sort(key=lambda j: (sign * (0.0 if f[i, j] == 0 else float(f[i, j])), j))
        chosen += rest[:krow - len(chosen)]
        rows.append(sorted(chosen))
    return rows


@pytest.mark.parametrize("select_high", [False, True])
@pytest.mark.parametrize("keep_diag", [False, True])
@pytest.mark.parametrize("causal", [False, True])
def test_mask_matches_brute_force(select_high, keep_diag, causal):
    rng = np.random.default_rng(6)
    m = 24
    f = rng.integers(-3, 4, size=(1, 2, m, m)).astype(np.float32)  # many ties
    f[0, 0, 3, 4] = -0.0
    mask, idx, cnt = O.generate_block_mask(f, 0.8, select_high, keep_diag, causal)
    k = O.keep_count(m, 0.8)
    for h in range(2):
        want = _brute_mask(f[0, h], k, select_high, keep_diag, causal)
        for i in range(m):
            got = idx[0, h, i, :cnt[0, h, i]].tolist()
            assert got == want[i]
            assert np.all(idx[0, h, i, cnt[0, h, i]:] == -1)
            assert sorted(np.flatnonzero(mask[0, h, i]).tolist()) == want[i]
            assert cnt[0, h, i] == min(k, i + 1 if causal else m)
            if keep_diag:
                assert mask[0, h, i, i]
            if causal:
                assert not mask[0, h, i, i + 1:].any()
    assert O.effective_sparsity(mask) == pytest.approx(1 - cnt.sum() / mask.size)


def _brute_hybrid(f, mag, k, kmag, select_high, keep_diag, causal):
    """Python-loop restatement of the hybrid rule, written independently of
    the oracle: diagonal, then the largest magnitudes, then FRC order."""
    m = f.shape[0]
    rows = []
    for i in range(m):
        cand = list(range(i + 1 if causal else m))
        krow = min(k, len(cand))
        chosen = [i] if keep_diag else []
        rest = [j for j in cand if not (keep_diag and j == i)]
        need = krow - len(chosen)
        nm = min(kmag, need)
        by_mag = sorted(rest, key=lambda j: (-(0.0 if mag[i, j] == 0 else float(mag[i, j])), j))
        chosen += by_mag[:nm]
        rest = [j for j in rest if j not in by_mag[:nm]]
        sign = -1.0 if select_high else 1.0
        rest.sort(key=lambda j: (sign * (0.0 if f[i, j] == 0 else float(f[i, j])), j))
        chosen += rest[:need - nm]
        rows.append(sorted(chosen))
    return rows


@pytest.mark.parametrize("ratio", [0.0, 0.25, 0.5, 1.0])
@pytest.mark.parametrize("select_high,keep_diag,causal", [(True, True, False), (False, True, True),
                                                          (True, False, True), (False, False, False)])
def test_hybrid_mask_matches_brute_force(ratio, select_high, keep_diag, causal):
    rng = np.random.default_rng(11)
    m = 30
    f = rng.integers(-3, 4, size=(1, 2, m, m)).astype(np.float32)    # many ties
    mag = rng.integers(0, 5, size=(1, 2, m, m)).astype(np.float32)
    mask, idx, cnt = O.generate_block_mask(f, 0.7, select_high, keep_diag, causal,
                                           magnitude_scores=mag, magnitude_ratio=ratio)
    k = O.keep_count(m, 0.7)
    kmag = O.magnitude_quota(k, ratio)
    assert kmag == int(k * ratio)
    for h in range(2):
        want = _brute_hybrid(f[0, h], mag[0, h], k, kmag, select_high, keep_diag, causal)
        for i in range(m):
            assert idx[0, h, i, :cnt[0, h, i]].tolist() == want[i]
            assert sorted(np.flatnonzero(mask[0, h, i]).tolist()) == want[i]


def test_hybrid_mask_special_cases():
    rng = np.random.default_rng(12)
    f = rng.standard_normal((1, 1, 40, 40)).astype(np.float32)
    mag = rng.standard_normal((1, 1, 40, 40)).astype(np.float32)
    pure, _, _ = O.generate_block_mask(f, 0.8)
    ratio0, _, _ = O.generate_block_mask(f, 0.8, magnitude_scores=mag, magnitude_ratio=0.0)
    np.testing.assert_array_equal(pure, ratio0)               # no magnitude share: pure FRC
    # ratio 1: every non-diagonal slot by magnitude = pure selection on -|mag| order
    ratio1, _, _ = O.generate_block_mask(f, 0.8, magnitude_scores=mag, magnitude_ratio=1.0)
    bymag, _, _ = O.generate_block_mask(mag, 0.8, select_high=True)
    np.testing.assert_array_equal(ratio1, bymag)
    with pytest.raises(ValueError):
        O.magnitude_quota(10, 1.5)


def test_mask_nan_and_signed_zero_order():
    f = np.array([[[[0.0, -0.0, np.nan, 1.0, -1.0]] * 5]], np.float32)
    _, idx, cnt = O.generate_block_mask(f, 0.4, keep_diagonal=False)   # k = 3 per row
    assert idx[0, 0, 0].tolist() == [0, 1, 4]        # -1, then the tied zeros
    _, idx, _ = O.generate_block_mask(f, 0.8, select_high=True, keep_diagonal=False)  # k = 1
    assert idx[0, 0, 0].tolist() == [2]              # NaN is the largest


def test_keep_count_matches_survey_figures():
    assert O.keep_count(2000, 0.95) == 100
    assert O.keep_count(1024, 0.95) == 51
    assert O.keep_count(64, 0.95) == 3
    assert O.keep_count(512, 0.95) == 25
    assert O.keep_count(2048, 0.99) == 20
    assert O.keep_count(10, 1.0) == 1 and O.keep_count(10, 0.0) == 10


# ---------------------------------------------------------------------------
# Sparse attention
# ---------------------------------------------------------------------------

def _rand_qkv(rng, b, h, n, d):
    return [rng.standard_normal((b, h, n, d)).astype(np.float32) for _ in range(3)]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", [64, 70])
def test_sparse_attention_equals_dense_masked(causal, n):
    rng = np.random.default_rng(7)
    bs, d = 16, 8
    q, k, v = _rand_qkv(rng, 1, 2, n, d)
    m = (n + bs - 1) // bs
    f = rng.standard_normal((1, 2, m, m)).astype(np.float32)
    mask, idx, cnt = O.generate_block_mask(f, 0.5, causal=causal)
    got = O.sparse_attention(q, k, v, idx, cnt, bs, causal=causal)
    tok = O.expand_block_mask(mask, bs, n)
    if causal:
        tok = tok & np.tril(np.ones((n, n), bool))
    want = O.dense_masked_attention(q, k, v, tok)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_sparse_attention_all_kept_is_softmax_attention():
    rng = np.random.default_rng(8)
    q, k, v = _rand_qkv(rng, 1, 1, 32, 8)
    m = 4
    idx = np.tile(np.arange(m, dtype=np.int32), (1, 1, m, 1))
    cnt = np.full((1, 1, m), m, np.int32)
    got = O.sparse_attention(q, k, v, idx, cnt, 8)
    s = q[0, 0].astype(np.float64) @ k[0, 0].T.astype(np.float64) / math.sqrt(8)
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    np.testing.assert_allclose(got[0, 0], p @ v[0, 0], rtol=1e-12, atol=1e-12)


def test_sparse_attention_constant_scores_and_empty_rows():
    rng = np.random.default_rng(9)
    _, k, v = _rand_qkv(rng, 1, 1, 32, 8)
    q = np.zeros_like(k)
    idx = np.array([[[[1, 3], [0, -1], [2, -1], [0, 0]]]], np.int32)
    cnt = np.array([[[2, 1, 0, 1]]], np.int32)
    got = O.sparse_attention(q, k, v, idx, cnt, 8)
    np.testing.assert_allclose(got[0, 0, :8], np.broadcast_to(
        np.concatenate([v[0, 0, 8:16], v[0, 0, 24:32]]).astype(np.float64).mean(0), (8, 8)),
        rtol=1e-12)
    assert np.all(got[0, 0, 16:24] == 0)


def test_sparse_attention_float32_mode_tracks_float64():
    """The CPU baseline's float32 mode runs the same steps as the float64
    checker: outputs agree to float32 rounding, empty rows stay 0."""
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((1, 2, 300, 64)).astype(np.float32) for _ in range(3))
    f = rng.standard_normal((1, 2, 5, 5)).astype(np.float32)
    _, idx, cnt = O.generate_block_mask(f, 0.5, causal=True)
    cnt[0, 1, 2] = 0
    a = O.sparse_attention(q, k, v, idx, cnt, 64, causal=True)
    b = O.sparse_attention(q, k, v, idx, cnt, 64, causal=True, compute_dtype=np.float32)
    assert b.dtype == np.float32
    np.testing.assert_allclose(b, a, atol=1e-5)
    assert np.all(b[0, 1, 128:192] == 0)


def test_frc_tolerance_closed_form():
    """1e-3 (|Ahat| + |lambda| |Ahat| @ |Ahat|): the |.| is taken before the
    product (a signed Ahat would cancel inside Ahat @ Ahat), and a given
    t_abs is used as is."""
    a = np.array([[[[1.0, -2.0], [3.0, -4.0]]]])
    absa = np.abs(a[0, 0])
    want = 1e-3 * (absa + 0.5 * (absa @ absa))
    np.testing.assert_allclose(O.frc_tolerance(a, -0.5)[0, 0], want)
    np.testing.assert_allclose(O.frc_tolerance(a, 0.5, t_abs=np.zeros_like(a)), 1e-3 * np.abs(a))


def test_mask_far_differences_bands():
    """Identical masks: agreement 1, nothing far. A swap across the row
    threshold between two scores closer than their tolerances is a near-tie;
    the same swap with a wider gap is two far entries; the selection it
    compares against is generate_block_mask's."""
    rng = np.random.default_rng(8)
    f = rng.standard_normal((1, 2, 12, 12))
    k = 4
    mask = O.generate_block_mask(f, 0.625)[0]
    assert O.keep_count(12, 0.625) == k
    tol = np.full_like(f, 1e-6)
    assert O.mask_far_differences(mask, f, tol, k) == (1.0, 0)
    i = 5
    others = np.array([j for j in range(12) if j != i])
    order = others[np.argsort(f[0, 0, i, others], kind="stable")]
    t, u = order[k - 2], order[k - 1]  # the threshold entry and the first one left out
    f[0, 0, i, u] = f[0, 0, i, t] + 1e-7
    mask = O.generate_block_mask(f, 0.625)[0]
    assert O.keep_count(12, 0.625) == k
    swapped = mask.copy()
    swapped[0, 0, i, t], swapped[0, 0, i, u] = False, True
    agree, far = O.mask_far_differences(swapped, f, tol, k)
    assert far == 0 and agree == 1 - 2 / f.size
    f[0, 0, i, u] = f[0, 0, i, t] + 1e-3
    agree, far = O.mask_far_differences(swapped, f, tol, k)
    assert far == 1  # u sits 1e-3 above the threshold; t is the threshold itself
    wide = swapped.copy()
    wide[0, 1, 0, :] = ~wide[0, 1, 0, :]
    assert O.mask_far_differences(wide, f, tol, k)[1] >= 1 + 8


def test_estimate_flops_closed_form():
    e = O.estimate_flops(131072, 128)
    assert e["M"] == 2048
    assert e["triangles"] == 2 * 2048 ** 3
    assert e["matmul"] == 2 * 2048 ** 2 * 128
    assert e["total"] == e["coarsening"] + e["matmul"] + e["triangles"]


# ---------------------------------------------------------------------------
# dense_attention_scores (dense attention with per-key attention totals)
# ---------------------------------------------------------------------------

def test_dense_scores_uniform_closed_forms():
    """q = 0: every visible key gets the same weight. Non-causal: out = mean
    of V, lse = log(N_k), score = N_q / N_k. Causal (queries are the last N_q
    positions): query t sees t + off + 1 keys, so key s receives
    sum_{t : t + off >= s} 1 / (t + off + 1)."""
    rng = np.random.default_rng(0)
    nq, nk, d = 5, 9, 8
    q = np.zeros((1, 1, nq, d))
    k = rng.standard_normal((1, 1, nk, d))
    v = rng.standard_normal((1, 1, nk, d))
    out, lse, sc = O.dense_attention_scores(q, k, v)
    np.testing.assert_allclose(out[0, 0], np.broadcast_to(v[0, 0].mean(0), (nq, d)), atol=1e-12)
    np.testing.assert_allclose(lse[0, 0], np.log(nk), atol=1e-12)
    np.testing.assert_allclose(sc[0, 0], nq / nk, atol=1e-12)
    out, lse, sc = O.dense_attention_scores(q, k, v, causal=True)
    off = nk - nq
    for t in range(nq):
        np.testing.assert_allclose(out[0, 0, t], v[0, 0, :t + off + 1].mean(0), atol=1e-12)
        assert lse[0, 0, t] == pytest.approx(math.log(t + off + 1))
    want = [sum(1.0 / (t + off + 1) for t in range(nq) if t + off >= s) for s in range(nk)]
    np.testing.assert_allclose(sc[0, 0], want, atol=1e-12)


def test_dense_scores_invariants_and_manual_form():
    """Each query's probabilities sum to 1, so the key totals sum to the
    number of queries that see a key; the output equals the manual masked
    softmax (dense_masked_attention) on the same mask; more queries than keys
    leave the first rows with no key (output 0, lse -inf)."""
    rng = np.random.default_rng(1)
    for nq, nk, causal in [(7, 7, False), (7, 7, True), (3, 11, True), (12, 5, True)]:
        q, k, v = (rng.standard_normal((2, 2, n, 16)) for n in (nq, nk, nk))
        out, lse, sc = O.dense_attention_scores(q, k, v, causal=causal)
        seen = (np.arange(nq) + nk - nq >= 0) if causal else np.ones(nq, bool)
        np.testing.assert_allclose(sc.sum(-1), seen.sum(), atol=1e-9)
        mask = np.ones((2, 2, nq, nk), bool)
        if causal:
            mask &= np.arange(nk)[None, :] <= np.arange(nq)[:, None] + (nk - nq)
        np.testing.assert_allclose(out, O.dense_masked_attention(q, k, v, mask), atol=1e-12)
        assert np.all(out[:, :, ~seen] == 0) and np.all(np.isneginf(lse[:, :, ~seen]))


def test_dense_scores_match_torch_float64():
    """An independent float64 computation with torch: softmax of the masked
    scaled scores (column sums = key totals, logsumexp = lse) and
    scaled_dot_product_attention with a boolean mask for the output."""
    rng = np.random.default_rng(2)
    nq, nk, d = 6, 10, 32
    q, k, v = (torch.from_numpy(rng.standard_normal((1, 2, n, d))) for n in (nq, nk, nk))
    mask = torch.arange(nk)[None, :] <= torch.arange(nq)[:, None] + (nk - nq)
    s = (q @ k.transpose(-1, -2)) / math.sqrt(d)
    s = s.masked_fill(~mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    ref_out = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    out, lse, sc = O.dense_attention_scores(q.numpy(), k.numpy(), v.numpy(), causal=True)
    np.testing.assert_allclose(out, ref_out.numpy(), atol=1e-12)
    np.testing.assert_allclose(sc, p.sum(-2).numpy(), atol=1e-12)
    np.testing.assert_allclose(lse, torch.logsumexp(s, -1).numpy(), atol=1e-12)


def test_dense_scores_grouped_heads_equal_repeated_heads():
    """K / V with H_kv heads give the same result as K / V with every head
    repeated H / H_kv times (head h uses K/V head h // (H / H_kv))."""
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 6, 5, 8))
    k = rng.standard_normal((1, 2, 9, 8))
    v = rng.standard_normal((1, 2, 9, 8))
    got = O.dense_attention_scores(q, k, v, causal=True)
    want = O.dense_attention_scores(q, np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1), causal=True)
    for a, b in zip(got, want):
        np.testing.assert_array_equal(a, b)


# ---------------------------------------------------------------------------
# evict_select / evict_connectivity / kv_gather (KV-cache eviction)
# ---------------------------------------------------------------------------

def _masked_topk(scores, exclude, k):
    """torch.topk over scores with the excluded positions at -inf, the way
    the reference policies select (policy.py:96-110, h2o.py:71-77)."""
    t = torch.from_numpy(np.asarray(scores, np.float32)).clone()
    t[torch.from_numpy(exclude)] = -float("inf")
    return set(torch.topk(t, k, largest=True).indices.tolist())


def test_evict_select_matches_torch_on_tie_free_scores():
    """Tie-free scores: importance = torch.topk of the scores outside the
    local window; bridges = torch.topk of -|s - torch.median(remaining)|;
    the counts follow the budgets."""
    rng = np.random.default_rng(0)
    for n, local, imp, br in [(1000, 30, 50, 20), (257, 0, 100, 100), (64, 64, 10, 5), (10, 3, 20, 20)]:
        s = (rng.standard_normal(n) * 3).astype(np.float32)  # distinct values and distances
        keep, cnt, cat = O.evict_select(s, n, local, imp, br, True, 1)
        loc = np.zeros(n, bool)
        loc[n - local:] = True
        n_imp = min(imp, n - local)
        assert cnt == (local, n_imp, min(br, n - local - n_imp))
        if n_imp:
            assert set(np.flatnonzero(cat == 2)) == _masked_topk(s, loc, n_imp)
        sel = cat > 0
        if cnt[2]:
            med = torch.median(torch.from_numpy(s[~(loc | (cat == 2))])).item()
            want = _masked_topk(-np.abs(s - np.float32(med)), loc | (cat == 2), cnt[2])
            assert set(np.flatnonzero(cat == 3)) == want
        assert np.array_equal(keep, np.flatnonzero(sel))
        assert np.all(cat[n - local:] == 1)


def test_evict_select_ties_nan_and_order_invariants():
    """With many equal scores, NaN, +-inf and -0: every kept importance
    position ranks at or above every evicted candidate (NaN highest), and
    among equal scores at the boundary the lower positions are kept; -0 and
    +0 tie."""
    rng = np.random.default_rng(1)
    n = 500
    s = rng.integers(0, 5, n).astype(np.float32)
    s[[3, 77]] = np.nan
    s[[10, 11]] = np.inf
    s[[20, 21]] = -np.inf
    s[30], s[31] = -0.0, 0.0
    keep, (loc, n_imp, _), cat = O.evict_select(s, n, 40, 100, 0, True, 0)
    rank = np.where(np.isnan(s), np.inf, s)  # NaN ranks with (above) +inf
    imp_pos = np.flatnonzero(cat == 2)
    rest = np.flatnonzero(cat == 0)
    assert {3, 77} <= set(imp_pos) and {10, 11} <= set(imp_pos)
    thr = rank[imp_pos].min()
    assert np.all(rank[rest] <= thr)
    eq_kept = imp_pos[rank[imp_pos] == thr]
    eq_evicted = rest[rank[rest] == thr]
    assert eq_kept.size == 0 or eq_evicted.size == 0 or eq_kept.max() < eq_evicted.min()
    _, _, cat0 = O.evict_select(np.array([1, -0.0, 0.0, 2], np.float32), 4, 0, 2, 0, True, 0)
    assert list(np.flatnonzero(cat0 == 2)) == [0, 3]
    _, _, cat1 = O.evict_select(np.array([1, -0.0, 0.0, 2, -1], np.float32), 5, 0, 3, 0, True, 0)
    assert list(np.flatnonzero(cat1 == 2)) == [0, 1, 3]  # -0 == +0: the lower position


def test_evict_select_branches_and_padding():
    """No scores: fallback keeps the positions before the local window, and
    bridges fall back to the middle third of the rest; scores shorter than
    the cache are zero-padded, longer ones truncated; a NaN among the
    remaining scores makes the median NaN (every distance NaN: bridges in
    position order); H2O-style calls (no fallback) keep nothing without
    scores."""
    keep, cnt, cat = O.evict_select(None, 30, 5, 7, 6, True, 1)
    assert cnt == (5, 7, 6)
    assert list(np.flatnonzero(cat == 2)) == list(range(18, 25))
    assert list(np.flatnonzero(cat == 3)) == list(range(6, 12))  # 18 free: ranks 6..11
    _, cnt, _ = O.evict_select(None, 30, 5, 7, 0, False, 0)
    assert cnt == (5, 0, 0)
    s = np.array([5, 1, 9], np.float32)
    _, _, cat = O.evict_select(s, 6, 0, 4, 0, True, 0)
    assert list(np.flatnonzero(cat == 2)) == [0, 1, 2, 3]  # 9, 5, 1, then the first padded 0
    _, _, cat = O.evict_select(np.arange(10, dtype=np.float32), 4, 0, 2, 0, True, 0)
    assert list(np.flatnonzero(cat == 2)) == [2, 3]
    s = np.array([0, 1, 2, np.nan, 4, 5, 6, 7], np.float32)
    _, cnt, cat = O.evict_select(s, 8, 2, 0, 3, True, 1)
    assert list(np.flatnonzero(cat == 3)) == [0, 1, 2]
    s = np.array([0, 10, 20, 30, 40, 50, 60, 70, 80], np.float32)
    _, cnt, cat = O.evict_select(s, 9, 0, 0, 2, True, 1)  # lower median 40: nearest 40, then 30
    assert list(np.flatnonzero(cat == 3)) == [3, 4]


def test_evict_connectivity_and_gather():
    rng = np.random.default_rng(2)
    a = rng.random((9, 9))
    cat = np.array([0, 2, 0, 2, 1, 0, 2, 0, 3], np.uint8)
    imp = [1, 3, 6]
    want = a[imp, :].sum(0) * a[:, imp].sum(1)
    np.testing.assert_allclose(O.evict_connectivity(a, cat), want, rtol=1e-15)
    x = rng.standard_normal((2, 3, 7, 4)).astype(np.float32)
    assert np.array_equal(O.kv_gather(x, np.arange(7)), x)
    assert np.array_equal(O.kv_gather(x, np.arange(6, -1, -1)), x[:, :, ::-1])
    g = O.kv_gather(x, np.array([1, 9, -1, 0]))
    assert np.array_equal(g[:, :, 0], x[:, :, 1]) and np.all(g[:, :, 1:3] == 0)


def test_evict_select_positional_bridges_are_a_truncated_slice():
    """The positional branch is remaining[len // 3 : len // 3 + budget]
    (policy.py:172-184): a budget above len - len // 3 keeps fewer bridges."""
    keep, cnt, cat = O.evict_select(None, 100, 5, 33, 100, True, 3)
    assert cnt == (5, 33, 62 - 62 // 3)
    assert list(np.flatnonzero(cat == 3)) == list(range(20, 62))
    assert keep.size == 5 + 33 + 42


def test_token_frc_matches_the_triangle_loop_and_closed_forms():
    """S and T against the reference Triton kernels' literal loops
    (frc_triton.py:47-62, :98-119), and closed forms: A = I gives (1, 1, 5);
    the all-ones graph gives S = n, T = n^2; a rank-1 graph u v^T gives
    S = u sum(v) and T = u (v . u) sum(v). Relabelling the nodes permutes
    the result."""
    rng = np.random.default_rng(11)
    a = rng.random((7, 7))
    s, t, f = O.token_frc(a)
    n = a.shape[0]
    s_loop = [sum(a[i, j] for j in range(n)) for i in range(n)]
    t_loop = [sum(a[i, j] * a[j, k] for j in range(n) for k in range(n)) for i in range(n)]
    np.testing.assert_allclose(s, s_loop, rtol=1e-13)
    np.testing.assert_allclose(t, t_loop, rtol=1e-13)
    np.testing.assert_allclose(f, 2 * np.asarray(s_loop) + 3 * np.asarray(t_loop), rtol=1e-13)
    s, t, f = O.token_frc(np.eye(5))
    assert np.all(s == 1) and np.all(t == 1) and np.all(f == 5)
    s, t, f = O.token_frc(np.ones((6, 6)))
    assert np.all(s == 6) and np.all(t == 36) and np.all(f == 2 * 6 + 3 * 36)
    u, v = rng.random(9), rng.random(9)
    s, t, _ = O.token_frc(np.outer(u, v))
    np.testing.assert_allclose(s, u * v.sum(), rtol=1e-13)
    np.testing.assert_allclose(t, u * (v @ u) * v.sum(), rtol=1e-13)
    p = rng.permutation(7)
    for x, y in zip(O.token_frc(a[p][:, p]), O.token_frc(a)):
        np.testing.assert_allclose(x, y[p], rtol=1e-13)


def _frc_from_keys_torch(keys):
    """The reference's call sequence (scoring/frc.py:73-89 with
    compute_frc_pytorch, frc_triton.py:279-293) in torch float64."""
    import torch.nn.functional as F
    k = torch.from_numpy(np.asarray(keys, np.float64))
    kn = F.normalize(k.mean(dim=(0, 1)), dim=-1)
    att = F.relu(torch.mm(kn, kn.t()))
    att = att / (att.sum(dim=1, keepdim=True) + 1e-8)
    s = att.sum(dim=1)
    t = torch.matmul(att, att).sum(dim=1)
    return s.numpy(), t.numpy(), (4.0 * s - 2.0 * s + 3.0 * t).numpy()


def test_frc_from_keys_matches_torch_and_closed_forms():
    """Against torch float64 through the reference's own steps; then closed
    forms. Orthonormal (or antipodal: relu drops the -1) keys give G = I, so
    sigma = 1 / (1 + 1e-8), S = sigma, T = sigma^2; parallel keys give the
    all-ones G: S = n / (n + 1e-8), T = S^2; a zero key scores 0. The mean
    runs over batch and heads."""
    rng = np.random.default_rng(12)
    keys = rng.standard_normal((2, 3, 40, 16))
    got = O.frc_from_keys(keys)
    for x, y in zip((got["strengths"], got["triangles"], got["frc"]), _frc_from_keys_torch(keys)):
        np.testing.assert_allclose(x, y, rtol=1e-12)
    sig = 1.0 / (1.0 + 1e-8)
    eye = np.zeros((1, 1, 5, 8))
    eye[0, 0, np.arange(5), np.arange(5)] = rng.random(5) + 0.5
    r = O.frc_from_keys(eye)
    np.testing.assert_allclose(r["row_sums"], 1.0, rtol=1e-14)
    np.testing.assert_allclose(r["strengths"], sig, rtol=1e-14)
    np.testing.assert_allclose(r["triangles"], sig * sig, rtol=1e-14)
    anti = np.zeros((1, 1, 2, 4))
    anti[0, 0, 0, 0], anti[0, 0, 1, 0] = 2.0, -3.0
    np.testing.assert_allclose(O.frc_from_keys(anti)["frc"], 2 * sig + 3 * sig * sig, rtol=1e-14)
    u = rng.standard_normal(8)
    par = (rng.random(6)[:, None] + 0.1) * u[None, :]
    r = O.frc_from_keys(par[None, None])
    sp = 6 / (6 + 1e-8)
    np.testing.assert_allclose(r["row_sums"], 6.0, rtol=1e-14)
    np.testing.assert_allclose(r["strengths"], sp, rtol=1e-14)
    np.testing.assert_allclose(r["triangles"], sp * sp, rtol=1e-14)
    z = rng.standard_normal((1, 2, 4, 8))
    z[:, :, 2] = 0.0
    r = O.frc_from_keys(z)
    assert r["frc"][2] == 0.0 and r["strengths"][2] == 0.0 and np.all(r["frc"][[0, 1, 3]] > 0)
    base = rng.standard_normal((5, 8))
    delta = rng.standard_normal((2, 2, 5, 8))
    delta -= delta.mean(axis=(0, 1), keepdims=True)
    np.testing.assert_allclose(O.frc_from_keys(base[None, None] + delta)["frc"],
                               O.frc_from_keys(base[None, None])["frc"], rtol=1e-12)


def test_symmetrize_attention_broadcasting():
    """(agg.T + agg) / 2 of the (b, h)-mean: an explicit element loop for
    N_q == N_kv, and torch's broadcasting for a single query (a decode step:
    (a_x + a_y) / 2) or a single key."""
    rng = np.random.default_rng(13)
    att = rng.random((2, 3, 6, 6))
    got = O.symmetrize_attention(att)
    m = att.mean(axis=(0, 1))
    want = np.array([[(m[y, x] + m[x, y]) / 2 for y in range(6)] for x in range(6)])
    np.testing.assert_allclose(got, want, rtol=1e-15)
    one_q = rng.random((2, 2, 1, 7))
    a = one_q.mean(axis=(0, 1))[0]
    np.testing.assert_allclose(O.symmetrize_attention(one_q), (a[:, None] + a[None, :]) / 2, rtol=1e-15)
    t = torch.from_numpy(one_q).mean(dim=(0, 1))
    np.testing.assert_allclose(O.symmetrize_attention(one_q), ((t.T + t) / 2.0).numpy(), rtol=1e-15)
    one_k = rng.random((1, 2, 5, 1))
    b = one_k.mean(axis=(0, 1))[:, 0]
    np.testing.assert_allclose(O.symmetrize_attention(one_k), (b[:, None] + b[None, :]) / 2, rtol=1e-15)
