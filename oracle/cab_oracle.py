"""float64 numpy restatement of CAB-Attention's block-sparse hot path.

TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the CPU
baseline in ``bench.py``. The shipped package never imports this module.

The reference's hot-path modules (``cab_attention/coarse_predictor.py``,
``cab_attention/cab_attention.py``, ``cab_attention/kernels/coarsening.py``,
``cab_attention/kernels/frc_kernel.py``) are absent from the reference tree;
their behaviour is fixed by their call sites, README prose and notebook
cells, cited per function below. Inputs are float32 arrays whose values are
exactly representable in the caller's dtype (bf16 and fp16 values are exact
in float32), so a gather compares bit-for-bit after widening.

Pinning of each function (tests/test_oracle.py):

- ``canonical_sqnorm``: exact-arithmetic cases (small integers, where every
  summation order is exact), a bound against the exactly rounded sum
  (``math.fsum``), a hand-derived input whose value differs between the
  chunked-pairwise order, a plain left-to-right sum and the exact sum, and
  zero-padding invariance for D not a power of two.
- ``coarsen_max_l2``: brute-force loop on tiny inputs, planted maximum,
  exact ties (lowest index wins), NaN handling, block_size 1 = identity,
  block_size >= N = one global argmax, ragged last block.
- ``compute_block_frc``: the reference's only stored known answer, the
  bridge FRC of -85.71 (test.ipynb:19) reproduced through the full
  coarse-FRC path, plus closed forms (identity, all-ones, rank-1 and
  block-diagonal affinities), minmax range and temperature invariance.
- ``generate_block_mask``: brute-force per-row sort, exact counts,
  causal/diagonal rules, ascending index lists; the global-top-k variant
  reproduces test.ipynb's stored retrieval booleans (test.ipynb:20-25).
- ``sparse_attention``: dense masked attention in the reference's manual
  form (CAB_Attention_Colab.ipynb:376-382), all-kept equals dense softmax
  attention, constant scores give the mean of the kept V rows.
- ``estimate_flops``: closed forms.
- ``dense_attention_scores``: uniform scores (closed forms for the output,
  the log-sum-exp and the harmonic causal key totals), key totals summing
  to the number of queries that see a key, agreement with
  ``dense_masked_attention`` and with torch's float64 softmax / SDPA, and
  grouped K / V equal to repeated heads.
- ``evict_select``: on tie-free scores, torch.topk / torch.median applied as
  the reference policies do (policy.py:96-170, h2o.py:71-77); with ties and
  NaN, the ordering invariants (every kept score ranks at or above every
  evicted candidate, equal scores kept in position order); the budget
  arithmetic; the positional and fallback branches.
- ``evict_connectivity``: explicit sums over the importance rows and
  columns against numpy's fancy-indexed reductions.
- ``kv_gather``: identity and reversal permutations, out-of-range rows.
- ``token_frc``: the reference Triton kernel's literal triple loop
  (sum_j sum_k A_ij A_jk, frc_triton.py:90-119) on small graphs, closed
  forms (identity, all-ones, rank-1 uv^T), permutation equivariance.
- ``frc_from_keys``: torch float64 through the reference's own call
  sequence (mean, F.normalize, mm, relu, row normalisation, compute_frc),
  and closed forms (orthonormal keys: G = I; parallel keys: G = all-ones;
  antipodal keys: relu removes the -1; zero keys give 0).
- ``symmetrize_attention``: torch broadcasting of (agg.T + agg) / 2 for
  N_q == N_kv and the size-1 cases, and an explicit (x, y) loop.
"""

from __future__ import annotations

import math

import numpy as np

__all__ = [
    "token_frc",
    "frc_from_keys",
    "symmetrize_attention",
    "evict_select",
    "evict_connectivity",
    "kv_gather",
    "dense_attention_scores",
    "canonical_sqnorm",
    "coarsen_max_l2",
    "num_blocks",
    "keep_count",
    "compute_block_frc",
    "order_keys",
    "generate_block_mask",
    "magnitude_quota",
    "expand_block_mask",
    "effective_sparsity",
    "sparse_attention",
    "dense_masked_attention",
    "global_topk_mask",
    "estimate_flops",
    "frc_tolerance",
    "mask_far_differences",
    "NORM_CHUNK",
    "FRC_RTOL",
]

# Elements summed sequentially per partial before the pairwise tree.
NORM_CHUNK = 8

# Relative FRC tolerance of the north star (fp32 accumulation), applied to
# the magnitude of F's two terms because F = Ahat - lambda T cancels.
FRC_RTOL = 1e-3


def num_blocks(n: int, block_size: int) -> int:
    """M = ceil(N / block_size) (CAB_Attention_Colab.ipynb:203; methods.py:446)."""
    return (n + block_size - 1) // block_size


def keep_count(m: int, sparsity: float) -> int:
    """Blocks kept per row: max(1, int(M * (1 - sparsity))), clamped to M.

    Same integer floor as the H2O block analogue (methods.py:252) and the
    notebook's k_keep (CAB_Attention_Colab.ipynb:372), applied per row.
    """
    return min(m, max(1, int(m * (1.0 - sparsity))))


# ---------------------------------------------------------------------------
# Max-L2 coarsening
# ---------------------------------------------------------------------------

def canonical_sqnorm(x: np.ndarray) -> np.ndarray:
    """Squared L2 norm over the last axis, in a fixed float64 order.

    Each element is widened to float64 and squared (exact for fp32/bf16/fp16
    inputs). The D squares are cut into chunks of 8 consecutive elements,
    each chunk summed left to right; the chunk sums (zero-padded to a power
    of two) are then added pairwise, adjacent pairs first. The order is part
    of the specification so that argmax ties and near-ties resolve the same
    way on every device.
    """
    d = x.shape[-1]
    if d % NORM_CHUNK:
        raise ValueError(f"head dim {d} is not a multiple of {NORM_CHUNK}")
    sq = np.square(x.astype(np.float64))
    sq = sq.reshape(*x.shape[:-1], d // NORM_CHUNK, NORM_CHUNK)
    part = sq[..., 0].copy()
    for e in range(1, NORM_CHUNK):
        part = part + sq[..., e]
    nchunk = d // NORM_CHUNK
    width = 1 << (nchunk - 1).bit_length()
    if width != nchunk:
        pad = np.zeros((*part.shape[:-1], width - nchunk), dtype=np.float64)
        part = np.concatenate([part, pad], axis=-1)
    while part.shape[-1] > 1:
        part = part[..., 0::2] + part[..., 1::2]
    return part[..., 0]


def coarsen_max_l2(x: np.ndarray, block_size: int, compute_dtype=np.float64):
    """Max-L2 pooling: one representative token per block.

    ``idx[b,h,m] = argmax_{t in block m} ||x[b,h,t]||`` (first index on
    ties, NaN counts as the maximum, a ragged last block looks only at its
    valid tokens) and ``xc[b,h,m] = x[b,h,idx]``, a bitwise copy.
    Follows README.md:30-33 (Max-L2 pooling) and the coarsening contract of
    benchmarks/kernel_benchmark.py:82-85 and CAB_Attention_Colab.ipynb:109-141.
    Returns ``(xc, idx)``; idx is the absolute token index (int32).
    ``compute_dtype=np.float32`` forms the norms as one float32 dot product
    per token (the reference's torch path): the CPU baseline's timing mode,
    not a checker (its ties and near-ties are not canonical).
    """
    b, h, n, d = x.shape
    m = num_blocks(n, block_size)
    if compute_dtype == np.float64:
        norms = canonical_sqnorm(x)
    else:
        xf = np.asarray(x, dtype=compute_dtype)
        norms = np.einsum("...d,...d->...", xf, xf)
    padded = np.full((b, h, m * block_size), -np.inf, dtype=np.float64)
    padded[..., :n] = norms
    local = np.argmax(padded.reshape(b, h, m, block_size), axis=-1)
    idx = (local + np.arange(m)[None, None, :] * block_size).astype(np.int32)
    xc = np.take_along_axis(x, idx[..., None].astype(np.int64), axis=2)
    return xc, idx


# ---------------------------------------------------------------------------
# Coarse FRC
# ---------------------------------------------------------------------------

def compute_block_frc(q_coarse, k_coarse, temperature: float = 1.0,
                      lambda_redundancy: float = 0.5, formula: str = "additive",
                      normalization: str = "minmax", compute_dtype=np.float64):
    """Block-level Forman-Ricci curvature, float64.

    - Affinity ``A = Qc Kc^T / sqrt(D) / temperature``
      (kernel_benchmark.py:135-137; CAB_Attention_Colab.ipynb:361; methods.py:332).
    - Normalisation ``minmax``: ``(A - min) / (max - min + 1e-8)`` per (b, h),
      left unchanged when max == min
      (CAB_Attention_Colab.ipynb:249, cell 11 src l.75-81); ``none``: A.
    - Redundancy ``T = Ahat @ Ahat`` (README.md:36, :240; kernel_benchmark.py:143-144).
    - ``additive``: ``F = Ahat - lambda T`` (README.md:37, :236; Colab :367).
      ``multiplicative``: ``F = Ahat / (1 + lambda T / (Ahat + 1e-8))``
      (Colab :249, cell 11 src l.83-97). Non-finite F becomes 0 (cell 11
      src l.100-104).
      ``augmented``: test.ipynb's graph curvature
      ``4 Ahat - S_i - S_j + 3 T`` on edges (Ahat > 0), 1000 elsewhere, with
      ``S`` the row sums of Ahat (test.ipynb:111-145).
    Returns ``(frc, affinity, redundancy)`` with affinity the normalised Ahat.
    ``compute_dtype=np.float32`` runs the same steps in float32 (BLAS sgemm,
    as the reference's torch path does): the CPU baseline's timing mode, not
    a checker.
    """
    qc = np.asarray(q_coarse, dtype=compute_dtype)
    kc = np.asarray(k_coarse, dtype=compute_dtype)
    d = qc.shape[-1]
    a = np.matmul(qc, np.swapaxes(kc, -1, -2)) * (1.0 / math.sqrt(d)) / temperature
    if normalization == "minmax":
        mn = a.min(axis=(-2, -1), keepdims=True)
        mx = a.max(axis=(-2, -1), keepdims=True)
        ahat = np.where(mx > mn, (a - mn) / (mx - mn + 1e-8), a)
    elif normalization == "none":
        ahat = a
    else:
        raise ValueError(f"unknown normalization {normalization!r}")
    t = np.matmul(ahat, ahat)
    lam = float(lambda_redundancy)
    with np.errstate(all="ignore"):
        if formula == "additive":
            f = ahat - lam * t
            f = np.where(np.isfinite(f), f, 0.0)
        elif formula == "multiplicative":
            f = ahat * (1.0 / (1.0 + lam * (t / (ahat + 1e-8))))
            f = np.where(np.isfinite(f), f, 0.0)
        elif formula == "augmented":
            s = ahat.sum(axis=-1)
            f = 4.0 * ahat - s[..., :, None] - s[..., None, :] + 3.0 * t
            f = np.where(ahat > 0, f, 1000.0)
        else:
            raise ValueError(f"unknown formula {formula!r}")
    return f, ahat, t


# ---------------------------------------------------------------------------
# Block mask
# ---------------------------------------------------------------------------

def order_keys(values: np.ndarray, select_high: bool) -> np.ndarray:
    """Unsigned keys whose ascending order is the selection order.

    Ascending float order, -0.0 equal to +0.0, NaN above +inf; inverted when
    ``select_high`` so that the highest value comes first. float32 input
    gives uint32 keys, float64 gives uint64.
    """
    v = np.asarray(values)
    if v.dtype == np.float32:
        u, bits, nan = np.uint32, 32, np.uint32(0x7FC00000)
    elif v.dtype == np.float64:
        u, bits, nan = np.uint64, 64, np.uint64(0x7FF8000000000000)
    else:
        raise TypeError(f"unsupported dtype {v.dtype}")
    v = np.where(v == 0, np.zeros((), v.dtype), v)  # -0 -> +0
    raw = v.view(u).copy()
    raw = np.where(np.isnan(v), nan, raw)
    sign = u(1) << u(bits - 1)
    allones = ~u(0)
    key = np.where(raw & sign, raw ^ allones, raw | sign)
    if select_high:
        key = ~key
    return key


def magnitude_quota(k: int, magnitude_ratio: float) -> int:
    """Blocks per row reserved for the magnitude ranking in the hybrid mask:
    ``int(k * magnitude_ratio)`` clamped to ``[0, k]`` (the same integer
    floor as ``keep_count``). The reference defines the split only in words,
    "reserve X% of budget for top-magnitude blocks" (methods.py:404-418)."""
    if not 0.0 <= float(magnitude_ratio) <= 1.0:
        raise ValueError(f"magnitude_ratio must be in [0, 1], got {magnitude_ratio}")
    return min(k, max(0, int(k * float(magnitude_ratio))))


def generate_block_mask(frc, sparsity: float, select_high: bool = False,
                        keep_diagonal: bool = True, causal: bool = False,
                        magnitude_scores=None, magnitude_ratio: float = 0.5):
    """Per-row block selection (README.md:40-42; methods.py:339-345).

    Row i keeps ``k = keep_count(M, sparsity)`` blocks (``min(k, i+1)`` when
    causal, candidates ``j <= i``) with the lowest FRC (highest when
    ``select_high``), ties to the lower j. With ``keep_diagonal`` the block
    ``j = i`` is always kept and counts toward k.

    Hybrid (CAB V4, methods.py:404-418, :465-473): with ``magnitude_scores``
    the row first keeps ``min(magnitude_quota(k, ratio), need)`` candidates
    with the highest magnitude (``need`` = the row's count after the forced
    diagonal), then fills the rest of its count from the remaining candidates
    in FRC order.

    Returns ``(mask bool[B,H,M,M], kv_idx int32[B,H,M,k] ascending, -1
    padded, kv_cnt int32[B,H,M])``.
    """
    f = np.asarray(frc)
    b, h, m, m2 = f.shape
    assert m == m2
    k = keep_count(m, sparsity)
    keys = order_keys(f, select_high)
    kmag = 0
    if magnitude_scores is not None:
        mag = np.asarray(magnitude_scores)
        assert mag.shape == f.shape
        mkeys = order_keys(mag, True)
        kmag = magnitude_quota(k, magnitude_ratio)
    mask = np.zeros((b, h, m, m), dtype=bool)
    kv_idx = np.full((b, h, m, k), -1, dtype=np.int32)
    kv_cnt = np.zeros((b, h, m), dtype=np.int32)
    for i in range(m):
        ncand = i + 1 if causal else m
        krow = min(k, ncand)
        cand = np.arange(ncand)
        others = cand[cand != i] if keep_diagonal else cand
        need = krow - (1 if keep_diagonal else 0)
        need_m = min(kmag, need)
        for bb in range(b):
            for hh in range(h):
                chosen = [i] if keep_diagonal else []
                rest = others
                if need_m > 0:
                    order = np.argsort(mkeys[bb, hh, i, rest], kind="stable")
                    pick = rest[order[:need_m]]
                    chosen += pick.tolist()
                    rest = np.setdiff1d(rest, pick)
                order = np.argsort(keys[bb, hh, i, rest], kind="stable")
                chosen += rest[order[:need - need_m]].tolist()
                chosen = np.sort(np.asarray(chosen, dtype=np.int64))
                kv_idx[bb, hh, i, :krow] = chosen
                kv_cnt[bb, hh, i] = krow
                mask[bb, hh, i, chosen] = True
    return mask, kv_idx, kv_cnt


def frc_tolerance(ahat, lambda_redundancy: float, t_abs=None) -> np.ndarray:
    """Per-entry FRC tolerance ``FRC_RTOL * (|Ahat| + |lambda| (|Ahat| @ |Ahat|))``.

    ``t_abs`` may pass ``|Ahat| @ |Ahat|`` when it is known (under minmax
    normalisation Ahat >= 0, so it is the oracle's own T).
    """
    a = np.abs(np.asarray(ahat, dtype=np.float64))
    if t_abs is None:
        t_abs = np.matmul(a, a)
    return FRC_RTOL * (a + abs(float(lambda_redundancy)) * np.asarray(t_abs, dtype=np.float64))


def mask_far_differences(gpu_mask, frc, tol, k: int, keep_diagonal: bool = True,
                         causal: bool = False, select_high: bool = False):
    """Compares a device mask with the oracle's selection on the oracle's
    scores ``frc`` and tolerances ``tol`` (``frc_tolerance``).

    A differing entry (i, j) is a near-tie when its score lies within
    ``tol[i, j] + tol[i, t]`` of the row's threshold score, t being the
    oracle's threshold entry (the last one kept): two scores each within
    their tolerance of the oracle's can only swap order inside that band.
    Returns ``(agreement, far)``: the fraction of identical entries and the
    number of differing entries that are not near-ties (0 for a pass).
    """
    f = np.asarray(frc, dtype=np.float64)
    gm = np.asarray(gpu_mask, dtype=bool)
    b, h, m, _ = f.shape
    want = np.zeros_like(gm)
    far = 0
    for bb in range(b):
        for hh in range(h):
            for i in range(m):
                ncand = i + 1 if causal else m
                cand = np.arange(ncand)
                others = cand[cand != i] if keep_diagonal else cand
                need = min(k, ncand) - (1 if keep_diagonal else 0)
                keys = order_keys(f[bb, hh, i, others], select_high)
                order = others[np.argsort(keys, kind="stable")]
                kept = order[:need]
                row = np.zeros(m, dtype=bool)
                row[kept] = True
                if keep_diagonal:
                    row[i] = True
                want[bb, hh, i] = row
                diff = np.flatnonzero(row != gm[bb, hh, i])
                if diff.size == 0:
                    continue
                if need <= 0:
                    far += diff.size
                    continue
                t = kept[-1]
                theta = f[bb, hh, i, t]
                for j in diff:
                    if abs(f[bb, hh, i, j] - theta) > tol[bb, hh, i, j] + tol[bb, hh, i, t]:
                        far += 1
    return float((want == gm).mean()), far


def expand_block_mask(block_mask: np.ndarray, block_size: int, seq_len: int) -> np.ndarray:
    """Token-level mask from a block mask (methods.py:103-119)."""
    t = np.repeat(np.repeat(block_mask, block_size, axis=-2), block_size, axis=-1)
    return t[..., :seq_len, :seq_len]


def effective_sparsity(mask: np.ndarray) -> float:
    """``1 - mean(mask)`` (methods.py:99-101)."""
    return 1.0 - float(np.asarray(mask, dtype=np.float64).mean())


def global_topk_mask(scores: np.ndarray, sparsity: float, largest: bool) -> np.ndarray:
    """test.ipynb's whole-matrix top-k with threshold ties kept (test.ipynb:151-175)."""
    flat = np.sort(np.asarray(scores).ravel())
    k = max(1, int((1.0 - sparsity) * scores.size))
    if largest:
        return scores >= flat[::-1][k - 1]
    return scores <= flat[k - 1]


# ---------------------------------------------------------------------------
# Block-sparse attention executor
# ---------------------------------------------------------------------------

def sparse_attention(q, k, v, kv_idx, kv_cnt, block_size: int, scale=None,
                     causal: bool = False, heads=None, query_blocks=None,
                     compute_dtype=np.float64) -> np.ndarray:
    """Softmax attention over the kept key blocks of each query block.

    ``O_t = sum_s softmax_s(q_t . k_s * scale) v_s`` over the tokens s of
    the blocks listed in ``kv_idx[b,h,i,:kv_cnt]`` for the query block i
    holding t; with ``causal`` keys s > t are dropped; a query with no key
    gets 0 (the manual path's nan_to_num, CAB_Attention_Colab.ipynb:376-382;
    methods.py:103-119). ``scale`` defaults to 1/sqrt(D). float64 output
    ``[B,H,N,D]``; ``heads`` restricts the work to a list of (b, h) pairs and
    ``query_blocks`` to a list of block rows (other outputs stay 0).
    ``compute_dtype=np.float32`` runs the same steps in float32 (the
    reference's torch path upcasts bf16 inputs to fp32): the CPU baseline's
    timing mode, not a checker.
    """
    q = np.asarray(q, dtype=compute_dtype)
    k = np.asarray(k, dtype=compute_dtype)
    v = np.asarray(v, dtype=compute_dtype)
    b, h, n, d = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    m = num_blocks(n, block_size)
    out = np.zeros_like(q)
    pairs = heads if heads is not None else [(bb, hh) for bb in range(b) for hh in range(h)]
    rows = range(m) if query_blocks is None else query_blocks
    for bb, hh in pairs:
        for i in rows:
            t0, t1 = i * block_size, min((i + 1) * block_size, n)
            cnt = int(kv_cnt[bb, hh, i])
            if cnt == 0:
                continue
            blocks = kv_idx[bb, hh, i, :cnt]
            toks = np.concatenate([np.arange(j * block_size, min((j + 1) * block_size, n))
                                   for j in blocks])
            s = (q[bb, hh, t0:t1] @ k[bb, hh, toks].T) * q.dtype.type(scale)
            if causal:
                s = np.where(toks[None, :] > np.arange(t0, t1)[:, None], -np.inf, s)
            mx = s.max(axis=-1, keepdims=True)
            valid = np.isfinite(mx)
            e = np.exp(np.where(valid, s - np.where(valid, mx, 0), -np.inf))
            den = e.sum(axis=-1, keepdims=True)
            p = np.divide(e, den, out=np.zeros_like(e), where=den > 0)
            out[bb, hh, t0:t1] = p @ v[bb, hh, toks]
    return out


def dense_masked_attention(q, k, v, token_mask, scale=None) -> np.ndarray:
    """The reference's manual executor: ``masked_fill(-inf)``, softmax,
    ``nan_to_num`` (CAB_Attention_Colab.ipynb:376-382), in float64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    s = np.where(token_mask, s, -np.inf)
    with np.errstate(invalid="ignore"):
        mx = s.max(axis=-1, keepdims=True)
        e = np.exp(s - mx)
        p = e / e.sum(axis=-1, keepdims=True)
    p = np.nan_to_num(p, nan=0.0)
    return np.matmul(p, v)


def estimate_flops(n: int, d: int, block_size: int = 64) -> dict:
    """Per-(b, h) operation counts of the predictor.

    ``coarsening = 2 N D`` (norm squares and adds), ``matmul = 2 M^2 D``
    (affinity), ``triangles = 2 M^3`` (T = A @ A), ``total`` their sum.
    Contract: examples/demo_cab_attention.py:192-207,
    benchmarks/benchmark_predictor.py:114-130.
    """
    m = num_blocks(n, block_size)
    c = 2 * n * d
    a = 2 * m * m * d
    t = 2 * m * m * m
    return {"M": m, "coarsening": c, "matmul": a, "triangles": t, "total": c + a + t}


def dense_attention_scores(q, k, v, scale=None, causal: bool = False):
    """Dense attention with per-key attention totals, in float64.

    The computation of flash_attention_with_cumulative_scores
    (cab_attention/kernels/flash_attention_accumulate.py:23-169, :172-261):
    ``out_t = sum_s softmax_s(q_t . k_s * scale) v_s`` over the N_k keys, and
    per key the attention it receives, ``score_s = sum_t softmax_t(s)`` --
    the normalised probabilities the reference's eager path sums
    (experiments/longbench_qa/runner.py:680-685), not the kernel's
    running-maximum exponentials (:145-156). ``causal`` lets query t see keys
    ``s <= t + N_k - N_q`` (the queries are the last N_q positions; the
    reference leaves its causal line commented out, :107). q: ``[B,H,N_q,D]``,
    k, v: ``[B,H_kv,N_k,D]`` with H_kv dividing H (head h uses K/V head
    ``h // (H // H_kv)``, the reference's repeat_kv, :470-481).

    Returns (out ``[B,H,N_q,D]``, lse ``[B,H,N_q]`` natural log, -inf for a
    query seeing no key, scores ``[B,H,N_k]``); a query seeing no key gets 0.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    b, h, nq, d = q.shape
    hkv, nk = k.shape[1], k.shape[2]
    if h % hkv:
        raise ValueError("query heads must be a multiple of K/V heads")
    group = h // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    out = np.zeros((b, h, nq, d))
    lse = np.full((b, h, nq), -np.inf)
    scores = np.zeros((b, h, nk))
    allowed = np.ones((nq, nk), bool)
    if causal:
        allowed = np.arange(nk)[None, :] <= np.arange(nq)[:, None] + (nk - nq)
    for bb in range(b):
        for hh in range(h):
            kk, vv = k[bb, hh // group], v[bb, hh // group]
            s = np.where(allowed, (q[bb, hh] @ kk.T) * scale, -np.inf)
            mx = s.max(axis=1, keepdims=True)
            seen = np.isfinite(mx[:, 0])
            e = np.exp(np.where(seen[:, None], s - np.where(seen[:, None], mx, 0.0), -np.inf))
            den = e.sum(axis=1, keepdims=True)
            p = np.divide(e, den, out=np.zeros_like(e), where=den > 0)
            out[bb, hh] = p @ vv
            lse[bb, hh] = np.where(seen, mx[:, 0] + np.log(np.where(seen, den[:, 0], 1.0)), -np.inf)
            scores[bb, hh] = p.sum(axis=0)
    return out, lse, scores


def _asc_keys(x) -> np.ndarray:
    """uint32 keys whose ascending order is the float order with -0 == +0
    and NaN above +inf (the selection order of cab_evict_select)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).copy()
    u[x == 0] = 0
    u[np.isnan(x)] = 0x7FC00000
    neg = (u & 0x80000000) != 0
    return np.where(neg, ~u, u | 0x80000000).astype(np.uint32)


def evict_select(scores, cache_len: int, local: int, imp: int, bridge: int,
                 fallback: bool, mode: int, bridge_scores=None):
    """The positions a KV cache keeps: local window, importance, bridges.

    Restates ThreeComponentEvictionPolicy.select_indices
    (cab_attention/eviction/policy.py:40-225) and h2o_select_indices
    (eviction/h2o.py:16-94) with cab_evict_select's tie rule (torch.topk's
    order is unspecified): among equal keys the lower position wins, NaN
    ranks above +inf, -0 equals +0, and a kept position is never chosen
    again. ``scores`` is zero-padded / truncated to cache_len (policy.py:84-95, h2o.py:58-69).
    ``mode``: 0 no bridges, 1 nearest the lower median of the remaining
    scores (NaN if one is NaN; policy.py:143-170), 2 highest bridge_scores
    (policy.py:122-141; falls back to 1, or 3 without scores, when no
    importance position was kept), 3 the remaining positions of rank
    [remaining // 3, +budget) (policy.py:172-184). ``fallback``: with no
    scores, the ``imp`` positions before the local window (policy.py:111-115).

    Returns (kept positions ascending int64, (local, importance, bridge)
    counts, category uint8: 0 evicted, 1 local, 2 importance, 3 bridge).
    """
    n = cache_len
    s = np.zeros(n, np.float32)
    if scores is not None:
        sc = np.asarray(scores, dtype=np.float32).reshape(-1)
        m = min(sc.size, n)
        s[:m] = sc[:m]
    kept = np.zeros(n, bool)
    cat = np.zeros(n, np.uint8)
    kept[n - local:] = True
    cat[n - local:] = 1

    def take_smallest(keys, need, c):
        cand = np.flatnonzero(~kept)
        order = cand[np.lexsort((cand, keys[cand]))]
        sel = order[:need]
        kept[sel] = True
        cat[sel] = c

    n_imp = 0
    if scores is not None:
        n_imp = min(imp, n - local)
        if n_imp > 0:
            take_smallest(~_asc_keys(s), n_imp, 2)
    elif fallback and imp > 0:
        s0 = max(0, n - local - imp)
        kept[s0:n - local] = True
        cat[s0:n - local] = 2
        n_imp = n - local - s0
    free1 = n - local - n_imp
    if mode == 2 and n_imp == 0:
        mode = 1 if scores is not None else 3
    if mode == 1 and scores is None:
        mode = 3
    n_br = min(bridge, free1) if (bridge > 0 and free1 > 0 and mode != 0) else 0
    if n_br > 0:
        if mode == 1:
            valid = s[~kept]
            if np.isnan(valid).any():
                med = np.float32(np.nan)
            else:
                med = np.sort(valid)[(free1 - 1) // 2]
            dist = np.abs((s - np.float32(med)).astype(np.float32))
            take_smallest(_asc_keys(dist), n_br, 3)
        elif mode == 2:
            take_smallest(~_asc_keys(np.asarray(bridge_scores, np.float32).reshape(-1)[:n]), n_br, 3)
        else:
            cand = np.flatnonzero(~kept)
            sel = cand[free1 // 3:free1 // 3 + n_br]  # a slice: cut at the end
            n_br = sel.size
            kept[sel] = True
            cat[sel] = 3
    return np.flatnonzero(kept).astype(np.int64), (local, n_imp, n_br), cat


def evict_connectivity(attention, category) -> np.ndarray:
    """Bridge scores of the attention-matrix mode (policy.py:122-131):
    (sum over importance rows of A) * (sum over importance columns of A), in
    float64, with importance = category == 2."""
    a = np.asarray(attention, dtype=np.float64)
    imp = np.flatnonzero(np.asarray(category) == 2)
    from_ = np.zeros(a.shape[1])
    to = np.zeros(a.shape[0])
    for i in imp:
        from_ += a[i, :]
        to += a[:, i]
    return from_ * to


def kv_gather(x, keep) -> np.ndarray:
    """``x[:, :, keep, :]`` with out-of-range positions giving zero rows
    (cab_cache.py:207-210)."""
    x = np.asarray(x)
    keep = np.asarray(keep, dtype=np.int64)
    out = np.zeros(x.shape[:2] + (keep.size,) + x.shape[3:], x.dtype)
    ok = (keep >= 0) & (keep < x.shape[2])
    out[:, :, ok] = x[:, :, keep[ok]]
    return out



def token_frc(attention):
    """Token-level Forman-Ricci curvature of a weighted directed graph
    (compute_frc_pytorch, cab_attention/kernels/frc_triton.py:269-293):
    S = A.sum(1), T = (A @ A).sum(1), F = 4 S - 2 S + 3 T (node weight
    taken equal to S, :155-160). Returns (S, T, F) in float64."""
    a = np.asarray(attention, np.float64)
    s = a.sum(axis=1)
    t = (a @ a).sum(axis=1)
    return s, t, 4.0 * s - 2.0 * s + 3.0 * t


def frc_from_keys(keys):
    """FRCTracker.compute_from_keys without its update interval
    (cab_attention/scoring/frc.py:68-89): x = keys.mean((0, 1)),
    kn = x / max(|x|, 1e-12) (F.normalize), G = kn kn^T, A = relu(G) row-
    normalised by (row sum + 1e-8), then token_frc(A). Returns a dict with
    strengths, triangles, frc and row_sums (sum_j relu(G_ij))."""
    x = np.asarray(keys, np.float64).mean(axis=(0, 1))
    kn = x / np.maximum(np.linalg.norm(x, axis=-1, keepdims=True), 1e-12)
    g = np.maximum(kn @ kn.T, 0.0)
    r = g.sum(axis=1)
    a = g / (r[:, None] + 1e-8)
    s, t, f = token_frc(a)
    return {"strengths": s, "triangles": t, "frc": f, "row_sums": r}


def symmetrize_attention(attention):
    """The key-key matrix of FRCTracker.compute_from_attention for a 4-D
    input (scoring/frc.py:110-121): agg = mean over (b, h), then
    (agg.T + agg) / 2 under numpy (= torch) broadcasting, cut to
    [:n, :n] with n = min of its shape."""
    agg = np.asarray(attention, np.float64).mean(axis=(0, 1))
    sym = (agg.T + agg) / 2.0
    n = min(sym.shape)
    return sym[:n, :n]
