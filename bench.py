"""Benchmark of the CAB-Attention hot path on one MI355X.

Headline metric: "predictor ms @N=128k + block-sparse attn
TFLOP/s, % of roofline".

- ``value``: block-sparse attention throughput at BASELINE config 4
  (CABAttention forward, causal, bf16, B=1 H=32 N=65536 D=128, block_size 64,
  sparsity 0.95): useful kept-tile TFLOP per second of one executor step
  (V packing + the attention kernel), with Q/K/V and the predictor's block
  lists resident in HBM. One step = one ``cab_block_sparse_attn_fwd`` call.
- ``roofline``: the attention kernel alone (``cab_block_sparse_attn_fwd_packed``
  on pre-packed V) against the bf16 dense MFMA peak, timed with HIP events on
  the launch stream; ``traffic`` from the committed rocprofv3 PMC summary.
- ``predictor``: latency of CoarseCurvaturePredictor.forward (coarsen + FRC +
  mask, dense bool mask out) at config 3 (B=2 H=8 N=128000 D=128), per-stage
  times and the config-4 predictor + attention end-to-end time.
- ``bridge``: config 5 (structured bridge stress test, B=1 H=8 N=131072,
  sparsity 0.99): planted bridges kept, mask agreement with the CPU oracle on
  two heads, predictor + attention latency.
- ``cpu_baseline``: the numpy oracle (in float32) on a bounded sample of the
  config-4 attention workload, on this host's cores.
- ``fp32_executor``, ``eviction_path``, ``token_frc``: config 4 with fp32
  inputs; dense attention + per-key totals, eviction selection and the
  multi-layer K/V prune (the KV-eviction path); token-level FRC of an
  attention graph and of cached keys.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import re
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
PKG = ROOT / "bridge-aware-kv-cache-eviction-for-efficient-long-context-transformers_amd"
for _p in (str(ROOT), str(PKG)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "predictor ms @N=128k + block-sparse attn TFLOP/s, % of roofline"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
PEAK_FP32_TFLOPS = 157.3    # MI355X dense fp32 MFMA
TRAFFIC_FILE = ROOT / "profiles" / "attn_pair_config4_traffic.md"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def seeded_gpu(shape, seed, dtype, dev):
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(dtype)


def time_events(fn, iters: int):
    """Average ms of ``fn`` over ``iters`` calls, from events on the current
    stream (the stream every kernel of this package is launched on)."""
    import torch
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def read_traffic():
    """HBM bytes per executor launch from the committed PMC summary, if any."""
    if not TRAFFIC_FILE.exists():
        return None
    m = re.search(r"hbm_bytes_per_launch:\s*([0-9.eE+]+)", TRAFFIC_FILE.read_text())
    return float(m.group(1)) if m else None


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info
        n = [i.get("num_threads", 0) for i in threadpool_info() if i.get("user_api") == "blas"]
        if n:
            return max(n)
    except Exception:
        pass
    return os.cpu_count() or 1


def cpu_attention_baseline(q, k, v, idx, cnt, heads, flops_fn):
    """The oracle's block-sparse attention in float32 (the reference's torch
    path upcasts bf16 to fp32) on every query block of a few heads."""
    import numpy as np
    from oracle import cab_oracle as O
    hs = list(heads)
    qs = q[:, hs].float().cpu().numpy()
    ks = k[:, hs].float().cpu().numpy()
    vs = v[:, hs].float().cpu().numpy()
    ii = idx[:, hs].cpu().numpy()
    cc = cnt[:, hs].cpu().numpy()
    t0 = time.perf_counter()
    O.sparse_attention(qs, ks, vs, ii, cc, 64, causal=True, compute_dtype=np.float32)
    dt = time.perf_counter() - t0
    flops = flops_fn(ii, cc)
    return flops / dt / 1e12, dt, flops


def cpu_predictor_baseline(q, k, block_size, sparsity):
    """The oracle's predictor steps in float32 (float32 norms, BLAS sgemm for
    A and T = Ahat @ Ahat, per-row selection), as the reference's torch path
    runs them on bf16 inputs upcast to fp32, on one (b, h) unit of config 3;
    returns seconds (best of two runs)."""
    import numpy as np
    from oracle import cab_oracle as O
    q1 = q[:1, :1].float().cpu().numpy()
    k1 = k[:1, :1].float().cpu().numpy()
    best = float("inf")
    for _ in range(2):
        t0 = time.perf_counter()
        qc, _ = O.coarsen_max_l2(q1, block_size, compute_dtype=np.float32)
        kc, _ = O.coarsen_max_l2(k1, block_size, compute_dtype=np.float32)
        f, _, _ = O.compute_block_frc(qc, kc, lambda_redundancy=0.5, compute_dtype=np.float32)
        O.generate_block_mask(f, sparsity)
        best = min(best, time.perf_counter() - t0)
    return best


PREDICTOR_SWEEP_N = (1024, 2048, 4096, 8192, 16384, 32768, 65536, 131072)


def predictor_sweep(dev):
    """The reference's predictor harness (benchmarks/benchmark_predictor.py:59-99,
    :196-234): CoarseCurvaturePredictor(block_size=64, sparsity=0.95) on fp16
    Q, K iid N(0, 1) of shape [1, 8, N, 128] for N = 1024 ... 131072; 3
    warm-up calls, then 10 trials, each synchronised and timed by its own
    pair of events, mean and standard deviation in ms, and the 5 ms check at
    N = 131072. The call is forward(q, k), which returns the block mask."""
    import numpy as np
    import torch
    from cab_attention import CoarseCurvaturePredictor
    pred = CoarseCurvaturePredictor(block_size=64, sparsity=0.95)
    rows = []
    for n in PREDICTOR_SWEEP_N:
        q = seeded_gpu((1, 8, n, 128), 21, torch.float16, dev)
        k = seeded_gpu((1, 8, n, 128), 22, torch.float16, dev)
        for _ in range(3):
            pred(q, k)
        times = []
        for _ in range(10):
            torch.cuda.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            pred(q, k)
            end.record()
            torch.cuda.synchronize()
            times.append(start.elapsed_time(end))
        rows.append({"N": n, "M": (n + 63) // 64, "mean_ms": round(float(np.mean(times)), 4),
                     "std_ms": round(float(np.std(times)), 4)})
        del q, k
    torch.cuda.empty_cache()
    at = rows[-1]["mean_ms"]
    log("predictor sweep: " + ", ".join(f"N={r['N']} {r['mean_ms']:.3f} ms" for r in rows))
    return {"config": "benchmark_predictor.py harness: CoarseCurvaturePredictor(block_size=64, "
                      "sparsity=0.95), fp16 Q/K [1, 8, N, 128] iid N(0,1), forward(q, k) -> "
                      "block mask; 3 warm-ups, 10 trials each synchronised and event-timed",
            "rows": rows, "ms_at_131072": at, "target_ms": 5.0, "meets_target": at < 5.0}


def bridge_inputs(B, H, N, D, seed, dev, dtype, bs=64, clusters=16, run_blocks=64, noise=0.1,
                  n_bridges=4, bridge_scale=0.05):
    """Config 5: clustered keys/queries with planted low-magnitude bridges.

    Per (b, h): ``clusters`` centres ~ N(0, I_D); key block m belongs to run
    ``m // run_blocks`` and takes centre ``run % clusters``; every token is its
    centre plus ``noise`` * N(0, 1) (queries and keys drawn separately).
    ``n_bridges`` (query block i, key block j) pairs from a seeded permutation,
    with j in a different cluster than i, get ``K[j block] = bridge_scale *
    Q[i block]``. Returns ``q, k, pairs``.
    """
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    M = (N + bs - 1) // bs
    centres = torch.randn((B, H, clusters, D), generator=g, device=dev)
    cl = (torch.arange(M, device=dev) // run_blocks) % clusters
    tok = cl.repeat_interleave(bs)[:N]
    base = centres[:, :, tok]
    q = base + noise * torch.randn((B, H, N, D), generator=g, device=dev)
    k = base + noise * torch.randn((B, H, N, D), generator=g, device=dev)
    del base
    perm = torch.randperm(M, generator=g, device=dev).tolist()
    clh = cl.tolist()
    used, pairs = set(), []
    for i in perm:
        if i in used:
            continue
        j = next((x for x in perm if x not in used and x != i and clh[x] != clh[i]), None)
        if j is None:
            continue
        pairs.append((i, j))
        used |= {i, j}
        if len(pairs) == n_bridges:
            break
    for i, j in pairs:
        k[:, :, j * bs:(j + 1) * bs] = bridge_scale * q[:, :, i * bs:(i + 1) * bs]
    return q.to(dtype), k.to(dtype), pairs


def mask_agreement(gpu_mask, of, oa, ot, lam, keep, keep_diag=True, causal=False,
                   select_high=False):
    """Fraction of mask entries identical to the oracle's selection, and the
    number of differing entries that are not near-ties: an entry is a
    near-tie when its oracle score lies within the stated FRC tolerance,
    1e-3 (|Ahat| + |lambda| |Ahat| @ |Ahat|), of its own entry plus that of
    the row's threshold entry (0 far entries means every difference is a
    near-tie). Minmax normalisation: |Ahat| @ |Ahat| is the oracle's T."""
    from oracle import cab_oracle as O
    tol = O.frc_tolerance(oa, lam, t_abs=ot)
    return O.mask_far_differences(gpu_mask.cpu().numpy(), of, tol, keep, keep_diag, causal,
                                  select_high)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def predictor_only(args, dev, bs, D) -> int:
    """Config-3 predictor timing alone (one JSON line, no headline fields)."""
    import torch
    from cab_attention import CoarseCurvaturePredictor
    B3, H3, N3 = 2, 8, 128000
    q3 = seeded_gpu((B3, H3, N3, D), 1, torch.bfloat16, dev)
    k3 = seeded_gpu((B3, H3, N3, D), 2, torch.bfloat16, dev)
    pred3 = CoarseCurvaturePredictor(block_size=bs, sparsity=0.95, lambda_redundancy=0.5)
    for _ in range(args.warmup):
        pred3(q3, k3)
    ms = time_events(lambda: pred3(q3, k3), args.steps)
    print(json.dumps({"predictor_config3_ms": round(ms, 4), "steps": args.steps}), flush=True)
    return 0


def eviction_path(args, dev, D):
    """Dense attention + per-key softmax totals (flash_attention_with_cumulative_scores)
    at B=1 H=32 H_kv=8 N=16384 causal bf16."""
    import torch
    from cab_attention.kernels import flash_attention, key_scores
    Be, He, Hkve, Ne = 1, 32, 8, 16384
    qe = seeded_gpu((Be, He, Ne, D), 7, torch.bfloat16, dev)
    ke = seeded_gpu((Be, Hkve, Ne, D), 8, torch.bfloat16, dev)
    ve = seeded_gpu((Be, Hkve, Ne, D), 9, torch.bfloat16, dev)
    oute, lsee = flash_attention(qe, ke, ve, causal=True, return_lse=True)
    sce = key_scores(qe, ke, lsee, causal=True)
    fwd_ms = time_events(lambda: flash_attention(qe, ke, ve, causal=True, out=oute),
                         max(3, args.steps // 4))
    sc_ms = time_events(lambda: key_scores(qe, ke, lsee, causal=True, scores=sce),
                        max(3, args.steps // 4))
    pairs_e = Be * He * Ne * (Ne + 1) // 2
    fwd_fl, sc_fl = 4 * D * pairs_e, 2 * D * pairs_e
    result_evict = {
        "config": "flash_attention_with_cumulative_scores: B=1 H=32 H_kv=8 N_q=N_k=16384 "
                  "D=128 causal bf16 (dense attention + per-key softmax totals)",
        "attention_ms": round(fwd_ms, 4),
        "attention_TFLOPs": round(fwd_fl / (fwd_ms * 1e-3) / 1e12, 1),
        "attention_frac_mfma": round(fwd_fl / (fwd_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "key_scores_ms": round(sc_ms, 4),
        "key_scores_TFLOPs": round(sc_fl / (sc_ms * 1e-3) / 1e12, 1),
        "key_scores_frac_mfma": round(sc_fl / (sc_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "total_ms": round(fwd_ms + sc_ms, 4),
    }
    log(f"eviction path: attention {fwd_ms:.3f} ms, key scores {sc_ms:.3f} ms")
    result_evict.update(eviction_prune(args, dev, sce.sum(dim=(0, 1)), ke))
    del qe, ke, ve, oute, lsee, sce
    torch.cuda.empty_cache()
    return result_evict


def eviction_prune(args, dev, importance, k_layer):
    """Position selection (cab_evict_select: local 30% / importance 50% /
    median bridges 20% of a keep budget of 20%) on the key totals of the
    dense pass, at N = 16384 and at the largest cache (2^20 positions), then
    the one-launch prune of 32 layers' K and V ([1, 8, 16384, 128] bf16) to
    the kept positions (cab_kv_gather), priced as HBM bytes moved."""
    import torch
    from cab_attention.eviction._select import BRIDGE_MEDIAN, select_positions
    from cab_attention.cache.prune import gather_into, gather_positions
    iters = max(5, args.steps)

    def budgets(n):
        keep = n // 5
        local, bridge = int(keep * 0.3), int(keep * 0.2)
        return local, keep - local - bridge, bridge

    n = importance.numel()
    sel = lambda sc, m: select_positions(m, sc, *budgets(m), False, BRIDGE_MEDIAN, dev)
    keep, cnt, _, _ = sel(importance, n)
    sel_ms = time_events(lambda: sel(importance, n), iters)
    big = 1 << 20
    big_scores = seeded_gpu((big,), 17, torch.float32, dev)
    sel(big_scores, big)
    sel_big_ms = time_events(lambda: sel(big_scores, big), iters)
    layers = 32
    tensors = [k_layer + i for i in range(2 * layers)]  # distinct K / V buffers
    # the store's prune path: rows gathered into the spare buffers it owns
    # (gather_positions, which allocates its outputs, is timed beside it)
    outs = gather_positions(tensors, keep)
    g_ms = time_events(lambda: gather_into(tensors, outs, keep, n, validate=False), iters)
    g_alloc_ms = time_events(lambda: gather_positions(tensors, keep), iters)
    B, H, _, D = k_layer.shape
    moved = 2 * len(tensors) * B * H * keep.numel() * D * k_layer.element_size()
    gbs = moved / (g_ms * 1e-3) / 1e9
    log(f"eviction prune: select {sel_ms * 1e3:.1f} us (N={n}), {sel_big_ms * 1e3:.1f} us "
        f"(N={big}); gather {g_ms * 1e3:.1f} us = {gbs:.0f} GB/s "
        f"({g_alloc_ms * 1e3:.1f} us with output allocation)")
    del tensors, big_scores, outs
    return {
        "select_config": f"cab_evict_select: keep {keep.numel()} of {n} (local/importance/"
                         f"bridge = {cnt}), median bridges, fp32 scores",
        "select_us": round(sel_ms * 1e3, 2),
        "select_us_at_2e20_positions": round(sel_big_ms * 1e3, 2),
        "gather_config": f"cab_kv_gather: {2 * layers} tensors [{B}, {H}, {n}, {D}] bf16 -> "
                         f"{keep.numel()} positions, into preallocated buffers (the store's "
                         f"prune path)",
        "gather_us_with_allocation": round(g_alloc_ms * 1e3, 2),
        "gather_us": round(g_ms * 1e3, 2),
        "gather_GBs": round(gbs, 1),
        "gather_frac_hbm": round(gbs / 8000.0, 4),
    }


def token_frc_section(args, dev):
    """Token-level FRC: compute_frc on a [16384, 16384] fp32 attention graph
    (two HBM passes, priced as 2 * 4 N^2 bytes) and
    FRCTracker.compute_from_keys on keys [1, 8, 16384, 128] bf16 (two MFMA
    Gram passes over the symmetric kn kn^T, priced as 2 * N^2 D useful flops,
    its upper triangle; the hi/lo split's extra products and the diagonal
    blocks' lower halves are not counted)."""
    import torch
    from cab_attention.kernels import frc_from_keys, token_frc
    iters = max(3, args.steps // 2)
    n = 16384
    a = torch.rand((n, n), generator=torch.Generator(device=dev).manual_seed(31), device=dev)
    a = a / a.sum(dim=1, keepdim=True)
    token_frc(a)
    m_ms = time_events(lambda: token_frc(a), iters)
    m_bytes = 2 * 4 * n * n
    del a
    torch.cuda.empty_cache()
    keys = seeded_gpu((1, 8, n, 128), 32, torch.bfloat16, dev)
    frc_from_keys(keys)
    k_ms = time_events(lambda: frc_from_keys(keys), iters)
    k_flops = 2 * n * n * 128
    del keys
    torch.cuda.empty_cache()
    log(f"token FRC: matrix {m_ms:.3f} ms ({m_bytes / (m_ms * 1e-3) / 1e9:.0f} GB/s), "
        f"keys {k_ms:.3f} ms ({k_flops / (k_ms * 1e-3) / 1e12:.0f} TFLOP/s)")
    return {
        "matrix_config": f"compute_frc: fp32 attention [{n}, {n}] (rows sum to 1)",
        "matrix_ms": round(m_ms, 4),
        "matrix_GBs": round(m_bytes / (m_ms * 1e-3) / 1e9, 1),
        "matrix_frac_hbm": round(m_bytes / (m_ms * 1e-3) / 8e12, 4),
        "keys_config": f"FRCTracker.compute_from_keys: keys [1, 8, {n}, 128] bf16",
        "keys_ms": round(k_ms, 4),
        "keys_TFLOPs": round(k_flops / (k_ms * 1e-3) / 1e12, 1),
        "keys_frac_mfma": round(k_flops / (k_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
    }


def reference_gemm(dev, kern_tflops, n=8192, iters=20):
    """torch.matmul on bf16 [n, n] x [n, n] (the vendor GEMM library PyTorch
    ships), event-timed: what a dense MFMA workload reaches on this box."""
    import torch
    a = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
    b = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
    f = lambda: torch.matmul(a, b)
    for _ in range(3):
        f()
    ms = time_events(f, iters)
    tf = 2 * n ** 3 / (ms * 1e-3) / 1e12
    del a, b
    torch.cuda.empty_cache()
    log(f"reference GEMM bf16 {n}^3: {ms:.3f} ms = {tf:.1f} TFLOP/s")
    return {"config": f"torch.matmul bf16 [{n}, {n}] x [{n}, {n}] (hipBLASLt), {iters} event-timed calls",
            "ms": round(ms, 4), "TFLOPs": round(tf, 1), "frac_of_peak": round(tf / PEAK_BF16_TFLOPS, 4),
            "executor_kernel_over_gemm": round(kern_tflops / tf, 4)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-heads", type=int, default=8,
                    help="config-4 heads the CPU baseline runs (every query block of each)")
    ap.add_argument("--attn-only", action="store_true",
                    help="skip the predictor and bridge sections")
    ap.add_argument("--predictor-only", action="store_true",
                    help="only time the config-3 predictor (for per-kernel profiles)")
    ap.add_argument("--predictor-sweep-only", action="store_true",
                    help="only run the reference predictor harness's sweep (N = 1k .. 128k)")
    ap.add_argument("--eviction-only", action="store_true",
                    help="only time the eviction path (dense attention + key totals; profiles)")
    ap.add_argument("--token-frc-only", action="store_true",
                    help="only time token-level FRC (matrix and keys forms; profiles)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(the path shards per (b, h) with no collectives; see the design notes).",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda:0")  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": src.numel() * 4,
                          "bytes_written": dst.numel() * 4, "launches": 3}))
        return 0

    from cab_attention import CoarseCurvaturePredictor
    from cab_attention.kernels import (block_sparse_attention, block_sparse_attention_packed,
                                       coarsen_qk_max_l2, compute_block_frc,
                                       generate_block_index, kept_tile_flops, pack_v)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bs, D = 64, 128
    if args.predictor_only:
        return predictor_only(args, dev, bs, D)
    if args.predictor_sweep_only:
        print(json.dumps({"predictor_sweep": predictor_sweep(dev)}), flush=True)
        return 0
    if args.token_frc_only:
        print(json.dumps({"token_frc": token_frc_section(args, dev)}), flush=True)
        return 0
    if args.eviction_only:
        print(json.dumps({"eviction_path": eviction_path(args, dev, D)}), flush=True)
        return 0

    # ---------------- config 4: predictor (causal) + block-sparse attention
    B, H, N, sp = 1, 32, 65536, 0.95
    log(f"config4 inputs B={B} H={H} N={N}")
    q = seeded_gpu((B, H, N, D), 1, torch.bfloat16, dev)
    k = seeded_gpu((B, H, N, D), 2, torch.bfloat16, dev)
    v = seeded_gpu((B, H, N, D), 3, torch.bfloat16, dev)
    pred4 = CoarseCurvaturePredictor(block_size=bs, sparsity=sp, lambda_redundancy=0.5,
                                     causal=True)
    idx, cnt = pred4.predict_index(q, k)
    torch.cuda.synchronize()
    flops = kept_tile_flops(idx, cnt, bs, D, N, causal=True)
    tiles = int(cnt.sum().item())
    out = torch.empty_like(q)
    # predictor + attention end to end first: it also brings the clocks up
    # before the timed executor steps
    e2e = lambda: block_sparse_attention(q, k, v, *pred4.predict_index(q, k), bs, causal=True,
                                         out=out)
    e2e()
    e2e_ms = time_events(e2e, max(3, args.steps // 4))
    attn = lambda: block_sparse_attention(q, k, v, idx, cnt, bs, causal=True, out=out)
    for _ in range(args.warmup):
        attn()
    torch.cuda.synchronize()
    log(f"timing {args.steps} executor steps ({flops / 1e12:.3f} TFLOP useful, {tiles} tiles)")
    attn_ms = time_events(attn, args.steps)
    attn_tflops = flops / (attn_ms * 1e-3) / 1e12
    # the attention kernel alone, on pre-packed V (roofline)
    vt = pack_v(v, bs)
    kern = lambda: block_sparse_attention_packed(q, k, vt, idx, cnt, bs, causal=True, out=out)
    for _ in range(args.warmup):
        kern()
    kern_ms = time_events(kern, args.steps)
    kern_tflops = flops / (kern_ms * 1e-3) / 1e12
    pack_ms = time_events(lambda: pack_v(v, bs), args.steps)
    log(f"step {attn_ms:.3f} ms = {attn_tflops:.1f} TFLOP/s; kernel {kern_ms:.3f} ms = "
        f"{kern_tflops:.1f} TFLOP/s; pack_v {pack_ms:.3f} ms; e2e {e2e_ms:.3f} ms")
    del vt

    result_pred = None
    result_bridge = None
    result_fp32 = None
    result_evict = None
    result_tfrc = None
    if not args.attn_only:
        # ---------------- config 4 in fp32 (split bf16 operands, fp32 output)
        q32, k32, v32 = (t.float() for t in (q, k, v))
        out32 = torch.empty_like(q32)
        run32 = lambda: block_sparse_attention(q32, k32, v32, idx, cnt, bs, causal=True, out=out32)
        run32()
        fp32_ms = time_events(run32, max(3, args.steps // 4))
        fp32_tflops = flops / (fp32_ms * 1e-3) / 1e12
        result_fp32 = {
            "config": "config4 inputs in fp32 (same lists); split bf16 hi+lo operands, three "
                      "bf16 MFMA products per product, fp32 output; step = pack K/V + attention",
            "ms": round(fp32_ms, 4),
            "TFLOPs": round(fp32_tflops, 1),
            "executed_bf16_mfma_TFLOPs": round(3 * fp32_tflops, 1),
            "executed_frac_of_bf16_mfma_peak": round(3 * fp32_tflops / PEAK_BF16_TFLOPS, 4),
        }
        log(f"fp32 executor {fp32_ms:.3f} ms = {result_fp32['TFLOPs']} TFLOP/s useful")
        del q32, k32, v32, out32
        torch.cuda.empty_cache()

        result_evict = eviction_path(args, dev, D)
        result_tfrc = token_frc_section(args, dev)

        # ---------------- config 3: predictor latency at N = 128k
        B3, H3, N3 = 2, 8, 128000
        q3 = seeded_gpu((B3, H3, N3, D), 1, torch.bfloat16, dev)
        k3 = seeded_gpu((B3, H3, N3, D), 2, torch.bfloat16, dev)
        pred3 = CoarseCurvaturePredictor(block_size=bs, sparsity=sp, lambda_redundancy=0.5)
        for _ in range(args.warmup):
            pred3(q3, k3)
        iters = max(5, args.steps)
        log("timing config3 predictor")
        pred_ms = time_events(lambda: pred3(q3, k3), iters)
        qc, kc = coarsen_qk_max_l2(q3, k3, bs)
        f3, _, _ = compute_block_frc(qc, kc, diagnostics=False)
        st_coarsen = time_events(lambda: coarsen_qk_max_l2(q3, k3, bs), iters)
        st_frc = time_events(lambda: compute_block_frc(qc, kc, diagnostics=False), iters)
        st_mask = time_events(lambda: generate_block_index(f3, sp, dense=True), iters)
        # CAB V4 hybrid selection (half of each row by magnitude): the coarse
        # affinity stands in for the block magnitudes here
        _, a3, _ = compute_block_frc(qc, kc)
        st_hybrid = time_events(lambda: generate_block_index(f3, sp, dense=True, select_high=True,
                                                             magnitude_scores=a3,
                                                             magnitude_ratio=0.5), iters)
        del a3
        M3 = (N3 + bs - 1) // bs
        k3keep = pred3.keep_per_row(N3)
        coarsen_bytes = 2 * B3 * H3 * N3 * D * 2 + 2 * B3 * H3 * M3 * (D * 2 + 4)
        tri_flops = 2 * M3 ** 3 * B3 * H3
        aff_flops = 2 * M3 ** 2 * D * B3 * H3
        mask_bytes = B3 * H3 * M3 * (M3 * 4 + k3keep * 4 + 4 + M3)
        result_pred = {
            "config": "config3: CoarseCurvaturePredictor B=2 H=8 N=128000 D=128 bs=64 "
                      "s=0.95 lambda=0.5 bf16, dense bool mask out",
            "ms": round(pred_ms, 4),
            "target_ms": 5.0,
            "stages_ms": {"coarsen": round(st_coarsen, 4), "frc": round(st_frc, 4),
                          "mask": round(st_mask, 4)},
            "coarsen_GBps": round(coarsen_bytes / (st_coarsen * 1e-3) / 1e9, 1),
            "coarsen_frac_hbm": round(coarsen_bytes / (st_coarsen * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "frc_TFLOPs": round((tri_flops + aff_flops) / (st_frc * 1e-3) / 1e12, 1),
            "frc_frac_mfma": round((tri_flops + aff_flops) / (st_frc * 1e-3) / 1e12
                                   / PEAK_BF16_TFLOPS, 4),
            "mask_GBps": round(mask_bytes / (st_mask * 1e-3) / 1e9, 1),
            "mask_frac_hbm": round(mask_bytes / (st_mask * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "hybrid_mask_ms": round(st_hybrid, 4),
            "config4_predictor_plus_attention_ms": round(e2e_ms, 4),
        }
        log(f"predictor {pred_ms:.3f} ms (coarsen {st_coarsen:.3f}, frc {st_frc:.3f}, "
            f"mask {st_mask:.3f})")
        if not args.no_cpu:
            cpu_s = cpu_predictor_baseline(q3, k3, bs, sp)
            result_pred["cpu_ms_estimate"] = round(cpu_s * 1e3 * B3 * H3, 1)
            result_pred["cpu_sample"] = ("oracle steps in float32 (BLAS sgemm) on 1 of 16 (b,h) "
                                         "units, scaled x16")
            result_pred["cpu_cores"] = blas_threads()
        del q3, k3, qc, kc, f3
        torch.cuda.empty_cache()
        result_pred["sweep"] = predictor_sweep(dev)

        # ---------------- config 5: structured bridge stress test
        B5, H5, N5, sp5 = 1, 8, 131072, 0.99
        log("config5 bridge inputs")
        q5, k5, pairs = bridge_inputs(B5, H5, N5, D, 5, dev, torch.bfloat16)
        v5 = seeded_gpu((B5, H5, N5, D), 6, torch.bfloat16, dev)
        pred5 = CoarseCurvaturePredictor(block_size=bs, sparsity=sp5, lambda_redundancy=0.5)
        out5 = torch.empty_like(q5)
        run5 = lambda: block_sparse_attention(q5, k5, v5, *pred5.predict_index(q5, k5), bs,
                                              out=out5)
        run5()
        e2e5_ms = time_events(run5, max(3, args.steps // 4))
        mask5, diag5 = pred5(q5, k5, return_diagnostics=True)
        kept = [[bool(mask5[0, h, i, j].item()) for (i, j) in pairs] for h in range(H5)]
        result_bridge = {
            "config": "config5: B=1 H=8 N=131072 D=128 bs=64 s=0.99 lambda=0.5 bf16; 16 "
                      "clusters in runs of 64 blocks, noise 0.1, 4 planted bridges "
                      "K[j] = 0.05 Q[i]",
            "bridges_qblock_kblock": pairs,
            "bridges_kept_per_head": [sum(r) for r in kept],
            "bridges_kept_total": f"{sum(sum(r) for r in kept)}/{len(pairs) * H5}",
            "predictor_plus_attention_ms": round(e2e5_ms, 4),
            "effective_sparsity": round(diag5["effective_sparsity"], 5),
        }
        # the reference's experiment wrappers keep the highest scores
        # (experiments/longbench_qa/methods.py:342)
        pred5h = CoarseCurvaturePredictor(block_size=bs, sparsity=sp5, lambda_redundancy=0.5,
                                          select_high=True)
        mask5h = pred5h(q5, k5)
        kept_h = [[bool(mask5h[0, h, i, j].item()) for (i, j) in pairs] for h in range(H5)]
        result_bridge["select_high_bridges_kept_per_head"] = [sum(r) for r in kept_h]
        result_bridge["select_high_bridges_kept_total"] = (
            f"{sum(sum(r) for r in kept_h)}/{len(pairs) * H5}")
        if not args.no_cpu:
            from oracle import cab_oracle as O
            heads5 = [0, 1]
            qh = q5[:, heads5].float().cpu().numpy()
            kh = k5[:, heads5].float().cpu().numpy()
            qc5, _ = O.coarsen_max_l2(qh, bs)
            kc5, _ = O.coarsen_max_l2(kh, bs)
            of5, oa5, ot5 = O.compute_block_frc(qc5, kc5, lambda_redundancy=0.5)
            k5keep = O.keep_count(of5.shape[-1], sp5)
            agree, far = mask_agreement(mask5[:, heads5], of5, oa5, ot5, 0.5, k5keep)
            agree_h, far_h = mask_agreement(mask5h[:, heads5], of5, oa5, ot5, 0.5, k5keep,
                                            select_high=True)
            om5 = O.generate_block_mask(of5, sp5)[0]
            om5h = O.generate_block_mask(of5, sp5, select_high=True)[0]
            okept = [[bool(om5[0, hh, i, j]) for (i, j) in pairs] for hh in range(len(heads5))]
            okept_h = [[bool(om5h[0, hh, i, j]) for (i, j) in pairs] for hh in range(len(heads5))]
            result_bridge["mask_agreement_vs_oracle"] = round(agree, 6)
            result_bridge["mask_diffs_not_near_threshold"] = far
            result_bridge["select_high_mask_agreement_vs_oracle"] = round(agree_h, 6)
            result_bridge["select_high_mask_diffs_not_near_threshold"] = far_h
            result_bridge["oracle_heads"] = heads5
            result_bridge["oracle_bridges_kept"] = [sum(r) for r in okept]
            result_bridge["oracle_select_high_bridges_kept"] = [sum(r) for r in okept_h]
            del mask5h
        log(f"bridge: kept {result_bridge['bridges_kept_total']}, e2e {e2e5_ms:.3f} ms")
        del q5, k5, v5, out5, mask5, diag5
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        heads = list(range(0, H, max(1, H // args.cpu_heads)))[:args.cpu_heads]

        def sample_flops(ii, cc):
            t = torch.from_numpy(ii)
            c = torch.from_numpy(cc)
            return kept_tile_flops(t, c, bs, D, N, causal=True)

        log(f"cpu baseline: oracle attention on heads {heads}")
        tfl, secs, fl = cpu_attention_baseline(q, k, v, idx, cnt, heads, sample_flops)
        cpu = {"value": round(tfl, 6), "unit": "TFLOP/s", "cores": blas_threads(),
               "kind": "port",
               "sample": f"numpy oracle in float32 (BLAS sgemm per query block), every query "
                         f"block of heads {heads} of config 4 ({fl / 1e9:.1f} GFLOP useful in "
                         f"{secs:.1f} s)",
               "host_cpu_count": os.cpu_count(), "host_cpu_model": cpu_model()}

    # The practical dense-MFMA ceiling of this box under the same sustained
    # load: torch's own bf16 GEMM (hipBLASLt), for context beside the
    # executor's roofline fraction. Not part of the measured path.
    result_gemm = reference_gemm(dev, kern_tflops)

    traffic = read_traffic()
    line = {
        "metric": METRIC,
        "value": round(attn_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(attn_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "config4: CABAttention causal block-sparse executor, B=1 H=32 "
                               "N=65536 D=128 bs=64 sparsity=0.95, predictor block lists",
                   "B": B, "H": H, "N": N, "D": D, "block_size": bs, "sparsity": sp,
                   "causal": True, "kept_tiles": tiles,
                   "useful_tflop_per_step": round(flops / 1e12, 4),
                   "pack_v_ms": round(pack_ms, 4), "attn_kernel_ms": round(kern_ms, 4)},
        "roofline": {"bound": "mfma", "achieved": round(kern_tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(kern_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic},
        "cpu_baseline": cpu,
        "predictor": result_pred,
        "bridge": result_bridge,
        "fp32_executor": result_fp32,
        "eviction_path": result_evict,
        "token_frc": result_tfrc,
        "reference_gemm": result_gemm,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
