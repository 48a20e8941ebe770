/*
 * cab_hip.h - C ABI of the MI355X (gfx950) CAB-Attention block-sparse path.
 *
 * libcab_hip.so exports the four stages of CAB-Attention's hot path:
 * Max-L2 coarsening, the coarse Forman-Ricci curvature (FRC) stage, the
 * per-row block-mask generator and the block-sparse attention executor.
 *
 * Conventions
 *  - Every buffer is device memory owned by the caller. The library never
 *    allocates, frees or synchronises; work is enqueued on `stream`
 *    (a hipStream_t, NULL for the default stream).
 *  - Tensors are [B, H, rows, cols]. Strides are in elements. The last
 *    dimension must be contiguous (stride 1) and rows 16-byte aligned.
 *  - All arguments are validated before any launch. A failed check returns
 *    a non-zero status and leaves a message for cab_last_error(); nothing
 *    is enqueued. A failed launch returns CAB_EHIP.
 *  - Calls are re-entrant; cab_last_error() is per host thread.
 *
 * The reference implementations these entry points replace are Python
 * functions that are imported by the reference's callers but are not in its
 * tree (cab_attention/kernels/coarsening.py, cab_attention/kernels/frc_kernel.py,
 * cab_attention/coarse_predictor.py, cab_attention/cab_attention.py); each
 * declaration cites the call sites that fix its contract.
 */
#ifndef CAB_HIP_H
#define CAB_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes, returned as cab_status_t. */
enum {
  CAB_OK = 0,
  CAB_EINVAL = 1,     /* bad scalar argument or null pointer */
  CAB_EDTYPE = 2,     /* unsupported element type */
  CAB_ESHAPE = 3,     /* unsupported or inconsistent shape / stride / alignment */
  CAB_EWORKSPACE = 4, /* workspace too small */
  CAB_EHIP = 5        /* HIP runtime error at launch */
};
typedef int32_t cab_status_t;

/* Element types, passed as cab_dtype_t. Both are plain 32-bit integers (an
 * enum's size and calling convention): any value a caller passes is a defined
 * value, which the validation rejects with CAB_EDTYPE unless it is one of these. */
enum { CAB_F32 = 0, CAB_F16 = 1, CAB_BF16 = 2 };
typedef int32_t cab_dtype_t;

/* Affinity normalisation (experiments/longbench_qa/config.py:466). */
enum { CAB_NORM_NONE = 0, CAB_NORM_MINMAX = 1 };

/* FRC combination (experiments/longbench_qa/config.py:465; test.ipynb:111-145). */
enum { CAB_FRC_ADDITIVE = 0, CAB_FRC_MULTIPLICATIVE = 1, CAB_FRC_AUGMENTED = 2 };

#define CAB_ABI_VERSION 10

int cab_abi_version(void);
const char* cab_last_error(void);

/*
 * Max-L2 coarsening of Q and K.
 * Replaces coarsen_qk_max_l2 / coarsen_qk_max_l2_pytorch (q, k, block_size)
 * -> (q_coarse, k_coarse) of cab_attention/kernels/coarsening.py (absent;
 * contract: benchmarks/kernel_benchmark.py:23, :82-85;
 * CAB_Attention_Colab.ipynb:109-141; README.md:30-33).
 *
 * For every (b, h, block m) of M = ceil(N / block_size) blocks, separately for
 * q and k: idx = argmax over the block's tokens of the squared L2 norm, summed
 * in float64 in a fixed order (chunks of 8 consecutive elements left to right,
 * then the chunk sums pairwise); ties go to the lowest token, NaN counts as
 * the largest. q_coarse[b,h,m,:] = q[b,h,idx,:] (bitwise copy).
 * q, k: [B,H,N,D] of `dtype`, D % 8 == 0, D <= 512. qc, kc: contiguous
 * [B,H,M,D] of `dtype`. q_idx, k_idx: contiguous int32 [B,H,M] (absolute token
 * index), may be NULL.
 */
cab_status_t cab_coarsen_maxl2(const void* q, const void* k, cab_dtype_t dtype,
                               int64_t B, int64_t H, int64_t N, int64_t D,
                               const int64_t q_strides[4], const int64_t k_strides[4],
                               int32_t block_size, void* qc, void* kc,
                               int32_t* q_idx, int32_t* k_idx, void* stream);

/*
 * Workspace bytes cab_block_frc needs for these sizes.
 */
size_t cab_block_frc_workspace_bytes(int64_t B, int64_t H, int64_t M, int64_t D,
                                     int normalization, int formula);

/*
 * Coarse FRC scores.
 * Replaces compute_block_frc(q_coarse, k_coarse, temperature, lambda_redundancy,
 * formula, normalization) -> (frc, affinity, redundancy) of
 * cab_attention/kernels/frc_kernel.py (absent; contract:
 * experiments/longbench_qa/methods.py:330-336; benchmarks/kernel_benchmark.py:149,
 * :253; README.md:34-38).
 *
 * A = qc kc^T * scale / temperature (fp32 accumulate on MFMA);
 * Ahat = minmax(A) per (b,h) ((A-min)/(max-min+1e-8), A unchanged if max==min)
 * or A; T = Ahat @ Ahat on MFMA with fp32 accumulate: under minmax with the
 * additive or multiplicative formula, one fp16 product per site (Ahat in
 * [0, 1]; |dT| <= 1e-3 (|Ahat| @ |Ahat|)), otherwise bf16 hi/lo operands
 * (three products, about 2^-16 relative). Additive without `triangles`: F is
 * accumulated directly as Ahat (I - lambda Ahat) (|lambda| <= 1024).
 * additive: F = Ahat - lambda T; multiplicative: F = Ahat / (1 + lambda T /
 * (Ahat + 1e-8)); non-finite F -> 0; augmented: 4 Ahat - S_i - S_j + 3 T on
 * entries with Ahat > 0 and 1000 elsewhere (S = row sums of Ahat).
 * qc, kc: contiguous [B,H,M,D] of `dtype`, D % 8 == 0, D <= 512.
 * frc (required), affinity (= Ahat) and triangles (= T) (nullable):
 * contiguous fp32 [B,H,M,M].
 */
cab_status_t cab_block_frc(const void* qc, const void* kc, cab_dtype_t dtype,
                           int64_t B, int64_t H, int64_t M, int64_t D,
                           float scale, float temperature, float lambda_redundancy,
                           int normalization, int formula,
                           float* frc, float* affinity, float* triangles,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * Per-row block selection.
 * Replaces generate_block_mask(frc, sparsity, select_high, keep_diagonal, causal)
 * of cab_attention/kernels/frc_kernel.py (absent; contract:
 * experiments/longbench_qa/methods.py:339-345; benchmarks/kernel_benchmark.py:197-205;
 * README.md:40-42); the caller computes k = max(1, int(M * (1 - sparsity))).
 *
 * Row i keeps min(k, #candidates) blocks: candidates are j <= i when causal,
 * all j otherwise; lowest scores first (highest when select_high), ties to the
 * lower j, -0.0 == +0.0, NaN above +inf. keep_diagonal forces j = i in (it
 * counts toward k).
 * frc: contiguous fp32 [B,H,M,M]. kv_idx: int32 [B,H,M,k], ascending, tail
 * filled with -1. kv_cnt: int32 [B,H,M]. dense_mask: uint8 0/1 [B,H,M,M] or NULL.
 * M <= 32768 (rows longer than 8192 take a slower kernel that re-reads the
 * row from memory on each search pass).
 */
cab_status_t cab_block_topk(const float* frc, int64_t B, int64_t H, int64_t M, int32_t k,
                            int select_high, int keep_diagonal, int causal,
                            int32_t* kv_idx, int32_t* kv_cnt, uint8_t* dense_mask,
                            void* stream);

/*
 * Hybrid per-row block selection (CAB V4).
 * Replaces generate_block_mask(frc, sparsity, select_high, keep_diagonal, causal,
 * magnitude_scores, magnitude_ratio) of cab_attention/kernels/frc_kernel.py
 * (absent; contract: experiments/longbench_qa/methods.py:404-418, :465-473;
 * benchmarks/kernel_benchmark.py:197-205); the caller computes
 * k_mag = int(k * magnitude_ratio).
 *
 * Row i selects as cab_block_topk, except that after the forced diagonal
 * its first min(k_mag, remaining count) blocks are the candidates with the
 * highest magnitude (ties to the lower j, -0.0 == +0.0, NaN above +inf); the
 * rest of its count comes from the remaining candidates in FRC order.
 * magnitude: contiguous fp32 [B,H,M,M]. 0 <= k_mag <= k.
 */
cab_status_t cab_block_topk_hybrid(const float* frc, const float* magnitude, int64_t B, int64_t H,
                                   int64_t M, int32_t k, int32_t k_mag, int select_high,
                                   int keep_diagonal, int causal, int32_t* kv_idx, int32_t* kv_cnt,
                                   uint8_t* dense_mask, void* stream);

/*
 * Workspace bytes cab_block_sparse_attn_fwd needs for `dtype`: per (b, h,
 * key block) one packed V^T tile (16 KB, bf16 / fp16) or one split K and
 * V^T image (64 KB, fp32). 0 for unsupported sizes or dtypes.
 */
size_t cab_block_sparse_attn_workspace_bytes(cab_dtype_t dtype, int64_t B, int64_t H, int64_t N,
                                             int64_t D, int32_t block_size);

/*
 * Workspace bytes cab_block_sparse_attn_fwd needs for any block size it
 * takes and lists of `kmax` entries: the packed tiles above, and for a
 * block size other than 64 the lists over 64-token tiles the call builds
 * (block_size 128, 256: kmax * block_size / 64 entries per 64-token row;
 * 8, 16, 32: kmax * 64 / block_size entries, each with a 64-bit sub-tile
 * mask). Equal to cab_block_sparse_attn_workspace_bytes for block_size 64.
 * 0 for unsupported arguments. Replaces nothing in the reference: its
 * FlexAttention executor sizes its own buffers (config.block_size,
 * experiments/longbench_qa/config.py:460; block sizes planned in TODO.md:117).
 */
size_t cab_block_sparse_attn_workspace_bytes_k(cab_dtype_t dtype, int64_t B, int64_t H, int64_t N,
                                               int64_t D, int32_t block_size, int32_t kmax);

/*
 * Block-sparse attention forward.
 * Replaces the executor inside CABAttention.forward of
 * cab_attention/cab_attention.py (absent; FlexAttention or the manual masked
 * softmax of README.md:44-46, CAB_Attention_Colab.ipynb:376-382 and
 * experiments/longbench_qa/methods.py:103-119).
 *
 * For query block i: out[t] = softmax_s(q_t . k_s * scale) v_s over the tokens
 * s of the key blocks kv_idx[b,h,i,0:kv_cnt[b,h,i]] (entries outside [0, M)
 * are skipped, kv_cnt is clamped to [0, kmax]); when causal, keys s > t are
 * dropped; a query with no key gets 0. fp32 online softmax, bf16/fp16 MFMA
 * (fp32 inputs: each operand split into a bf16 hi + lo pair, three MFMA
 * products per product, fp32 output; relative error near 2^-16 per product).
 * q, k, v: [B,H,N,D] (strides), out: [B,H,N,D] (strides), dtype bf16, fp16
 * or fp32.
 * block_size 8, 16, 32, 64, 128 or 256 (M = ceil(N / block_size)); for
 * 8, 16 and 32, kmax * 64 / block_size <= 4096. D == 64 or 128, scale > 0.
 * kv_idx: contiguous int32 [B,H,M,kmax], kv_cnt: contiguous int32 [B,H,M].
 * A block listed twice in a row counts twice. lse: fp32 [B,H,N]
 * natural-log log-sum-exp of the scaled scores (-inf for a query with no
 * key), or NULL. workspace: cab_block_sparse_attn_workspace_bytes_k(dtype,
 * ..., block_size, kmax) bytes (for block_size 64 also
 * cab_block_sparse_attn_workspace_bytes()), 16-byte aligned, overwritten
 * (V, and for fp32 K, is repacked there first; other block sizes' lists
 * are rewritten there over 64-token tiles).
 */
cab_status_t cab_block_sparse_attn_fwd(const void* q, const void* k, const void* v,
                                       cab_dtype_t dtype, int64_t B, int64_t H,
                                       int64_t N, int64_t D,
                                       const int64_t q_strides[4], const int64_t k_strides[4],
                                       const int64_t v_strides[4], const int64_t o_strides[4],
                                       int32_t block_size, const int32_t* kv_idx,
                                       const int32_t* kv_cnt, int32_t kmax, float scale,
                                       int causal, void* out, float* lse, void* workspace,
                                       size_t workspace_bytes, void* stream);

/*
 * The two halves of cab_block_sparse_attn_fwd, for callers that run several
 * executor passes over the same V (the packed tiles can be reused while V is
 * unchanged) or time the attention kernel alone. No counterpart in the
 * reference: its executor has no V preparation step.
 *
 * cab_block_sparse_attn_pack_v: writes V's packed V^T tiles (64 * D * 2 bytes
 * per (b, h, key block), zero past N) into `workspace`
 * (cab_block_sparse_attn_workspace_bytes() bytes, 16-byte aligned).
 * bf16 / fp16 only (CAB_EDTYPE for fp32, whose packed form also holds K).
 */
cab_status_t cab_block_sparse_attn_pack_v(const void* v, cab_dtype_t dtype, int64_t B, int64_t H,
                                          int64_t N, int64_t D, const int64_t v_strides[4],
                                          int32_t block_size, void* workspace,
                                          size_t workspace_bytes, void* stream);

/*
 * cab_block_sparse_attn_fwd_packed: cab_block_sparse_attn_fwd with V given
 * as the tiles cab_block_sparse_attn_pack_v wrote (`vt`, `vt_bytes` bytes).
 * Same arguments, rules and result otherwise; block_size 64 only.
 */
cab_status_t cab_block_sparse_attn_fwd_packed(const void* q, const void* k, const void* vt,
                                              cab_dtype_t dtype, int64_t B, int64_t H, int64_t N,
                                              int64_t D, const int64_t q_strides[4],
                                              const int64_t k_strides[4],
                                              const int64_t o_strides[4], int32_t block_size,
                                              const int32_t* kv_idx, const int32_t* kv_cnt,
                                              int32_t kmax, float scale, int causal, void* out,
                                              float* lse, size_t vt_bytes, void* stream);

/*
 * Dense attention with per-key attention totals, for KV-cache eviction.
 * Replaces _flash_attention_fwd_kernel / flash_attention_with_cumulative_scores
 * of cab_attention/kernels/flash_attention_accumulate.py:23-169, :172-261
 * (callers: :384-445 in the HF attention patch, read back by
 * experiments/longbench_qa/runner.py:493-538), as two calls:
 *
 * cab_flash_attn_fwd: out[t] = softmax_s(q_t . k_s * scale) v_s over every key
 * s (when causal, s <= t + N_k - N_q: the queries are the last N_q positions
 * of the key sequence); lse[t] = the natural-log log-sum-exp of the scaled
 * scores (-inf for a query that sees no key), or lse = NULL. H query heads
 * share H_kv K / V heads (query head h reads K / V head h / (H / H_kv)).
 * q, out: [B,H,N_q,D]; k, v: [B,H_kv,N_k,D] (strides); lse: contiguous fp32
 * [B,H,N_q]. D == 64 or 128; bf16, fp16 or fp32 (fp32: split bf16 MFMA as in
 * cab_block_sparse_attn_fwd). workspace: cab_flash_attn_workspace_bytes()
 * bytes, 16-byte aligned, overwritten.
 *
 * cab_attn_key_scores: score[b,h,s] (+)= sum over queries t of
 * exp(q_t . k_s * scale - lse[b,h,t]), i.e. the total softmax probability
 * key s receives from the N_q queries (same masking), with the lse rows of
 * cab_flash_attn_fwd on the same q, k. Written when accumulate == 0, added
 * to the existing values otherwise (the reference's running total across
 * calls). scores: fp32 [B,H,N_k] with strides {b, h, 1}. bf16, fp16 or fp32
 * (fp32: each product as three bf16 MFMA products of split operands, as in
 * cab_flash_attn_fwd).
 * Each key's total is summed in a fixed order (no atomics): the result is
 * deterministic. The reference's kernel adds exp(s - running maximum)
 * instead, a value that depends on its tiling; this is the quantity its
 * eager fallback sums (runner.py:680-685).
 */
size_t cab_flash_attn_workspace_bytes(cab_dtype_t dtype, int64_t B, int64_t H_kv, int64_t N_k,
                                      int64_t D);

cab_status_t cab_flash_attn_fwd(const void* q, const void* k, const void* v, cab_dtype_t dtype,
                                int64_t B, int64_t H, int64_t H_kv, int64_t N_q, int64_t N_k,
                                int64_t D, const int64_t q_strides[4], const int64_t k_strides[4],
                                const int64_t v_strides[4], const int64_t o_strides[4],
                                float scale, int causal, void* out, float* lse, void* workspace,
                                size_t workspace_bytes, void* stream);

cab_status_t cab_attn_key_scores(const void* q, const void* k, const float* lse,
                                 cab_dtype_t dtype, int64_t B, int64_t H, int64_t H_kv,
                                 int64_t N_q, int64_t N_k, int64_t D, const int64_t q_strides[4],
                                 const int64_t k_strides[4], float scale, int causal,
                                 float* scores, const int64_t score_strides[3], int accumulate,
                                 void* stream);

/*
 * KV-cache eviction: which cache positions to keep, and the pruned cache.
 *
 * cab_evict_select replaces the selection of
 * ThreeComponentEvictionPolicy.select_indices (cab_attention/eviction/policy.py:40-225)
 * and h2o_select_indices (cab_attention/eviction/h2o.py:16-94), called by
 * CABCache._evict / H2OCache._evict (cache/cab_cache.py:177-226). Over
 * cache_len positions (<= 2^20), with score[i] = importance_scores[i] for
 * i < n_scores and 0 beyond (the reference's zero padding), it keeps:
 *   1. the local window, the last local_budget positions;
 *   2. importance: the min(importance_budget, remaining) remaining positions
 *      with the highest score (a tie goes to the lower position; NaN ranks
 *      above +inf; -0 == +0) -- or, with no scores and importance_fallback,
 *      the importance_budget positions just before the local window;
 *   3. bridges, min(bridge_budget, remaining) of the remaining positions by
 *      bridge_mode: 1 nearest |score - m| with m the lower median of the
 *      remaining scores (NaN if any is NaN; ties to the lower position),
 *      2 highest bridge_scores[i] (falls back to 1, or to 3 without scores,
 *      when step 2 kept nothing), 3 the remaining positions of rank
 *      [remaining / 3, min(remaining, remaining / 3 + budget)) in position
 *      order; 0 none.
 * A kept position is never selected again. Outputs: keep_indices (int64,
 * ascending, up to cache_len entries), counts = {local, importance, bridge,
 * total} (int32) and, if not NULL, category[i] = 0 evicted, 1 local,
 * 2 importance, 3 bridge (uint8, cache_len entries). All device buffers.
 * Below 32768 positions one workgroup does the whole selection and the
 * workspace may be NULL; from 32768 on, one workgroup per 4096-position
 * segment, with the kept-set bitmap, histograms and segment counts in the
 * workspace of cab_evict_select_workspace_bytes(cache_len) bytes (256-byte
 * aligned). Both give the same positions.
 */
size_t cab_evict_select_workspace_bytes(int64_t cache_len);
cab_status_t cab_evict_select(const float* importance_scores, int64_t n_scores,
                              const float* bridge_scores, int64_t cache_len,
                              int32_t local_budget, int32_t importance_budget,
                              int32_t bridge_budget, int importance_fallback, int bridge_mode,
                              int64_t* keep_indices, int32_t* counts, uint8_t* category,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * cab_evict_select without a workspace argument: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops that forbid hipMalloc). Same arguments,
 * rules and results as cab_evict_select; the multi-workgroup path (cache_len
 * >= 32768) uses a built-in device scratch array of 206080 bytes (the
 * workspace of the largest cache, 2^20 positions), one per GPU, held until
 * the process ends; larger caches return CAB_ESHAPE. The call allocates
 * nothing. Every call on one GPU shares that GPU's scratch: calls that
 * overlap in time on one GPU (different streams or host threads without
 * ordering) race and must be serialised by the caller.
 */
cab_status_t cab_evict_select_noalloc(const float* importance_scores, int64_t n_scores,
                                      const float* bridge_scores, int64_t cache_len,
                                      int32_t local_budget, int32_t importance_budget,
                                      int32_t bridge_budget, int importance_fallback,
                                      int bridge_mode, int64_t* keep_indices, int32_t* counts,
                                      uint8_t* category, void* stream);

/*
 * Bridge scores of the policy's attention-matrix mode (policy.py:122-131):
 * with imp = {i : category[i] == 2} (cab_evict_select's output),
 * bridge_scores[j] = (sum_{i in imp} A[i, j]) * (sum_{i in imp} A[j, i]).
 * attention: fp32 [cache_len, cache_len], row stride row_stride (elements).
 * Sums run in increasing i.
 */
cab_status_t cab_evict_connectivity(const float* attention, int64_t cache_len, int64_t row_stride,
                                    const uint8_t* category, float* bridge_scores, void* stream);

/*
 * Prunes a cache: for each of n_tensors tensors (every layer's K and V),
 * dst[t][b, h, r, :] = src[t][b, h, keep_indices[r], :] for r < n_keep (rows
 * of row_bytes bytes; an index outside [0, n_src) gives a zero row).
 * Replaces the per-layer `cache[:, :, keep_indices, :]` of cab_cache.py:207-210
 * and h2o_cache.py with one launch per 32 tensors. src / dst: host arrays of
 * device pointers (16-byte aligned); strides in bytes {b, h, row}, multiples
 * of 16; keep_indices: int64 device array. dst must not overlap src.
 */
cab_status_t cab_kv_gather(const void* const* src, void* const* dst, int32_t n_tensors, int64_t B,
                           int64_t H, int64_t n_src, int64_t row_bytes,
                           const int64_t src_strides[3], const int64_t dst_strides[3],
                           const int64_t* keep_indices, int64_t n_keep, void* stream);

/*
 * Token-level Forman-Ricci curvature of a weighted directed graph A [n, n]
 * (compute_frc / compute_frc_triton / compute_frc_pytorch,
 * cab_attention/kernels/frc_triton.py:21-314):
 *   strengths[i] = S_i = sum_j A[i, j],
 *   triangles[i] = T_i = sum_j sum_k A[i, j] A[j, k] = sum_j A[i, j] S_j,
 *   frc[i]       = 4 S_i - 2 S_i + 3 T_i   (node weight taken equal to S).
 * attention: [n, n] of dtype, row stride row_stride (elements). Two passes
 * over A, fp32 accumulation in a fixed order. strengths and frc are
 * required (strengths feeds the second pass), triangles may be NULL; fp32
 * device arrays of n entries.
 */
cab_status_t cab_token_frc(const void* attention, cab_dtype_t dtype, int64_t n, int64_t row_stride,
                           float* strengths, float* triangles, float* frc, void* stream);

/*
 * The key-key matrix of FRCTracker.compute_from_attention for a 4-D input
 * (cab_attention/scoring/frc.py:110-121): with agg = mean over (b, h) of
 * attention [B, H, N_q, N_k] (element strides), out = (agg^T + agg) / 2 under
 * broadcasting, so N_q == N_k, or N_q == 1, or N_k == 1; out is fp32
 * [n, n], n = max(N_q, N_k), row stride out_stride.
 */
cab_status_t cab_attention_symmetrize(const void* attention, cab_dtype_t dtype, int64_t B,
                                      int64_t H, int64_t N_q, int64_t N_k,
                                      const int64_t strides[4], float* out, int64_t out_stride,
                                      void* stream);

/*
 * FRCTracker.compute_from_keys (cab_attention/scoring/frc.py:36-95) without
 * the [N, N] matrix: with x_n = mean over (b, h) of keys[b, h, n, :],
 * kn_n = x_n / max(|x_n|, 1e-12), r_i = sum_j relu(kn_i . kn_j) and
 * A[i, j] = relu(kn_i . kn_j) / (r_i + 1e-8), writes the token curvature of
 * A as cab_token_frc defines it: S_i = r_i / (r_i + 1e-8),
 * T_i = (sum_j relu(kn_i . kn_j) S_j) / (r_i + 1e-8). The Gram products run
 * on MFMA (bf16 hi/lo split of kn, fp32 accumulate). keys: [B, H, N, D] of
 * dtype (element strides), D <= 256. frc is required; strengths,
 * triangles and row_sums (r) may be NULL; fp32 arrays of N entries. The
 * workspace is cab_token_frc_keys_workspace_bytes(N, D) bytes.
 */
size_t cab_token_frc_keys_workspace_bytes(int64_t N, int64_t D);
cab_status_t cab_token_frc_from_keys(const void* keys, cab_dtype_t dtype, int64_t B, int64_t H,
                                     int64_t N, int64_t D, const int64_t strides[4],
                                     float* strengths, float* triangles, float* row_sums,
                                     float* frc, void* workspace, size_t workspace_bytes,
                                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CAB_HIP_H */
