// KV-cache eviction: position selection (cab_evict_select), the attention-
// matrix bridge scores (cab_evict_connectivity) and the multi-layer K/V
// gather that prunes a cache to the kept positions (cab_kv_gather).
//
// evict_select_kernel: one workgroup of 1024 threads per call. The kept set
// lives in an LDS bitmap (one bit per cache position, up to 2^20 positions).
// Each component is a k-smallest selection over the positions not yet kept:
//   local window:  the last `local` positions;
//   importance:    the highest scores (position > score: the lower position
//                  wins a tie; NaN ranks above +inf, -0 equals +0);
//   bridges:       by bridge_mode: the positions whose score is nearest the
//                  lower median of the remaining scores, the highest given
//                  bridge scores, or the middle third of the remaining
//                  positions in order.
// A selection is a 4-pass radix select over order-preserving uint32 keys
// (8 bits per pass, a 256-bin LDS histogram, coalesced reads of the scores),
// then a marking pass: every key below the threshold, and the keys equal to
// it in position order (thread-contiguous chunks and a block-wide prefix
// scan) until the count is met. The kept positions are written in ascending
// order by a last scan over the bitmap. Work: a few passes over 4 bytes per
// position, L2-resident.
//
// kv_gather_kernel: out[t] = in[keep[t]] for the rows of up to 32 tensors
// per launch (every layer's K and V), 16 bytes per thread; HBM-bound.
#include "cab_internal.h"

namespace cab {
namespace {

constexpr int SEL_THREADS = 1024;
constexpr int SEL_MAX_LEN = 1 << 20;  // cache positions (the LDS bitmap: 128 KB)

// Ascending float order as uint32: -0 == +0, NaN above +inf.
__device__ __forceinline__ uint32_t asc_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (f == 0.f) u = 0u;
  if (isnan(f)) u = 0x7fc00000u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

struct SelArgs {
  const float* scores;  // importance scores (n_scores entries), or null
  const float* bridge;  // bridge_mode 2: one score per position
  int64_t* keep;        // out: kept positions, ascending
  int32_t* counts;      // out: local, importance, bridge, total
  uint8_t* category;    // out, optional: 0 evicted, 1 local, 2 importance, 3 bridge
  int32_t n, n_scores;
  int32_t local, imp, bridge_budget;
  int32_t imp_fallback;  // no scores: keep the imp positions just before the local window
  int32_t bridge_mode;   // 0 none, 1 median, 2 given scores, 3 positional
};

struct SelShared {
  uint32_t bits[SEL_MAX_LEN / 32];
  uint32_t hist[256];
  int32_t scan[SEL_THREADS];
  int32_t misc[4];
};

// Exclusive prefix sum of v over the workgroup; *total gets the sum.
__device__ int block_scan(int v, SelShared& sh, int* total) {
  const int t = threadIdx.x;
  sh.scan[t] = v;
  __syncthreads();
  for (int off = 1; off < SEL_THREADS; off <<= 1) {
    const int x = t >= off ? sh.scan[t - off] : 0;
    __syncthreads();
    sh.scan[t] += x;
    __syncthreads();
  }
  const int incl = sh.scan[t];
  *total = sh.scan[SEL_THREADS - 1];
  __syncthreads();
  return incl - v;
}

__device__ __forceinline__ bool kept(const SelShared& sh, int i) {
  return (sh.bits[i >> 5] >> (i & 31)) & 1u;
}

// Positions in thread-contiguous chunks (for position-ordered passes).
__device__ __forceinline__ void my_chunk(int n, int* lo, int* hi) {
  const int c = (n + SEL_THREADS - 1) / SEL_THREADS;
  *lo = threadIdx.x * c < n ? threadIdx.x * c : n;
  *hi = *lo + c < n ? *lo + c : n;
}

// Keeps the `need` candidates (positions not yet kept) with the smallest
// keys; equal keys go to the lower position. 1 <= need <= #candidates.
template <class Key>
__device__ void select_smallest(int n, int need, Key key, SelShared& sh, uint8_t* category,
                                uint8_t cat) {
  uint32_t prefix = 0, mask = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (threadIdx.x < 256) sh.hist[threadIdx.x] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += SEL_THREADS) {
      if (kept(sh, i)) continue;
      const uint32_t k = key(i);
      if ((k & mask) == prefix) atomicAdd(&sh.hist[(k >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int run = 0, bin = 0;
      for (; bin < 255; ++bin) {
        if (run + static_cast<int>(sh.hist[bin]) >= need) break;
        run += static_cast<int>(sh.hist[bin]);
      }
      sh.misc[0] = bin;
      sh.misc[1] = run;
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(sh.misc[0]) << shift;
    mask |= 255u << shift;
    need -= sh.misc[1];
    __syncthreads();
  }
  // need = how many keys equal to the threshold complete the selection.
  int lo, hi;
  my_chunk(n, &lo, &hi);
  int eq = 0;
  for (int i = lo; i < hi; ++i)
    if (!kept(sh, i) && key(i) == prefix) ++eq;
  int total;
  int take = need - block_scan(eq, sh, &total);
  // Every thread has counted before any bit of this selection is set.
  for (int i = lo; i < hi; ++i) {
    if (kept(sh, i)) continue;
    const uint32_t k = key(i);
    bool sel = k < prefix;
    if (!sel && k == prefix && take > 0) {
      sel = true;
      --take;
    }
    if (sel) {
      atomicOr(&sh.bits[i >> 5], 1u << (i & 31));
      if (category) category[i] = cat;
    }
  }
  __syncthreads();
}

// Keeps the not-yet-kept positions of rank [first, first + count) among them,
// in position order.
__device__ void select_ranks(int n, int first, int count, SelShared& sh, uint8_t* category,
                             uint8_t cat) {
  int lo, hi;
  my_chunk(n, &lo, &hi);
  int c = 0;
  for (int i = lo; i < hi; ++i) c += kept(sh, i) ? 0 : 1;
  int total;
  int r = block_scan(c, sh, &total);
  for (int i = lo; i < hi; ++i) {
    if (kept(sh, i)) continue;
    if (r >= first && r < first + count) {
      atomicOr(&sh.bits[i >> 5], 1u << (i & 31));
      if (category) category[i] = cat;
    }
    ++r;
  }
  __syncthreads();
}

__global__ __launch_bounds__(SEL_THREADS) void evict_select_kernel(SelArgs a) {
  __shared__ SelShared sh;
  const int n = a.n, tid = threadIdx.x;
  const int words = (n + 31) >> 5;
  const int l0 = n - a.local;  // first local position
  for (int w = tid; w < words; w += SEL_THREADS) {
    // local window bits, positions >= l0 (and < n)
    uint32_t m = 0u;
    const int b0 = w * 32;
    if (b0 + 32 <= l0) {
      m = 0u;
    } else {
      for (int j = 0; j < 32; ++j)
        if (b0 + j >= l0 && b0 + j < n) m |= 1u << j;
    }
    sh.bits[w] = m;
  }
  if (a.category)
    for (int i = l0 + tid; i < n; i += SEL_THREADS) a.category[i] = 1;
  __syncthreads();
  auto score = [&](int i) -> float { return i < a.n_scores ? a.scores[i] : 0.f; };
  const int free0 = n - a.local;  // positions not in the local window

  // importance
  int n_imp = 0;
  if (a.scores) {
    n_imp = a.imp < free0 ? a.imp : free0;
    if (n_imp > 0)
      select_smallest(n, n_imp, [&](int i) { return ~asc_key(score(i)); }, sh, a.category, 2);
  } else if (a.imp_fallback && a.imp > 0) {
    const int s0 = n - a.local - a.imp > 0 ? n - a.local - a.imp : 0;
    n_imp = l0 - s0;
    for (int i = s0 + tid; i < l0; i += SEL_THREADS) {
      atomicOr(&sh.bits[i >> 5], 1u << (i & 31));
      if (a.category) a.category[i] = 2;
    }
    __syncthreads();
  }

  // bridges
  const int free1 = free0 - n_imp;
  int mode = a.bridge_mode;
  if (mode == 2 && n_imp == 0) mode = a.scores ? 1 : 3;
  if (mode == 1 && !a.scores) mode = 3;
  int n_br = 0;
  if (a.bridge_budget > 0 && free1 > 0 && mode != 0) {
    n_br = a.bridge_budget < free1 ? a.bridge_budget : free1;
    if (mode == 1) {
      // lower median of the remaining scores (NaN if any of them is NaN)
      if (tid == 0) sh.misc[2] = 0;
      __syncthreads();
      for (int i = tid; i < n; i += SEL_THREADS)
        if (!kept(sh, i) && isnan(score(i))) sh.misc[2] = 1;
      __syncthreads();
      const bool has_nan = sh.misc[2] != 0;
      __syncthreads();
      float med = __uint_as_float(0x7fc00000u);
      if (!has_nan) {
        // the ((free1 - 1) / 2 + 1)-th smallest remaining score: a radix
        // select that marks nothing (its result is read back below)
        uint32_t prefix = 0, mask = 0;
        int need = (free1 - 1) / 2 + 1;
        for (int shift = 24; shift >= 0; shift -= 8) {
          if (tid < 256) sh.hist[tid] = 0u;
          __syncthreads();
          for (int i = tid; i < n; i += SEL_THREADS) {
            if (kept(sh, i)) continue;
            const uint32_t k = asc_key(score(i));
            if ((k & mask) == prefix) atomicAdd(&sh.hist[(k >> shift) & 255u], 1u);
          }
          __syncthreads();
          if (tid == 0) {
            int run = 0, bin = 0;
            for (; bin < 255; ++bin) {
              if (run + static_cast<int>(sh.hist[bin]) >= need) break;
              run += static_cast<int>(sh.hist[bin]);
            }
            sh.misc[0] = bin;
            sh.misc[1] = run;
          }
          __syncthreads();
          prefix |= static_cast<uint32_t>(sh.misc[0]) << shift;
          mask |= 255u << shift;
          need -= sh.misc[1];
          __syncthreads();
        }
        med = key_float(prefix);
      }
      select_smallest(n, n_br, [&](int i) { return asc_key(fabsf(score(i) - med)); }, sh,
                      a.category, 3);
    } else if (mode == 2) {
      select_smallest(n, n_br, [&](int i) { return ~asc_key(a.bridge[i]); }, sh, a.category, 3);
    } else {
      // remaining[free1 / 3 : free1 / 3 + budget], cut at the end
      if (n_br > free1 - free1 / 3) n_br = free1 - free1 / 3;
      select_ranks(n, free1 / 3, n_br, sh, a.category, 3);
    }
  }

  // kept positions, ascending
  int lo, hi;
  my_chunk(n, &lo, &hi);
  int c = 0;
  for (int i = lo; i < hi; ++i) c += kept(sh, i) ? 1 : 0;
  int total;
  int pos = block_scan(c, sh, &total);
  for (int i = lo; i < hi; ++i) {
    if (kept(sh, i))
      a.keep[pos++] = i;
    else if (a.category)
      a.category[i] = 0;
  }
  if (tid == 0) {
    a.counts[0] = a.local;
    a.counts[1] = n_imp;
    a.counts[2] = n_br;
    a.counts[3] = total;
  }
}

// Bridge scores from an attention matrix A [n, n] (row stride `ld`) and the
// importance positions (category == 2): from[j] = sum_{i imp} A[i, j],
// to[j] = sum_{i imp} A[j, i], score[j] = from[j] to[j]. Fixed summation order.
__global__ __launch_bounds__(256) void connectivity_kernel(const float* A, int64_t ld, int n,
                                                           const uint8_t* category, float* out) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= n) return;
  float from = 0.f, to = 0.f;
  const float* row_j = A + static_cast<int64_t>(j) * ld;
  for (int i = 0; i < n; ++i) {
    if (category[i] != 2) continue;
    from += A[static_cast<int64_t>(i) * ld + j];
    to += row_j[i];
  }
  out[j] = from * to;
}

constexpr int GATHER_MAX = 32;  // tensors per launch

struct GatherArgs {
  const char* src[GATHER_MAX];
  char* dst[GATHER_MAX];
  const int64_t* idx;
  int64_t ss[3], ds[3];  // byte strides (b, h, token)
  int64_t H, n_src, n_keep, chunks;  // chunks: 16-byte pieces per row
  int64_t units;                     // B * H * n_keep * chunks
};

__global__ __launch_bounds__(256) void kv_gather_kernel(GatherArgs a) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (u >= a.units) return;
  const int tns = blockIdx.y;
  const int64_t c = u % a.chunks;
  const int64_t row = u / a.chunks;  // (b, h, t)
  const int64_t t = row % a.n_keep;
  const int64_t bh = row / a.n_keep;
  const int64_t b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int64_t s = a.idx[t];
  u32x4 x = {0u, 0u, 0u, 0u};
  if (s >= 0 && s < a.n_src)
    x = *reinterpret_cast<const u32x4*>(a.src[tns] + b * a.ss[0] + h * a.ss[1] + s * a.ss[2] +
                                        16 * c);
  *reinterpret_cast<u32x4*>(a.dst[tns] + b * a.ds[0] + h * a.ds[1] + t * a.ds[2] + 16 * c) = x;
}

}  // namespace
}  // namespace cab

using namespace cab;

extern "C" cab_status_t cab_evict_select(const float* importance_scores, int64_t n_scores,
                                         const float* bridge_scores, int64_t cache_len,
                                         int32_t local_budget, int32_t importance_budget,
                                         int32_t bridge_budget, int importance_fallback,
                                         int bridge_mode, int64_t* keep_indices, int32_t* counts,
                                         uint8_t* category, void* stream) {
  const char* fn = "cab_evict_select";
  clear_error();
  CAB_REQUIRE(cache_len >= 0 && cache_len <= SEL_MAX_LEN, CAB_ESHAPE,
              "%s: cache_len %lld outside [0, 2^20]", fn, (long long)cache_len);
  CAB_REQUIRE(local_budget >= 0 && local_budget <= cache_len && importance_budget >= 0 &&
                  bridge_budget >= 0,
              CAB_EINVAL, "%s: budgets must be >= 0 and local <= cache_len", fn);
  CAB_REQUIRE(bridge_mode >= 0 && bridge_mode <= 3, CAB_EINVAL, "%s: bridge_mode %d unknown", fn,
              bridge_mode);
  CAB_REQUIRE(n_scores >= 0 && n_scores <= INT32_MAX, CAB_ESHAPE, "%s: bad n_scores", fn);
  CAB_REQUIRE(importance_scores != nullptr || n_scores == 0, CAB_EINVAL,
              "%s: n_scores > 0 with null scores", fn);
  CAB_REQUIRE(bridge_mode != 2 || bridge_scores != nullptr, CAB_EINVAL,
              "%s: bridge_mode 2 needs bridge scores", fn);
  CAB_REQUIRE(keep_indices != nullptr && counts != nullptr, CAB_EINVAL, "%s: null output", fn);
  SelArgs a;
  a.scores = importance_scores;
  a.bridge = bridge_scores;
  a.keep = keep_indices;
  a.counts = counts;
  a.category = category;
  a.n = static_cast<int32_t>(cache_len);
  a.n_scores = static_cast<int32_t>(n_scores < cache_len ? n_scores : cache_len);
  a.local = local_budget;
  a.imp = importance_budget;
  a.bridge_budget = bridge_budget;
  a.imp_fallback = importance_fallback ? 1 : 0;
  a.bridge_mode = bridge_mode;
  evict_select_kernel<<<1, SEL_THREADS, 0, static_cast<hipStream_t>(stream)>>>(a);
  return launch_status(fn);
}

extern "C" cab_status_t cab_evict_connectivity(const float* attention, int64_t cache_len,
                                               int64_t row_stride, const uint8_t* category,
                                               float* bridge_scores, void* stream) {
  const char* fn = "cab_evict_connectivity";
  clear_error();
  CAB_REQUIRE(cache_len >= 0 && cache_len <= SEL_MAX_LEN, CAB_ESHAPE,
              "%s: cache_len %lld outside [0, 2^20]", fn, (long long)cache_len);
  if (cache_len == 0) return CAB_OK;
  CAB_REQUIRE(attention && category && bridge_scores, CAB_EINVAL, "%s: null pointer", fn);
  CAB_REQUIRE(row_stride >= cache_len, CAB_ESHAPE, "%s: row stride below cache_len", fn);
  connectivity_kernel<<<static_cast<unsigned>(ceil_div(cache_len, 256)), 256, 0,
                        static_cast<hipStream_t>(stream)>>>(attention, row_stride,
                                                            static_cast<int>(cache_len), category,
                                                            bridge_scores);
  return launch_status(fn);
}

extern "C" cab_status_t cab_kv_gather(const void* const* src, void* const* dst, int32_t n_tensors,
                                      int64_t B, int64_t H, int64_t n_src, int64_t row_bytes,
                                      const int64_t src_strides[3], const int64_t dst_strides[3],
                                      const int64_t* keep_indices, int64_t n_keep, void* stream) {
  const char* fn = "cab_kv_gather";
  clear_error();
  CAB_REQUIRE(n_tensors >= 0 && B >= 0 && H >= 0 && n_src >= 0 && n_keep >= 0, CAB_ESHAPE,
              "%s: negative size", fn);
  CAB_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0, CAB_ESHAPE,
              "%s: row_bytes %lld must be a positive multiple of 16", fn, (long long)row_bytes);
  if (n_tensors == 0 || B == 0 || H == 0 || n_keep == 0) return CAB_OK;
  CAB_REQUIRE(src && dst && src_strides && dst_strides && keep_indices, CAB_EINVAL,
              "%s: null argument", fn);
  for (int d = 0; d < 3; ++d)
    CAB_REQUIRE(src_strides[d] >= 0 && src_strides[d] % 16 == 0 && dst_strides[d] >= 0 &&
                    dst_strides[d] % 16 == 0,
                CAB_ESHAPE, "%s: byte strides must be >= 0 and multiples of 16", fn);
  for (int t = 0; t < n_tensors; ++t)
    CAB_REQUIRE(src[t] && dst[t] && reinterpret_cast<uintptr_t>(src[t]) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(dst[t]) % 16 == 0,
                CAB_EINVAL, "%s: tensor %d null or not 16-byte aligned", fn, t);
  const int64_t chunks = row_bytes / 16;
  const int64_t units = B * H * n_keep * chunks;
  CAB_REQUIRE(ceil_div(units, 256) <= INT32_MAX, CAB_ESHAPE, "%s: too large", fn);
  GatherArgs a;
  a.idx = keep_indices;
  for (int d = 0; d < 3; ++d) {
    a.ss[d] = src_strides[d];
    a.ds[d] = dst_strides[d];
  }
  a.H = H;
  a.n_src = n_src;
  a.n_keep = n_keep;
  a.chunks = chunks;
  a.units = units;
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int t0 = 0; t0 < n_tensors; t0 += GATHER_MAX) {
    const int nt = n_tensors - t0 < GATHER_MAX ? n_tensors - t0 : GATHER_MAX;
    for (int t = 0; t < nt; ++t) {
      a.src[t] = static_cast<const char*>(src[t0 + t]);
      a.dst[t] = static_cast<char*>(dst[t0 + t]);
    }
    kv_gather_kernel<<<dim3(static_cast<unsigned>(ceil_div(units, 256)), nt), 256, 0, s>>>(a);
    cab_status_t st = launch_status(fn);
    if (st != CAB_OK) return st;
  }
  return CAB_OK;
}
