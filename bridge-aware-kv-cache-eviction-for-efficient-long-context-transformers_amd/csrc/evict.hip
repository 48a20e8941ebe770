// KV-cache eviction: position selection (cab_evict_select), the attention-
// matrix bridge scores (cab_evict_connectivity) and the multi-layer K/V
// gather that prunes a cache to the kept positions (cab_kv_gather).
//
// evict_select_kernel (caches below MULTI_MIN positions): one workgroup of
// 1024 threads (16 waves) per call. The kept set lives in an LDS bitmap (one
// bit per cache position). Larger caches (up to 2^20 positions) run the
// msel_* kernels further down: the same selection, one workgroup per
// 4096-position segment, with the bitmap and the radix histograms in a
// workspace. Each component is a k-smallest selection over the positions
// not yet kept:
//   local window:  the last `local` positions;
//   importance:    the highest scores (position > score: the lower position
//                  wins a tie; NaN ranks above +inf, -0 equals +0);
//   bridges:       by bridge_mode: the positions whose score is nearest the
//                  lower median of the remaining scores, the highest given
//                  bridge scores, or the middle third of the remaining
//                  positions in order.
// Every pass over the positions gives wave w the contiguous segment
// [w * seg, (w + 1) * seg) (seg a multiple of 256) and walks it 256
// positions per step, lane l on positions 4l..4l+3 (one 16-byte load, four
// steps in flight). Ranks in position order come from ballots: a lane's
// offset is the mbcnt of the ballots of its count's bits, a wave's offset
// the sum of the earlier waves' totals.
// A selection is a radix select over order-preserving uint32 keys in three
// passes of 11, 11 and 10 bits (a 2048-bin LDS histogram; the lanes of a
// wave that share a bin add once), then a marking pass: every key below the
// threshold, and the keys equal to it in position order until the count is
// met (one more pass only when some but not all of them are taken). The
// kept positions are written in ascending order from the bitmap. Work: four
// to five passes over 4 bytes per position and selection, L2-resident.
//
// kv_gather_kernel: out[t] = in[keep[t]] for the rows of up to 32 tensors
// per launch (every layer's K and V), 16 bytes per thread; HBM-bound.
#include <mutex>

#include "cab_internal.h"

namespace cab {
namespace {

constexpr int SEL_THREADS = 1024;
constexpr int SEL_WAVES = SEL_THREADS / 64;
constexpr int SEL_MAX_LEN = 1 << 20;  // cache positions (the LDS bitmap: 128 KB)
constexpr int SEL_BINS = 2048;        // radix histogram (11 bits)
constexpr uint32_t NAN_KEY = 0xffc00000u;

// Ascending float order as uint32: -0 == +0, NaN (any) above +inf.
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
  uint32_t hist[SEL_BINS];
  int32_t wave_tot[SEL_WAVES];
  int32_t misc[4];
};

// Keys of the positions: KEY_DESC ~asc(x) (highest first), KEY_DIST
// asc(|x - med|), KEY_ASC asc(x), KEY_NONE no scores read (positional).
enum { KEY_DESC = 0, KEY_DIST = 1, KEY_ASC = 2, KEY_NONE = 3 };

struct KeySrc {
  const float* p;  // scores; positions >= n_valid read as 0
  int n_valid;
  float med;
};

template <int KIND>
__device__ __forceinline__ uint32_t key_of(float x, float med) {
  if (KIND == KEY_DESC) return ~asc_key(x);
  if (KIND == KEY_DIST) return asc_key(fabsf(x - med));
  return asc_key(x);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Set bits of m in the lanes below this one.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
}

// Sum of v (0 <= v < 2^BITS) over the lanes below this one, and over the wave.
template <int BITS>
__device__ __forceinline__ void lane_offsets(int v, int* below, int* total) {
  int b = 0, t = 0;
#pragma unroll
  for (int i = 0; i < BITS; ++i) {
    const uint64_t m = __ballot((v >> i) & 1);
    b += lanes_below(m) << i;
    t += __popcll(m) << i;
  }
  *below = b;
  *total = t;
}

// hist[bin] += 1 for the active lanes; lanes sharing the wave's commonest
// bins add once (same-address LDS atomics serialise).
__device__ __forceinline__ void hist_add(uint32_t* hist, bool act, uint32_t bin) {
  uint64_t todo = __ballot(act);
  for (int it = 0; it < 2 && todo; ++it) {
    const int leader = __builtin_ctzll(todo);
    const uint32_t lb = __builtin_amdgcn_readlane(bin, leader);
    const uint64_t peers = __ballot(act && bin == lb) & todo;
    if (lane_id() == leader) atomicAdd(&hist[lb], static_cast<uint32_t>(__popcll(peers)));
    todo &= ~peers;
  }
  if ((todo >> lane_id()) & 1ull) atomicAdd(&hist[bin], 1u);
}

// This wave's segment of [0, n), in positions (multiples of 256).
__device__ __forceinline__ void wave_segment(int n, int* beg, int* end) {
  const int seg = ((n + SEL_WAVES - 1) / SEL_WAVES + 255) & ~255;
  const int w = threadIdx.x >> 6;
  *beg = w * seg < n ? w * seg : n;
  *end = *beg + seg < n ? *beg + seg : n;
}

// Exclusive prefix of the waves' totals for this wave, and the grand total.
__device__ __forceinline__ int wave_start(SelShared& sh, int mine, int* total) {
  if (lane_id() == 0) sh.wave_tot[threadIdx.x >> 6] = mine;
  __syncthreads();
  int s = 0, t = 0;
  for (int w = 0; w < SEL_WAVES; ++w) {
    const int v = sh.wave_tot[w];
    if (w < static_cast<int>(threadIdx.x >> 6)) s += v;
    t += v;
  }
  __syncthreads();
  *total = t;
  return s;
}

__device__ __forceinline__ float4 load4(const KeySrc s, int p, int end) {
  if (p + 3 < s.n_valid && (reinterpret_cast<uintptr_t>(s.p) & 15u) == 0)
    return *reinterpret_cast<const float4*>(s.p + p);
  float x[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = (p + e < end && p + e < s.n_valid) ? s.p[p + e] : 0.f;
  return make_float4(x[0], x[1], x[2], x[3]);
}

// Walks this wave's segment in position order, 256 positions per step with
// the next four steps' loads in flight: f(p, cand, key) per step, called by
// every lane of the wave (ballots inside are wave-wide). cand bit e =
// position p + e exists and is not kept. The loop stays rolled: one
// workgroup runs this code, so its size matters more than loop overhead.
template <int KIND, class F>
__device__ __forceinline__ void walk(int n, const SelShared& sh, const KeySrc s, F f) {
  int beg, end;
  wave_segment(n, &beg, &end);
  const int lane4 = 4 * lane_id();
  const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 x1 = zero, x2 = zero, x3 = zero, x4 = zero;
  if (KIND != KEY_NONE) {
    if (beg + lane4 < end) x1 = load4(s, beg + lane4, end);
    if (beg + 256 + lane4 < end) x2 = load4(s, beg + 256 + lane4, end);
    if (beg + 512 + lane4 < end) x3 = load4(s, beg + 512 + lane4, end);
    if (beg + 768 + lane4 < end) x4 = load4(s, beg + 768 + lane4, end);
  }
#pragma unroll 1
  for (int base = beg; base < end; base += 256) {
    const int p = base + lane4;
    const float4 x = x1;
    x1 = x2;
    x2 = x3;
    x3 = x4;
    if (KIND != KEY_NONE && p + 1024 < end) x4 = load4(s, p + 1024, end);
    uint32_t cand = 0u;
    if (p < end) {
      cand = ~(sh.bits[p >> 5] >> (p & 31)) & 0xfu;
      if (end - p < 4) cand &= (1u << (end - p)) - 1u;
    }
    u32x4 k = {0u, 0u, 0u, 0u};
    if (KIND != KEY_NONE) {
      k[0] = key_of<KIND>(x.x, s.med);
      k[1] = key_of<KIND>(x.y, s.med);
      k[2] = key_of<KIND>(x.z, s.med);
      k[3] = key_of<KIND>(x.w, s.med);
    }
    f(p, cand, k);
  }
}

__device__ __forceinline__ void mark(SelShared& sh, int p, uint32_t m, uint8_t* category,
                                     uint8_t cat) {
  if (!m) return;
  atomicOr(&sh.bits[p >> 5], m << (p & 31));
  if (category)
    for (int e = 0; e < 4; ++e)
      if ((m >> e) & 1u) category[p + e] = cat;
}

// Inclusive prefix sum of v over the lanes of the wave.
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = lane_id();
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(v, off);
    if (lane >= off) v += y;
  }
  return v;
}

struct Threshold {
  uint32_t key;  // the need-th smallest candidate key
  int need_eq;   // how many candidates with this key complete the selection
  int eq;        // candidates with this key
  int nan;       // candidates with a NaN score (KEY_ASC only)
};

// Radix select of the need-th smallest candidate key, 1 <= need <= #candidates.
template <int KIND>
__device__ __forceinline__ Threshold radix_select(int n, int need, const KeySrc s, SelShared& sh) {
  uint32_t prefix = 0u, mask = 0u;
  Threshold th = {0u, 0, 0, 0};
  if (threadIdx.x == 0) sh.misc[3] = 0;
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : pass == 1 ? 10 : 0;  // bits 31..21, 20..10, 9..0
    const int nb = pass == 2 ? 1024 : 2048;
    for (int b = threadIdx.x; b < nb; b += SEL_THREADS) sh.hist[b] = 0u;
    __syncthreads();
    walk<KIND>(n, sh, s, [&](int, uint32_t cand, u32x4 k) {
      int nan = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool act = ((cand >> e) & 1u) && (k[e] & mask) == prefix;
        hist_add(sh.hist, act, (k[e] >> shift) & static_cast<uint32_t>(nb - 1));
        if (KIND == KEY_ASC && pass == 0) nan += (act && k[e] == NAN_KEY) ? 1 : 0;
      }
      if (KIND == KEY_ASC && pass == 0 && nan) atomicAdd(&sh.misc[3], nan);
    });
    __syncthreads();
    if (threadIdx.x < 64) {
      // wave 0: lane l sums bins [l * per, (l + 1) * per); the first lane
      // whose inclusive sum reaches need owns the threshold bin, which a
      // second scan over the owner's bins (one per lane) finds
      const int per = nb / 64, lane = threadIdx.x;
      int sum = 0;
      for (int b = 0; b < per; ++b) sum += static_cast<int>(sh.hist[lane * per + b]);
      const int incl = wave_incl_scan(sum);
      const uint64_t hit = __ballot(incl >= need);
      const int owner = hit ? __builtin_ctzll(hit) : 63;
      const int run0 = __builtin_amdgcn_readlane(incl - sum, owner);
      const int h = lane < per ? static_cast<int>(sh.hist[owner * per + lane]) : 0;
      const int incl2 = run0 + wave_incl_scan(h);
      const uint64_t hit2 = __ballot(lane < per && incl2 >= need);
      const int j = hit2 ? __builtin_ctzll(hit2) : per - 1;
      if (lane == j) {
        sh.misc[0] = owner * per + j;
        sh.misc[1] = incl2 - h;
        sh.misc[2] = h;
      }
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(sh.misc[0]) << shift;
    mask |= static_cast<uint32_t>(nb - 1) << shift;
    need -= sh.misc[1];
    th.eq = sh.misc[2];
    th.nan = sh.misc[3];
    __syncthreads();
  }
  th.key = prefix;
  th.need_eq = need;
  return th;
}

// Sum of v over the wave (every lane gets it).
__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Marks, in position order, the candidates with q set (the 4-bit masks a
// walk produces) whose rank among them lies in [first, first + count);
// `start` is the number of such candidates in the earlier waves' segments.
template <int KIND, class Q>
__device__ __forceinline__ void mark_ranked(int n, const KeySrc s, SelShared& sh, int start, int first, int count,
                            Q q_of, uint8_t* category, uint8_t cat) {
  int carry = start;
  walk<KIND>(n, sh, s, [&](int p, uint32_t cand, u32x4 k) {
    const uint32_t q = q_of(cand, k);
    int below, tot;
    lane_offsets<3>(__popc(q), &below, &tot);
    if (carry < first + count && carry + tot > first) {
      uint32_t m = 0u;
      int r = carry + below;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (!((q >> e) & 1u)) continue;
        if (r >= first && r < first + count) m |= 1u << e;
        ++r;
      }
      mark(sh, p, m, category, cat);
    }
    carry += tot;
  });
  __syncthreads();
}

// Keeps the `need` candidates with the smallest keys; equal keys go to the
// lower position. 1 <= need <= #candidates.
template <int KIND>
__device__ __forceinline__ void select_smallest(int n, int need, const KeySrc s, SelShared& sh,
                                uint8_t* category, uint8_t cat) {
  const Threshold th = radix_select<KIND>(n, need, s, sh);
  const bool all_eq = th.need_eq == th.eq;
  int eq_mine = 0;
  walk<KIND>(n, sh, s, [&](int p, uint32_t cand, u32x4 k) {
    uint32_t m = 0u, q = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (!((cand >> e) & 1u)) continue;
      if (k[e] < th.key) m |= 1u << e;
      if (k[e] == th.key) q |= 1u << e;
    }
    if (all_eq)
      m |= q;
    else
      eq_mine += __popc(q);
    mark(sh, p, m, category, cat);
  });
  if (all_eq) {
    __syncthreads();
    return;
  }
  // Ties: the first need_eq equal keys in position order. The walk above
  // marked only keys below the threshold, so the equal keys are still
  // candidates.
  int total;
  const int start = wave_start(sh, wave_sum(eq_mine), &total);
  const uint32_t key = th.key;
  mark_ranked<KIND>(n, s, sh, start, 0, th.need_eq, [key](uint32_t cand, u32x4 k) {
    uint32_t q = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (((cand >> e) & 1u) && k[e] == key) q |= 1u << e;
    return q;
  }, category, cat);
}

// Keeps the candidates of rank [first, first + count) among them, in
// position order.
__device__ __forceinline__ void select_ranks(int n, int first, int count, SelShared& sh, uint8_t* category,
                             uint8_t cat) {
  const KeySrc none = {nullptr, 0, 0.f};
  int mine = 0;
  walk<KEY_NONE>(n, sh, none, [&](int, uint32_t cand, u32x4) { mine += __popc(cand); });
  int total;
  const int start = wave_start(sh, wave_sum(mine), &total);
  mark_ranked<KEY_NONE>(n, none, sh, start, first, count,
                        [](uint32_t cand, u32x4) { return cand; }, category, cat);
}

__global__ __launch_bounds__(SEL_THREADS) void evict_select_kernel(SelArgs a) {
  __shared__ SelShared sh;
  const int n = a.n, tid = threadIdx.x;
  const int words = (n + 31) >> 5;
  const int l0 = n - a.local;  // first local position
  for (int w = tid; w < words; w += SEL_THREADS) {
    // local window bits: positions in [l0, n)
    const int b0 = w * 32;
    uint32_t m = 0u;
    if (b0 + 32 > l0)
      for (int j = 0; j < 32; ++j)
        if (b0 + j >= l0 && b0 + j < n) m |= 1u << j;
    sh.bits[w] = m;
  }
  if (a.category)
    for (int i = l0 + tid; i < n; i += SEL_THREADS) a.category[i] = 1;
  __syncthreads();
  const KeySrc imp_src = {a.scores, a.n_scores, 0.f};
  const int free0 = n - a.local;  // positions not in the local window

  // importance
  int n_imp = 0;
  if (a.scores) {
    n_imp = a.imp < free0 ? a.imp : free0;
    if (n_imp > 0) select_smallest<KEY_DESC>(n, n_imp, imp_src, sh, a.category, 2);
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
      // lower median of the remaining scores (NaN if any of them is NaN):
      // the ((free1 - 1) / 2 + 1)-th smallest
      const Threshold th = radix_select<KEY_ASC>(n, (free1 - 1) / 2 + 1, imp_src, sh);
      const float med = th.nan ? __uint_as_float(0x7fc00000u) : key_float(th.key);
      const KeySrc dist = {a.scores, a.n_scores, med};
      select_smallest<KEY_DIST>(n, n_br, dist, sh, a.category, 3);
    } else if (mode == 2) {
      const KeySrc given = {a.bridge, n, 0.f};
      select_smallest<KEY_DESC>(n, n_br, given, sh, a.category, 3);
    } else {
      // remaining[free1 / 3 : free1 / 3 + budget], cut at the end
      if (n_br > free1 - free1 / 3) n_br = free1 - free1 / 3;
      select_ranks(n, free1 / 3, n_br, sh, a.category, 3);
    }
  }

  // kept positions, ascending: wave segments of whole words, one word per
  // lane and step, ranks from the ballots of the popcounts' bits
  const int wseg = ((words + SEL_WAVES - 1) / SEL_WAVES + 63) & ~63;
  const int wb = (tid >> 6) * wseg < words ? (tid >> 6) * wseg : words;
  const int we = wb + wseg < words ? wb + wseg : words;
  const int lane = lane_id();
  int mine = 0;
  for (int w0 = wb; w0 < we; w0 += 64) {
    const int w = w0 + lane;
    mine += w < we ? __popc(sh.bits[w]) : 0;
  }
  int total;
  int pos = wave_start(sh, wave_sum(mine), &total);
  for (int w0 = wb; w0 < we; w0 += 64) {
    const int w = w0 + lane;
    const uint32_t bits = w < we ? sh.bits[w] : 0u;
    int below, tot;
    lane_offsets<6>(__popc(bits), &below, &tot);
    int64_t* out = a.keep + pos + below;
    for (uint32_t m = bits; m; m &= m - 1) *out++ = w * 32 + __builtin_ctz(m);
    if (a.category && w < we) {
      const int hi = w * 32 + 32 < n ? w * 32 + 32 : n;
      for (int i = w * 32; i < hi; ++i)
        if (!((bits >> (i & 31)) & 1u)) a.category[i] = 0;
    }
    pos += tot;
  }
  if (tid == 0) {
    a.counts[0] = a.local;
    a.counts[1] = n_imp;
    a.counts[2] = n_br;
    a.counts[3] = total;
  }
}

// ---------------------------------------------------------------------------
// Multi-workgroup selection (caches of MULTI_MIN positions and more). The
// same selection as evict_select_kernel, spread over one workgroup per
// MSEG-position segment: the kept set is a bitmap in the workspace (each
// workgroup owns its segment's words), each radix pass adds its segment's
// LDS histogram into a global histogram row, and every workgroup re-derives
// the threshold from the rows of the earlier passes. Ranks in position order
// come from per-segment counts (a prefix over the earlier segments) and,
// inside a segment, the per-wave ballot ranks of the single-workgroup path.
// ---------------------------------------------------------------------------
constexpr int MSEG = 4096;           // positions per workgroup (4 waves x 1024)
constexpr int MTHREADS = 256;
constexpr int MULTI_MIN = 1 << 15;   // cache_len from which the multi-workgroup path runs
constexpr int MHIST_ROWS = 9;        // importance 0..2, median 3..5, bridges 6..8

struct MArgs {
  const float* scores;
  const float* bridge;
  int64_t* keep;
  int32_t* counts;
  uint8_t* category;
  uint32_t* bits;    // ceil(n / 32) words
  uint32_t* hist;    // [MHIST_ROWS][SEL_BINS]
  int32_t* segcnt;   // [G]
  int32_t* state;    // [0]: NaN scores among the median's candidates
  int32_t n, n_scores, G;
  int32_t local, n_imp, n_br, imp_fallback_lo;  // imp_fallback_lo: first fallback position, or n
};

struct MStep {
  KeySrc src;
  int32_t hbase, pass, need;
  int32_t med_hbase, med_need;  // KEY_DIST: the median's rows and rank
  int32_t first, count;         // positional ranks
  uint8_t cat;
};

struct Resolved {
  uint32_t prefix;
  int need;  // how many keys equal to prefix complete the selection (after 3 passes)
  int eq;    // keys equal to prefix (after 3 passes)
};

// The threshold after npass recorded passes of the radix select for rank
// need (histogram rows h0 ..); every thread of the workgroup gets it.
__device__ Resolved resolve(const uint32_t* hist, int h0, int npass, int need, int* sm) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    uint32_t prefix = 0u;
    int rem = need, eq = 0;
    for (int p = 0; p < npass; ++p) {
      const int shift = p == 0 ? 21 : p == 1 ? 10 : 0;
      const int nb = p == 2 ? 1024 : 2048;
      const uint32_t* h = hist + static_cast<int64_t>(h0 + p) * SEL_BINS;
      const int per = nb / 64;
      int sum = 0;
      for (int b = 0; b < per; ++b) sum += static_cast<int>(h[lane * per + b]);
      const int incl = wave_incl_scan(sum);
      const uint64_t hit = __ballot(incl >= rem);
      const int owner = hit ? __builtin_ctzll(hit) : 63;
      const int run0 = __builtin_amdgcn_readlane(incl - sum, owner);
      const int hv = lane < per ? static_cast<int>(h[owner * per + lane]) : 0;
      const int incl2 = run0 + wave_incl_scan(hv);
      const uint64_t hit2 = __ballot(lane < per && incl2 >= rem);
      const int j = hit2 ? __builtin_ctzll(hit2) : per - 1;
      const int below = __builtin_amdgcn_readlane(incl2 - hv, j);
      eq = __builtin_amdgcn_readlane(hv, j);
      prefix |= static_cast<uint32_t>(owner * per + j) << shift;
      rem -= below;
    }
    if (lane == 0) {
      sm[0] = static_cast<int>(prefix);
      sm[1] = rem;
      sm[2] = eq;
    }
  }
  __syncthreads();
  Resolved r{static_cast<uint32_t>(sm[0]), sm[1], sm[2]};
  __syncthreads();
  return r;
}

__device__ __forceinline__ uint32_t prefix_mask(int npass) {
  return npass == 0 ? 0u : npass == 1 ? 0xffe00000u : npass == 2 ? 0xfffffc00u : 0xffffffffu;
}

// This wave's positions of the workgroup's segment: [beg, end).
__device__ __forceinline__ void mseg_wave(int n, int* beg, int* end) {
  const int s0 = blockIdx.x * MSEG + (threadIdx.x >> 6) * (MSEG / 4);
  *beg = s0 < n ? s0 : n;
  *end = s0 + MSEG / 4 < n ? s0 + MSEG / 4 : n;
}

// Walks this wave's quarter of the segment in position order (256 positions
// per step, lane l on 4l .. 4l + 3): f(p, cand, key), called by every lane.
// sbits: the segment's bitmap words in LDS.
template <int KIND, class F>
__device__ __forceinline__ void mwalk(int n, const uint32_t* sbits, const KeySrc s, F f) {
  int beg, end;
  mseg_wave(n, &beg, &end);
  const int lane4 = 4 * lane_id();
  const int s0 = blockIdx.x * MSEG;
#pragma unroll 1
  for (int base = beg; base < end; base += 256) {
    const int p = base + lane4;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (KIND != KEY_NONE && p < end) x = load4(s, p, end);
    uint32_t cand = 0u;
    if (p < end) {
      cand = ~(sbits[(p - s0) >> 5] >> (p & 31)) & 0xfu;
      if (end - p < 4) cand &= (1u << (end - p)) - 1u;
    }
    u32x4 k = {0u, 0u, 0u, 0u};
    if (KIND != KEY_NONE) {
      k[0] = key_of<KIND>(x.x, s.med);
      k[1] = key_of<KIND>(x.y, s.med);
      k[2] = key_of<KIND>(x.z, s.med);
      k[3] = key_of<KIND>(x.w, s.med);
    }
    f(p, cand, k);
  }
}

__device__ __forceinline__ void mload_bits(const MArgs& a, uint32_t* sbits) {
  const int w0 = blockIdx.x * (MSEG / 32), words = (a.n + 31) >> 5;
  for (int t = threadIdx.x; t < MSEG / 32; t += MTHREADS) sbits[t] = w0 + t < words ? a.bits[w0 + t] : 0u;
  __syncthreads();
}

__device__ __forceinline__ void mstore_bits(const MArgs& a, const uint32_t* sbits) {
  __syncthreads();
  const int w0 = blockIdx.x * (MSEG / 32), words = (a.n + 31) >> 5;
  for (int t = threadIdx.x; t < MSEG / 32; t += MTHREADS)
    if (w0 + t < words) a.bits[w0 + t] = sbits[t];
}

__device__ __forceinline__ void mmark(uint32_t* sbits, int p, uint32_t m, uint8_t* category, uint8_t cat) {
  if (!m) return;
  atomicOr(&sbits[(p - static_cast<int>(blockIdx.x) * MSEG) >> 5], m << (p & 31));
  if (category)
    for (int e = 0; e < 4; ++e)
      if ((m >> e) & 1u) category[p + e] = cat;
}

// Sum of segcnt over the segments before this one.
__device__ __forceinline__ int mseg_start(const MArgs& a, int* sm) {
  int v = 0;
  for (int g = threadIdx.x; g < static_cast<int>(blockIdx.x); g += MTHREADS) v += a.segcnt[g];
  v = wave_sum(v);
  if (lane_id() == 0) sm[threadIdx.x >> 6] = v;
  __syncthreads();
  const int r = sm[0] + sm[1] + sm[2] + sm[3];
  __syncthreads();
  return r;
}

// Exclusive prefix of the four waves' totals, plus the workgroup's start.
__device__ __forceinline__ int mwave_start(int mine, int* sm) {
  if (lane_id() == 0) sm[threadIdx.x >> 6] = mine;
  __syncthreads();
  int s = 0;
  for (int w = 0; w < static_cast<int>(threadIdx.x >> 6); ++w) s += sm[w];
  __syncthreads();
  return s;
}

// Bitmap words of the local window and (no scores) of the fallback range;
// clears the histograms and counters.
__global__ __launch_bounds__(MTHREADS) void msel_init_kernel(MArgs a) {
  const int words = (a.n + 31) >> 5;
  const int l0 = a.n - a.local, f0 = a.imp_fallback_lo;
  for (int t = threadIdx.x; t < MSEG / 32; t += MTHREADS) {
    const int w = blockIdx.x * (MSEG / 32) + t;
    if (w >= words) continue;
    uint32_t m = 0u;
    for (int j = 0; j < 32; ++j) {
      const int p = 32 * w + j;
      if (p < a.n && (p >= l0 || (p >= f0 && p < l0))) m |= 1u << j;
    }
    a.bits[w] = m;
  }
  if (a.category) {
    const int s0 = blockIdx.x * MSEG, s1 = s0 + MSEG < a.n ? s0 + MSEG : a.n;
    for (int p = s0 + threadIdx.x; p < s1; p += MTHREADS) {
      if (p >= l0) a.category[p] = 1;
      else if (p >= f0) a.category[p] = 2;
    }
  }
  for (int i = blockIdx.x * MTHREADS + threadIdx.x; i < MHIST_ROWS * SEL_BINS; i += a.G * MTHREADS)
    a.hist[i] = 0u;
  if (blockIdx.x == 0 && threadIdx.x == 0) a.state[0] = 0;
}

template <int KIND>
__device__ __forceinline__ KeySrc msrc_resolved(const MArgs& a, const MStep& st, int* sm) {
  KeySrc s = st.src;
  if (KIND == KEY_DIST) {
    const Resolved m = resolve(a.hist, st.med_hbase, 3, st.med_need, sm);
    s.med = a.state[0] ? __uint_as_float(0x7fc00000u) : key_float(m.prefix);
  }
  return s;
}

// Radix pass st.pass of a selection: the segment's histogram of the
// candidates matching the prefix of the earlier passes, added into row
// hbase + pass.
template <int KIND>
__global__ __launch_bounds__(MTHREADS) void msel_hist_kernel(MArgs a, MStep st) {
  __shared__ uint32_t sbits[MSEG / 32];
  __shared__ uint32_t hist[SEL_BINS];
  __shared__ int sm[4];
  const KeySrc s = msrc_resolved<KIND>(a, st, sm);
  const uint32_t prefix = st.pass ? resolve(a.hist, st.hbase, st.pass, st.need, sm).prefix : 0u;
  const uint32_t mask = prefix_mask(st.pass);
  const int shift = st.pass == 0 ? 21 : st.pass == 1 ? 10 : 0;
  const uint32_t nbm = st.pass == 2 ? 1023u : 2047u;
  for (int b = threadIdx.x; b < SEL_BINS; b += MTHREADS) hist[b] = 0u;
  mload_bits(a, sbits);  // (its barrier also orders the clearing)
  int nan = 0;
  mwalk<KIND>(a.n, sbits, s, [&](int, uint32_t cand, u32x4 k) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool act = ((cand >> e) & 1u) && (k[e] & mask) == prefix;
      hist_add(hist, act, (k[e] >> shift) & nbm);
      if (KIND == KEY_ASC) nan += (act && k[e] == NAN_KEY) ? 1 : 0;
    }
  });
  __syncthreads();
  uint32_t* row = a.hist + static_cast<int64_t>(st.hbase + st.pass) * SEL_BINS;
  for (int b = threadIdx.x; b < SEL_BINS; b += MTHREADS)
    if (hist[b]) atomicAdd(&row[b], hist[b]);
  if (KIND == KEY_ASC && st.pass == 0) {
    nan = wave_sum(nan);
    if (lane_id() == 0 && nan) atomicAdd(&a.state[0], nan);
  }
}

// Keys below the threshold are kept; keys equal to it too when all of them
// complete the selection, else their count per segment goes to segcnt.
template <int KIND>
__global__ __launch_bounds__(MTHREADS) void msel_mark_kernel(MArgs a, MStep st) {
  __shared__ uint32_t sbits[MSEG / 32];
  __shared__ int sm[4];
  const KeySrc s = msrc_resolved<KIND>(a, st, sm);
  const Resolved th = resolve(a.hist, st.hbase, 3, st.need, sm);
  const bool all_eq = th.need == th.eq;
  mload_bits(a, sbits);
  int eq = 0;
  mwalk<KIND>(a.n, sbits, s, [&](int p, uint32_t cand, u32x4 k) {
    uint32_t m = 0u, q = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (!((cand >> e) & 1u)) continue;
      if (k[e] < th.prefix) m |= 1u << e;
      if (k[e] == th.prefix) q |= 1u << e;
    }
    if (all_eq)
      m |= q;
    else
      eq += __popc(q);
    mmark(sbits, p, m, a.category, st.cat);
  });
  mstore_bits(a, sbits);
  eq = wave_sum(eq);
  if (lane_id() == 0) sm[threadIdx.x >> 6] = eq;
  __syncthreads();
  if (threadIdx.x == 0) a.segcnt[blockIdx.x] = sm[0] + sm[1] + sm[2] + sm[3];
}

// Position-ordered marking of the candidates with q set whose global rank
// lies in [first, first + count); wave_tot: the waves' counts of such
// candidates, start: those of the earlier segments.
template <int KIND, class Q>
__device__ __forceinline__ void mmark_ranked(const MArgs& a, const KeySrc s, uint32_t* sbits, int start,
                                             int first, int count, Q q_of, uint8_t cat, int* sm) {
  int mine = 0;
  mwalk<KIND>(a.n, sbits, s, [&](int, uint32_t cand, u32x4 k) { mine += __popc(q_of(cand, k)); });
  int carry = start + mwave_start(wave_sum(mine), sm);
  mwalk<KIND>(a.n, sbits, s, [&](int p, uint32_t cand, u32x4 k) {
    const uint32_t q = q_of(cand, k);
    int below, tot;
    lane_offsets<3>(__popc(q), &below, &tot);
    if (carry < first + count && carry + tot > first) {
      uint32_t m = 0u;
      int r = carry + below;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (!((q >> e) & 1u)) continue;
        if (r >= first && r < first + count) m |= 1u << e;
        ++r;
      }
      mmark(sbits, p, m, a.category, cat);
    }
    carry += tot;
  });
}

// Ties: the first need keys equal to the threshold, in position order.
template <int KIND>
__global__ __launch_bounds__(MTHREADS) void msel_tie_kernel(MArgs a, MStep st) {
  __shared__ uint32_t sbits[MSEG / 32];
  __shared__ int sm[4];
  const KeySrc s = msrc_resolved<KIND>(a, st, sm);
  const Resolved th = resolve(a.hist, st.hbase, 3, st.need, sm);
  if (th.need == th.eq) return;  // the mark pass kept them all (uniform)
  const int start = mseg_start(a, sm);
  if (start >= th.need) return;
  mload_bits(a, sbits);
  const uint32_t key = th.prefix;
  mmark_ranked<KIND>(a, s, sbits, start, 0, th.need, [key](uint32_t cand, u32x4 k) {
    uint32_t q = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (((cand >> e) & 1u) && k[e] == key) q |= 1u << e;
    return q;
  }, st.cat, sm);
  mstore_bits(a, sbits);
}

// Positional bridges: candidates per segment, then ranks [first, first + count).
__global__ __launch_bounds__(MTHREADS) void msel_rank_count_kernel(MArgs a) {
  __shared__ uint32_t sbits[MSEG / 32];
  __shared__ int sm[4];
  mload_bits(a, sbits);
  const KeySrc none = {nullptr, 0, 0.f};
  int mine = 0;
  mwalk<KEY_NONE>(a.n, sbits, none, [&](int, uint32_t cand, u32x4) { mine += __popc(cand); });
  mine = wave_sum(mine);
  if (lane_id() == 0) sm[threadIdx.x >> 6] = mine;
  __syncthreads();
  if (threadIdx.x == 0) a.segcnt[blockIdx.x] = sm[0] + sm[1] + sm[2] + sm[3];
}

__global__ __launch_bounds__(MTHREADS) void msel_rank_mark_kernel(MArgs a, MStep st) {
  __shared__ uint32_t sbits[MSEG / 32];
  __shared__ int sm[4];
  const int start = mseg_start(a, sm);
  if (start >= st.first + st.count) return;
  mload_bits(a, sbits);
  const KeySrc none = {nullptr, 0, 0.f};
  mmark_ranked<KEY_NONE>(a, none, sbits, start, st.first, st.count,
                         [](uint32_t cand, u32x4) { return cand; }, st.cat, sm);
  mstore_bits(a, sbits);
}

// Kept positions per segment, then the ascending list, the evicted
// categories and the counts.
__global__ __launch_bounds__(MTHREADS) void msel_compact_count_kernel(MArgs a) {
  __shared__ int sm[4];
  const int w0 = blockIdx.x * (MSEG / 32), words = (a.n + 31) >> 5;
  int c = 0;
  for (int t = threadIdx.x; t < MSEG / 32; t += MTHREADS)
    if (w0 + t < words) c += __popc(a.bits[w0 + t]);
  c = wave_sum(c);
  if (lane_id() == 0) sm[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) a.segcnt[blockIdx.x] = sm[0] + sm[1] + sm[2] + sm[3];
}

__global__ __launch_bounds__(MTHREADS) void msel_compact_write_kernel(MArgs a) {
  __shared__ int sm[4];
  const int start = mseg_start(a, sm);
  const int words = (a.n + 31) >> 5;
  // wave v: words 32 v .. 32 v + 31 of the segment, lane l < 32 one word
  const int lane = lane_id();
  const int w = blockIdx.x * (MSEG / 32) + (threadIdx.x >> 6) * 32 + lane;
  const uint32_t bits = lane < 32 && w < words ? a.bits[w] : 0u;
  int below, tot;
  lane_offsets<6>(__popc(bits), &below, &tot);
  const int pos = start + mwave_start(tot, sm) + below;
  int64_t* out = a.keep + pos;
  for (uint32_t m = bits; m; m &= m - 1) *out++ = 32 * w + __builtin_ctz(m);
  if (a.category && lane < 32 && w < words) {
    const int hi = 32 * w + 32 < a.n ? 32 * w + 32 : a.n;
    for (int i = 32 * w; i < hi; ++i)
      if (!((bits >> (i & 31)) & 1u)) a.category[i] = 0;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    int total = 0;
    for (int g = 0; g < a.G; ++g) total += a.segcnt[g];
    a.counts[0] = a.local;
    a.counts[1] = a.n_imp;
    a.counts[2] = a.n_br;
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
    x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
        a.src[tns] + b * a.ss[0] + h * a.ss[1] + s * a.ss[2] + 16 * c));
  // rows are moved once: non-temporal loads and stores (10 % faster)
  __builtin_nontemporal_store(
      x, reinterpret_cast<u32x4*>(a.dst[tns] + b * a.ds[0] + h * a.ds[1] + t * a.ds[2] + 16 * c));
}

}  // namespace
}  // namespace cab

using namespace cab;

namespace {

struct MLayout {
  int64_t G;
  size_t off_bits, off_hist, off_seg, off_state, total;
};

// Bytes of the multi-workgroup workspace for n positions (mlayout's total).
constexpr size_t mworkspace_bytes(int64_t n) {
  const int64_t G = ((n > 0 ? n : 1) + MSEG - 1) / MSEG;
  auto r256 = [](int64_t b) { return static_cast<size_t>((b + 255) / 256 * 256); };
  return r256(G * (MSEG / 32) * 4) + r256(int64_t{MHIST_ROWS} * SEL_BINS * 4) + r256(G * 4) +
         r256(64 * 4);
}

// Scratch of cab_evict_select_noalloc: the workspace of the largest cache
// (SEL_MAX_LEN positions, 206080 bytes), one copy per GPU for the life of
// the process. Host code never passes the symbol itself to a kernel: it
// takes the device address from hipGetSymbolAddress, per device.
constexpr size_t NOALLOC_SCRATCH_BYTES = mworkspace_bytes(SEL_MAX_LEN);
static_assert(NOALLOC_SCRATCH_BYTES == 206080, "the size the header documents");
__device__ __align__(256) char scratch[NOALLOC_SCRATCH_BYTES];

MLayout mlayout(int64_t n) {
  MLayout L;
  L.G = ceil_div(n > 0 ? n : 1, MSEG);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += static_cast<size_t>(round_up(static_cast<int64_t>(bytes), 256));
    return at;
  };
  L.off_bits = take(static_cast<size_t>(L.G) * (MSEG / 32) * 4);
  L.off_hist = take(static_cast<size_t>(MHIST_ROWS) * SEL_BINS * 4);
  L.off_seg = take(static_cast<size_t>(L.G) * 4);
  L.off_state = take(64 * 4);
  L.total = o;
  return L;
}

// One radix selection (three histogram passes, the mark pass, the tie pass).
template <int KIND>
cab_status_t msel_select(const MArgs& a, MStep st, hipStream_t s, const char* fn) {
  const dim3 grid(static_cast<unsigned>(a.G));
  for (int pass = 0; pass < 3; ++pass) {
    st.pass = pass;
    msel_hist_kernel<KIND><<<grid, MTHREADS, 0, s>>>(a, st);
    cab_status_t r = launch_status(fn);
    if (r != CAB_OK) return r;
  }
  msel_mark_kernel<KIND><<<grid, MTHREADS, 0, s>>>(a, st);
  cab_status_t r = launch_status(fn);
  if (r != CAB_OK) return r;
  msel_tie_kernel<KIND><<<grid, MTHREADS, 0, s>>>(a, st);
  return launch_status(fn);
}

}  // namespace

extern "C" size_t cab_evict_select_workspace_bytes(int64_t cache_len) {
  if (cache_len < 0 || cache_len > SEL_MAX_LEN) return 0;
  return mlayout(cache_len).total;
}

extern "C" cab_status_t cab_evict_select(const float* importance_scores, int64_t n_scores,
                                         const float* bridge_scores, int64_t cache_len,
                                         int32_t local_budget, int32_t importance_budget,
                                         int32_t bridge_budget, int importance_fallback,
                                         int bridge_mode, int64_t* keep_indices, int32_t* counts,
                                         uint8_t* category, void* workspace,
                                         size_t workspace_bytes, void* stream) {
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
  const bool multi = cache_len >= MULTI_MIN;
  const MLayout L = mlayout(cache_len);
  if (multi) {
    CAB_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, CAB_EWORKSPACE,
                "%s: workspace of %zu bytes given, %zu needed", fn, workspace_bytes, L.total);
    CAB_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, CAB_EWORKSPACE,
                "%s: workspace not 256-byte aligned", fn);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int32_t n = static_cast<int32_t>(cache_len);
  const int32_t n_sc = static_cast<int32_t>(n_scores < cache_len ? n_scores : cache_len);
  if (!multi) {
    SelArgs a;
    a.scores = importance_scores;
    a.bridge = bridge_scores;
    a.keep = keep_indices;
    a.counts = counts;
    a.category = category;
    a.n = n;
    a.n_scores = n_sc;
    a.local = local_budget;
    a.imp = importance_budget;
    a.bridge_budget = bridge_budget;
    a.imp_fallback = importance_fallback ? 1 : 0;
    a.bridge_mode = bridge_mode;
    evict_select_kernel<<<1, SEL_THREADS, 0, s>>>(a);
    return launch_status(fn);
  }

  // The plan evict_select_kernel follows, known from the budgets alone.
  const bool has_scores = importance_scores != nullptr;
  const int32_t free0 = n - local_budget;
  int32_t n_imp = 0, f0 = n;
  if (has_scores) {
    n_imp = importance_budget < free0 ? importance_budget : free0;
  } else if (importance_fallback && importance_budget > 0) {
    f0 = n - local_budget - importance_budget > 0 ? n - local_budget - importance_budget : 0;
    n_imp = free0 - f0;
  }
  const int32_t free1 = free0 - n_imp;
  int mode = bridge_mode;
  if (mode == 2 && n_imp == 0) mode = has_scores ? 1 : 3;
  if (mode == 1 && !has_scores) mode = 3;
  int32_t n_br = 0;
  if (bridge_budget > 0 && free1 > 0 && mode != 0) {
    n_br = bridge_budget < free1 ? bridge_budget : free1;
    if (mode == 3 && n_br > free1 - free1 / 3) n_br = free1 - free1 / 3;
  }

  char* ws = static_cast<char*>(workspace);
  MArgs a;
  a.scores = importance_scores;
  a.bridge = bridge_scores;
  a.keep = keep_indices;
  a.counts = counts;
  a.category = category;
  a.bits = reinterpret_cast<uint32_t*>(ws + L.off_bits);
  a.hist = reinterpret_cast<uint32_t*>(ws + L.off_hist);
  a.segcnt = reinterpret_cast<int32_t*>(ws + L.off_seg);
  a.state = reinterpret_cast<int32_t*>(ws + L.off_state);
  a.n = n;
  a.n_scores = n_sc;
  a.G = static_cast<int32_t>(L.G);
  a.local = local_budget;
  a.n_imp = n_imp;
  a.n_br = n_br;
  a.imp_fallback_lo = has_scores ? n : f0;
  const dim3 grid(static_cast<unsigned>(L.G));
  msel_init_kernel<<<grid, MTHREADS, 0, s>>>(a);
  cab_status_t r = launch_status(fn);
  if (r != CAB_OK) return r;
  MStep st{};
  st.src = KeySrc{importance_scores, n_sc, 0.f};
  if (has_scores && n_imp > 0) {
    st.hbase = 0;
    st.need = n_imp;
    st.cat = 2;
    if ((r = msel_select<KEY_DESC>(a, st, s, fn)) != CAB_OK) return r;
  }
  if (n_br > 0) {
    if (mode == 1) {
      MStep md = st;  // the lower median: the ((free1 - 1) / 2 + 1)-th smallest score
      md.hbase = 3;
      md.need = (free1 - 1) / 2 + 1;
      for (int pass = 0; pass < 3; ++pass) {
        md.pass = pass;
        msel_hist_kernel<KEY_ASC><<<grid, MTHREADS, 0, s>>>(a, md);
        if ((r = launch_status(fn)) != CAB_OK) return r;
      }
      MStep bs = st;
      bs.hbase = 6;
      bs.need = n_br;
      bs.med_hbase = 3;
      bs.med_need = md.need;
      bs.cat = 3;
      if ((r = msel_select<KEY_DIST>(a, bs, s, fn)) != CAB_OK) return r;
    } else if (mode == 2) {
      MStep bs = st;
      bs.src = KeySrc{bridge_scores, n, 0.f};
      bs.hbase = 6;
      bs.need = n_br;
      bs.cat = 3;
      if ((r = msel_select<KEY_DESC>(a, bs, s, fn)) != CAB_OK) return r;
    } else {
      msel_rank_count_kernel<<<grid, MTHREADS, 0, s>>>(a);
      if ((r = launch_status(fn)) != CAB_OK) return r;
      MStep rk = st;
      rk.first = free1 / 3;
      rk.count = n_br;
      rk.cat = 3;
      msel_rank_mark_kernel<<<grid, MTHREADS, 0, s>>>(a, rk);
      if ((r = launch_status(fn)) != CAB_OK) return r;
    }
  }
  msel_compact_count_kernel<<<grid, MTHREADS, 0, s>>>(a);
  if ((r = launch_status(fn)) != CAB_OK) return r;
  msel_compact_write_kernel<<<grid, MTHREADS, 0, s>>>(a);
  return launch_status(fn);
}

namespace {

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch[NOALLOC_MAX_DEVICES] = {};

// The device address of the current device's scratch, looked up once per
// device (with that device current) and kept.
cab_status_t scratch_of_current_device(const char* fn, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  CAB_REQUIRE(e == hipSuccess, CAB_EHIP, "%s: hipGetDevice failed: %s", fn, hipGetErrorString(e));
  CAB_REQUIRE(dev >= 0 && dev < NOALLOC_MAX_DEVICES, CAB_EINVAL, "%s: device %d beyond %d", fn,
              dev, NOALLOC_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    CAB_REQUIRE(e == hipSuccess && p != nullptr, CAB_EHIP,
                "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev,
                hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return CAB_OK;
}

}  // namespace

extern "C" cab_status_t cab_evict_select_noalloc(const float* importance_scores,
                                                 int64_t n_scores, const float* bridge_scores,
                                                 int64_t cache_len, int32_t local_budget,
                                                 int32_t importance_budget, int32_t bridge_budget,
                                                 int importance_fallback, int bridge_mode,
                                                 int64_t* keep_indices, int32_t* counts,
                                                 uint8_t* category, void* stream) {
  const char* fn = "cab_evict_select_noalloc";
  clear_error();
  CAB_REQUIRE(cache_len >= 0 && cache_len <= SEL_MAX_LEN, CAB_ESHAPE,
              "%s: cache_len %lld outside [0, %d] (the size of the built-in scratch)", fn,
              (long long)cache_len, SEL_MAX_LEN);
  void* ws = nullptr;
  if (cache_len >= MULTI_MIN) {
    const size_t need = mlayout(cache_len).total;
    CAB_REQUIRE(need <= NOALLOC_SCRATCH_BYTES, CAB_EWORKSPACE,
                "%s: %zu scratch bytes needed, %zu built in", fn, need, NOALLOC_SCRATCH_BYTES);
    cab_status_t st = scratch_of_current_device(fn, &ws);
    if (st != CAB_OK) return st;
  }
  return cab_evict_select(importance_scores, n_scores, bridge_scores, cache_len, local_budget,
                          importance_budget, bridge_budget, importance_fallback, bridge_mode,
                          keep_indices, counts, category, ws, ws ? NOALLOC_SCRATCH_BYTES : 0,
                          stream);
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
