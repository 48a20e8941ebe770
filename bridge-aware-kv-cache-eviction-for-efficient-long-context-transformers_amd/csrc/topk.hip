// Per-row block selection (cab_block_topk).
//
// One wave64 per FRC row. The row's M scores are read once (coalesced, lane l
// holds columns j = 64 c + l, through a buffer descriptor: no per-lane 64-bit
// addresses, columns past M read as zero) and mapped branch-free to
// order-preserving uint32 keys in registers (NaN scores in a second pass run
// only for rows holding one), non-candidates to a sentinel.
// The k-th smallest key is found by a radix select (8-bit digit windows
// from the highest bit where two candidates differ, a 256-bin LDS histogram
// per wave with four copies per bin, a wave-wide DPP prefix scan, the bin
// chosen in scalar registers, ending early at a bin of one key, whose largest
// value then serves as the threshold). A last pass in ascending j keeps every
// key below the threshold and the first (in j) keys equal to it -- when every
// key equal to the threshold is kept, simply every key at most the threshold
// -- assigns output slots with v_mbcnt over the selection mask, and writes the
// compact ascending index list and, optionally, the dense 0/1 row through
// buffer stores.
//
// Hybrid selection (cab_block_topk_hybrid) first runs the same search on
// the row's magnitude keys for its magnitude quota, marks those blocks taken,
// and then searches the FRC keys of the remaining candidates.
//
// Rows longer than 8192 (up to the 32768 the FRC stage accepts) go to
// topk_stream_kernel: the same search and tie rules with the row read again
// from memory on every pass instead of held in registers. Its hybrid form
// marks the magnitude picks by their threshold and the position of the last
// kept tie.
//
// HBM traffic per row: 4 M bytes read (8 M hybrid); 4 k + 4 (+ M for the
// dense mask) bytes written. Bound by HBM bandwidth. The streaming kernel
// reads the row once per pass (up to 6 passes, mostly from L2 and MALL).
#include "cab_internal.h"

namespace cab {
namespace {

struct TopkArgs {
  const float* frc;
  const float* mag;  // hybrid only: magnitude scores, the highest kept first
  int32_t* kv_idx;
  int32_t* kv_cnt;
  uint8_t* dense;
  int64_t rows, M;
  int32_t k;
  int32_t kmag;      // hybrid only: per-row magnitude quota
  int select_high, keep_diagonal, causal;
};

// The streaming kernel's histogram keeps HSUB interleaved copies of every bin
// (lane % HSUB picks one), so that keys of a row that share the digit do not
// all update one LDS word.
constexpr int HSUB = 8;
// Orders one wave's LDS accesses across its lanes (the histogram is shared
// by the lanes of a wave; other waves of the workgroup may have exited).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// A key no real score maps to (order_key_fast never returns all ones): it stands
// for a column that is not a candidate, so that every candidate ranks below
// it.
constexpr uint32_t KEY_NONE = 0xffffffffu;

// theta = the need-th smallest key among the candidates (the largest theta
// with count(key < theta) < need), by a radix select over the key bits, most
// significant first, for keys held in registers with KEY_NONE for
// non-candidates. The digit windows are not byte-aligned: the first covers
// the 8 bits below and at the highest bit where two candidates differ (the
// candidates share every bit above it), each later one the next 8 bits down,
// so the first pass spreads a narrow range of scores over up to 256 bins
// (fewer same-bin LDS atomics, fewer keys left in the chosen bin). The
// histogram keeps HSUB_REG copies of every bin, copy s of bin b at word
// s * HSTRIDE + b: copies of one bin fall into different LDS banks (HSTRIDE %
// 64 == 4), and lane l clears and sums bins 4 l .. 4 l + 3 of a copy with one
// 16-byte access. The first pass counts every key (a KEY_NONE key lands in the
// top bin, after every candidate of that bin: it is the largest key); later
// passes count the keys matching the prefix. need_eq returns how many keys
// equal to theta (the first ones in j order) complete the selection,
// eq_total how many keys equal theta.
constexpr int HSTRIDE = 260;
constexpr int HSUB_REG = 4;  // copies per bin (fewer copies: more waves per CU fit the LDS)

// Inclusive prefix sum over the 64 lanes of a wave: DPP row shifts by 1, 2,
// 4 and 8 within each row of 16 lanes, then row_bcast:15 (a row's last lane
// added to the next row, rows 1 and 3) and row_bcast:31 (lane 31 added to
// rows 2 and 3). Lanes whose source is outside the row or whose row is
// masked off add the old value 0. No LDS round trips.
template <int CTRL, int ROW_MASK, int OLD>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(OLD, static_cast<int>(v), CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t x) {
  x += dpp_u32<0x111, 0xf, 0>(x);  // row_shr:1
  x += dpp_u32<0x112, 0xf, 0>(x);  // row_shr:2
  x += dpp_u32<0x114, 0xf, 0>(x);  // row_shr:4
  x += dpp_u32<0x118, 0xf, 0>(x);  // row_shr:8
  x += dpp_u32<0x142, 0xa, 0>(x);  // row_bcast:15
  x += dpp_u32<0x143, 0xc, 0>(x);  // row_bcast:31
  return x;
}

// Wave-wide minimum (MAX false) or maximum of x, uniform: DPP row shifts by
// 1, 2, 4 and 8 leave each row's result in its lane 15 (a lane whose source
// is outside its row takes the identity), and the four rows' values are read
// into scalars.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_min_max(uint32_t x) {
  constexpr int ID = MAX ? 0 : -1;
  auto op = [](uint32_t a, uint32_t b) { return MAX ? max(a, b) : min(a, b); };
  x = op(x, dpp_u32<0x111, 0xf, ID>(x));
  x = op(x, dpp_u32<0x112, 0xf, ID>(x));
  x = op(x, dpp_u32<0x114, 0xf, ID>(x));
  x = op(x, dpp_u32<0x118, 0xf, ID>(x));
  auto rl = [&](int l) { return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), l)); };
  return op(op(rl(15), rl(31)), op(rl(47), rl(63)));
}

// The threshold it returns need not be a key of the row: when the search ends
// at a bin holding a single key, it returns the largest key value of that bin
// (the bin's prefix with every lower bit set), which selects the same keys by
// "at most theta" (the bin's one key and everything below it) and equals no
// other key; eq_total and need_eq are then 1. need is at most 64 NCH.
template <int NCH>
__device__ __forceinline__ uint32_t kth_key_reg(const uint32_t (&key)[NCH], int32_t need,
                                                int32_t& need_eq, uint32_t& eq_total, uint32_t* hist) {
  const int lane = lane_id();
  need_eq = 0;
  eq_total = 0;
  if (need <= 0) return 0u;
  // The smallest and the largest candidate key: every candidate lies between
  // them, so the bits above the highest bit where the two differ are shared
  // by all. KEY_NONE never decides the minimum, and KEY_NONE + 1 wraps to 0,
  // so it never decides the maximum of key + 1 (need > 0: a candidate exists).
  uint32_t kmin = 0xffffffffu, kmax1 = 0u;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    kmin = min(kmin, key[c]);
    kmax1 = max(kmax1, key[c] + 1u);
  }
  kmin = wave_min_max<false>(kmin);
  kmax1 = wave_min_max<true>(kmax1);
  const uint32_t diff = kmin ^ (kmax1 - 1u);
  if (diff == 0u) {  // every candidate holds the same key
    need_eq = need;
    eq_total = 0xffffffffu;  // unknown: the caller ranks the ties
    return kmin;
  }
  int hb = 31 - __builtin_clz(diff);          // highest bit where candidates differ
  uint32_t pmask = ~((2u << hb) - 1u);        // the bits above it (none for hb = 31)
  uint32_t prefix = kmin & pmask;
  int32_t rem = need;
  bool first = true;
  char* hp = reinterpret_cast<char*>(hist) + (lane % HSUB_REG) * HSTRIDE * 4;
  while (hb >= 0) {  // at most four windows
    const int lo = hb >= 7 ? hb - 7 : 0;
    const uint32_t wbits = static_cast<uint32_t>(hb - lo + 1);
    const uint32_t wmask = (2u << (hb - lo)) - 1u;
    wave_sync();  // the previous pass's reads are done
#pragma unroll
    for (int q = 0; q < HSUB_REG; ++q)
      *reinterpret_cast<u32x4*>(hist + q * HSTRIDE + 4 * lane) = u32x4{0u, 0u, 0u, 0u};
    wave_sync();
    // Bin of key k: its bits lo .. hb (one bit-field extract).
    auto bin_of = [&](uint32_t k) { return __builtin_amdgcn_ubfe(k, static_cast<uint32_t>(lo), wbits); };
    if (first) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) atomicAdd(reinterpret_cast<uint32_t*>(hp + (bin_of(key[c]) << 2)), 1u);
    } else {
      // After the first window few keys still match the prefix: only the
      // matching lanes add (exec-masked), and a chunk with none skips the
      // atomic altogether.
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const uint32_t kc = key[c];
        if ((kc & pmask) == prefix) atomicAdd(reinterpret_cast<uint32_t*>(hp + (bin_of(kc) << 2)), 1u);
      }
    }
    first = false;
    wave_sync();
    uint32_t hv[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < HSUB_REG; ++q) {
      const u32x4 x = *reinterpret_cast<const u32x4*>(hist + q * HSTRIDE + 4 * lane);
      hv[0] += x[0];
      hv[1] += x[1];
      hv[2] += x[2];
      hv[3] += x[3];
    }
    const uint32_t mine = hv[0] + hv[1] + hv[2] + hv[3];
    const uint32_t incl = wave_incl_sum(mine);
    // The first lane whose bins reach rank rem (a uniform index); its four
    // bin counts and the count below them go to scalars, and the bin is
    // found there.
    const uint64_t reach = ballot64(static_cast<int32_t>(incl) >= rem);
    const int src = __builtin_ctzll(reach);
    auto from_src = [&](uint32_t v) {
      return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), src));
    };
    int32_t below = static_cast<int32_t>(from_src(incl - mine));
    const uint32_t h[4] = {from_src(hv[0]), from_src(hv[1]), from_src(hv[2]), from_src(hv[3])};
    uint32_t q = 0;
    while (q < 3 && below + static_cast<int32_t>(h[q]) < rem) below += static_cast<int32_t>(h[q++]);
    const uint32_t sel_bin = 4u * static_cast<uint32_t>(src) + q;
    const uint32_t sel_cnt = h[q];
    rem -= below;
    prefix |= sel_bin << lo;
    pmask |= wmask << lo;
    eq_total = sel_cnt;
    if (sel_cnt == 1u && lo > 0) {
      // One key left in the bin (rem == 1): it is a candidate (a KEY_NONE
      // key matching the prefix would share its bin), and every key of the
      // row is either below the bin, the bin's one key, or above the bin's
      // largest value.
      need_eq = 1;
      return prefix | ((1u << lo) - 1u);
    }
    hb = lo - 1;
  }
  need_eq = rem;  // keys below theta: need - rem; the rest are ties at theta
  return prefix;
}

// kth_key_reg's search for rows read again from memory on every pass
// (topk_stream_kernel): key(c) loads this lane's key of chunk c and
// is_cand(c) tells whether it is a candidate. The candidates' minimum and
// maximum fix the bits they share; each window of 8 bits from the highest bit
// where two differ is counted in the wave's LDS histogram (HSUB copies per
// bin: 16-byte slot (q, l) at index 64 q + l holds copies 4 (q % 2) .. +3 of
// bin 4 l + q / 2, so lane l clears and sums its own four bins with
// lane-contiguous accesses), a DPP scan and scalar registers pick the bin,
// and a bin holding a single candidate ends the search with the bin's
// largest value as theta, as in kth_key_reg. need_eq returns how many keys
// equal to theta (the first ones in j order) complete the selection.
template <typename Key, typename Cand>
__device__ __forceinline__ uint32_t kth_key_stream(Key key, Cand is_cand, int nch, int32_t need,
                                                   int32_t& need_eq, uint32_t* hist) {
  const int lane = lane_id();
  need_eq = 0;
  if (need <= 0) return 0u;
  uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll 4
  for (int c = 0; c < nch; ++c) {
    if (!is_cand(c)) continue;
    const uint32_t kc = key(c);
    kmin = min(kmin, kc);
    kmax = max(kmax, kc);
  }
  kmin = wave_min_max<false>(kmin);
  kmax = wave_min_max<true>(kmax);
  const uint32_t diff = kmin ^ kmax;
  if (diff == 0u) {  // every candidate holds the same key
    need_eq = need;
    return kmin;
  }
  int hb = 31 - __builtin_clz(diff);
  uint32_t pmask = ~((2u << hb) - 1u);
  uint32_t prefix = kmin & pmask;
  int32_t rem = need;  // rank still to find among the keys matching the prefix
  u32x4* slots = reinterpret_cast<u32x4*>(hist);
  const uint32_t sub = static_cast<uint32_t>(lane % HSUB);
  while (hb >= 0) {  // at most four windows
    const int lo = hb >= 7 ? hb - 7 : 0;
    const uint32_t wmask = (2u << (hb - lo)) - 1u;
    wave_sync();  // the previous pass's reads are done
#pragma unroll
    for (int q = 0; q < HSUB; ++q) slots[64 * q + lane] = u32x4{0u, 0u, 0u, 0u};
    wave_sync();
#pragma unroll 4
    for (int c = 0; c < nch; ++c) {
      if (!is_cand(c)) continue;
      const uint32_t kc = key(c);
      if ((kc & pmask) == prefix) {
        const uint32_t bn = (kc >> lo) & wmask;
        const uint32_t q = 2u * (bn & 3u) + (sub >> 2);
        atomicAdd(&hist[4u * (64u * q + (bn >> 2)) + (sub & 3u)], 1u);
      }
    }
    wave_sync();
    uint32_t hv[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < HSUB; ++q) {
      const u32x4 x = slots[64 * q + lane];
      hv[q / 2] += x[0] + x[1] + x[2] + x[3];
    }
    const uint32_t mine = hv[0] + hv[1] + hv[2] + hv[3];
    const uint32_t incl = wave_incl_sum(mine);
    const uint64_t reach = ballot64(static_cast<int32_t>(incl) >= rem);
    const int src = __builtin_ctzll(reach);
    auto from_src = [&](uint32_t v) {
      return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), src));
    };
    int32_t below = static_cast<int32_t>(from_src(incl - mine));
    const uint32_t h[4] = {from_src(hv[0]), from_src(hv[1]), from_src(hv[2]), from_src(hv[3])};
    uint32_t q = 0;
    while (q < 3 && below + static_cast<int32_t>(h[q]) < rem) below += static_cast<int32_t>(h[q++]);
    const uint32_t sel_cnt = h[q];
    rem -= below;
    prefix |= (4u * static_cast<uint32_t>(src) + q) << lo;
    pmask |= wmask << lo;
    if (sel_cnt == 1u && lo > 0) {  // one candidate left in the bin (rem == 1)
      need_eq = 1;
      return prefix | ((1u << lo) - 1u);
    }
    hb = lo - 1;
  }
  need_eq = rem;  // keys below theta: need - rem; the rest are ties at theta
  return prefix;
}

// Number of set bits of the wave mask m below this lane (v_mbcnt).
__device__ __forceinline__ uint32_t rank_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}

// Order key of the score bits u: ascending key order is the selection order,
// float order with -0 == +0 and NaN above +inf, inverted when the highest
// scores are wanted. Three VALU operations for every score but NaN: f = s x +
// 0 with s = +1, or s = -1 when the highest scores are wanted (-x orders as x
// reversed), turns -0 into +0 (fp32 denormals are kept, so no other value
// changes), and the sign-magnitude bits of f become an unsigned order.
// Non-NaN scores map into [KEY_LO, KEY_HI] (the keys of -inf and +inf), NaN
// scores outside it; the caller gives NaN scores their own key, 0xffc00000
// (the quiet NaN's bits as an unsigned order, above +inf) or its complement
// when the order is reversed.
constexpr uint32_t KEY_LO = 0x007fffffu, KEY_HI = 0xff800000u;
__device__ __forceinline__ uint32_t order_key_fast(uint32_t u, float s) {
  const uint32_t v = __float_as_uint(__builtin_fmaf(__uint_as_float(u), s, 0.0f));
  return v ^ (static_cast<uint32_t>(static_cast<int32_t>(v) >> 31) | 0x80000000u);
}

template <bool B>
struct BoolC {
  static constexpr bool value = B;
};

template <int NCH, bool HYB>
__global__ __launch_bounds__(256) void topk_kernel(TopkArgs a) {
  // The wave index through readfirstlane: the row and everything derived
  // from it (descriptors, limits, the histogram) stay in scalar registers.
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wv;
  if (row >= a.rows) return;  // uniform per wave
  const int lane = lane_id();
  const int64_t i = row % a.M;
  const int64_t ncand = a.causal ? i + 1 : a.M;
  const int32_t krow = static_cast<int32_t>(min(static_cast<int64_t>(a.k), ncand));
  const bool kd = a.keep_diagonal != 0;
  const int32_t need = kd ? krow - 1 : krow;
  __shared__ __attribute__((aligned(16))) uint32_t hist_all[4][HSUB_REG * HSTRIDE];
  uint32_t* hist = hist_all[wv];

  // Lane l holds column j = 64 c + l of chunk c. The row is read through a
  // buffer descriptor (columns past M read as zero), all NCH loads in flight
  // together. The whole byte offset 4 (64 c + lane) goes in the per-lane
  // offset (the compiler folds 256 c into the instruction's immediate): the
  // descriptor's range check covers the per-lane offset plus the immediate,
  // while a scalar offset is not range-checked on gfx9, so chunks past M
  // must not be addressed through it.
  // Non-candidates (columns j >= ncand and the forced diagonal) carry
  // KEY_NONE. Only the chunk holding the limit compares lanes, the chunks
  // past it hold no candidate, and only the diagonal's chunk marks a lane;
  // these chunk indices are the same for every lane, so marking is a few
  // register-indexed moves after the mapping instead of a test per chunk.
  const int lim = static_cast<int>(ncand);
  const int cl = lim >> 6;                               // the chunk holding the limit
  const int dch = static_cast<int>(i >> 6);              // the diagonal's chunk
  const bool dlane = lane == static_cast<int>(i & 63);   // and lane
  // Rows of more than 32 chunks mark by a uniform test per chunk instead:
  // register-indexed access to a longer key array makes the compiler keep the
  // array in scratch memory.
  auto mark = [&](uint32_t (&kk)[NCH]) {
    if constexpr (NCH <= 32) {
      if (cl < NCH) {
        kk[cl] = lane < lim - 64 * cl ? kk[cl] : KEY_NONE;
#pragma nounroll
        for (int c = cl + 1; c < NCH; ++c) kk[c] = KEY_NONE;
      }
      if (kd) kk[dch] = dlane ? KEY_NONE : kk[dch];
    } else {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if (c > cl)
          kk[c] = KEY_NONE;
        else if (c == cl)
          kk[c] = lane < lim - 64 * cl ? kk[c] : KEY_NONE;
        if (kd && c == dch) kk[c] = dlane ? KEY_NONE : kk[c];
      }
    }
  };
  // Loads a row's scores and maps them to keys (high: the order reversed).
  // The keys' minimum and maximum show whether any lane holds a NaN; only
  // then (a uniform branch) do the keys outside [KEY_LO, KEY_HI] take NaN's
  // key, the one above every other (below every other when reversed).
  auto load_keys = [&](const float* src, bool high, uint32_t (&kk)[NCH]) {
    const brsrc_t rs = make_rsrc(src, static_cast<uint32_t>(a.M * 4));
    uint32_t u[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      u[c] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rs, 4u * (64u * c + lane), 0u, 0));
    const float s = high ? -1.0f : 1.0f;
    uint32_t kmn = 0xffffffffu, kmx = 0u;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      kk[c] = order_key_fast(u[c], s);
      kmn = min(kmn, kk[c]);
      kmx = max(kmx, kk[c]);
    }
    if (ballot64(kmn < KEY_LO || kmx > KEY_HI) != 0u) {
      const uint32_t nan_key = high ? ~0xffc00000u : 0xffc00000u;
#pragma unroll
      for (int c = 0; c < NCH; ++c) kk[c] = kk[c] - KEY_LO > KEY_HI - KEY_LO ? nan_key : kk[c];
    }
    mark(kk);
  };
  uint32_t key[NCH];
  load_keys(a.frc + row * a.M, a.select_high != 0, key);

  // Hybrid: the need_m candidates of highest magnitude first (bit c of msel
  // marks register c of this lane as taken).
  uint64_t msel[(NCH + 63) / 64];
#pragma unroll
  for (int w = 0; w < (NCH + 63) / 64; ++w) msel[w] = 0;
  int32_t need_m = 0;
  if constexpr (HYB) {
    need_m = min(a.kmag, need);
    uint32_t mkey[NCH];
    load_keys(a.mag + row * a.M, true, mkey);
    int32_t meq = 0;
    uint32_t mtot = 0;
    const uint32_t mtheta = kth_key_reg<NCH>(mkey, need_m, meq, mtot, hist);
    int32_t eq_seen = 0;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const bool cand = mkey[c] != KEY_NONE && need_m > 0;
      const bool eq = cand && mkey[c] == mtheta;
      const uint64_t eqb = ballot64(eq);
      const int32_t eq_rank = eq_seen + static_cast<int32_t>(rank_below(eqb));
      if ((cand && mkey[c] < mtheta) || (eq && eq_rank < meq)) msel[c >> 6] |= 1ull << (c & 63);
      eq_seen += __popcll(eqb);
    }
  }
  auto taken = [&](int c) { return ((msel[c >> 6] >> (c & 63)) & 1ull) != 0; };
  if constexpr (HYB) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) key[c] = taken(c) ? KEY_NONE : key[c];
  }

  // FRC order for the rest of the row (taken columns now carry KEY_NONE).
  const int32_t need_f = need - need_m;
  int32_t need_eq = 0;
  uint32_t eq_total = 0;
  const uint32_t theta = kth_key_reg<NCH>(key, need_f, need_eq, eq_total, hist);

  // The compact list goes out through buffer stores from the selected lanes
  // only (exec-masked: no offset to compute for the others), the dense row
  // from every lane, through a descriptor that drops columns past M. Output
  // slots come from v_mbcnt over the selection mask.
  // The forced diagonal takes key 0, below every real key (order_key_fast
  // never returns 0), so the selection tests below keep it.
  if constexpr (NCH <= 32) {
    if (kd) key[dch] = dlane ? 0u : key[dch];
  } else {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      if (kd && c == dch) key[c] = dlane ? 0u : key[c];
  }
  uint32_t pos = 0;
  int32_t* out = a.kv_idx + row * a.k;
  const brsrc_t ors = make_rsrc(out, static_cast<uint32_t>(a.k * 4));
  const bool dense = a.dense != nullptr;
  const brsrc_t drs = make_rsrc(dense ? a.dense + row * a.M : nullptr, dense ? static_cast<uint32_t>(a.M) : 0u);
  // One copy of the output pass with the dense row and one without, so the
  // choice is one branch instead of one per chunk.
  auto output_pass = [&](auto dense_c) {
    constexpr bool DENSE = decltype(dense_c)::value;
    auto emit = [&](int c, bool sel) {
      const uint64_t selb = ballot64(sel);
      const uint32_t j = 64u * c + lane;
      if (sel) __builtin_amdgcn_raw_buffer_store_b32(j, ors, 4u * (pos + rank_below(selb)), 0u, 0);
      // the dense row is never read back here: non-temporal stores (4 % faster)
      if constexpr (DENSE)
        __builtin_amdgcn_raw_buffer_store_b8(static_cast<unsigned char>(sel ? 1 : 0), drs, j, 0u, CPOL_NT);
      pos += static_cast<uint32_t>(__popcll(selb));
    };
    if (need_f <= 0 || static_cast<uint32_t>(need_eq) == eq_total) {
      // Every key equal to theta is kept: a key is selected iff it is at most
      // theta (KEY_NONE ranks above every real theta).
      const uint32_t th = need_f > 0 ? theta : 0u;  // nothing but the diagonal when no candidate is kept
#pragma unroll
      for (int c = 0; c < NCH; ++c) emit(c, key[c] <= th || (HYB && taken(c)));
    } else {
      int32_t eq_seen = 0;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const bool cand = key[c] != KEY_NONE;
        const bool eq = cand && key[c] == theta;
        const uint64_t eqb = ballot64(eq);
        const int32_t eq_rank = eq_seen + static_cast<int32_t>(rank_below(eqb));
        emit(c, (cand && key[c] < theta) || (eq && eq_rank < need_eq) || (HYB && taken(c)));
        eq_seen += __popcll(eqb);
      }
    }
  };
  if (dense)
    output_pass(BoolC<true>{});
  else
    output_pass(BoolC<false>{});
  for (int64_t p = pos + lane; p < a.k; p += 64) out[p] = -1;
  if (lane == 0) a.kv_cnt[row] = static_cast<int32_t>(pos);
}

// One wave per row for M > 8192: every pass reads the row's keys again
// (lane l, columns 64 c + l, coalesced). Same selection and tie rules as
// topk_kernel; in the hybrid form a candidate is taken by magnitude when its
// key is below the magnitude threshold, or equal to it and no later in j
// than the last tie the quota keeps.
template <bool HYB>
__global__ __launch_bounds__(256) void topk_stream_kernel(TopkArgs a) {
  // The wave index through readfirstlane: the row and everything derived
  // from it (descriptors, limits, the histogram) stay in scalar registers.
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wv;
  if (row >= a.rows) return;  // uniform per wave
  const int lane = lane_id();
  const int64_t i = row % a.M;
  const int64_t ncand = a.causal ? i + 1 : a.M;
  const int32_t krow = static_cast<int32_t>(min(static_cast<int64_t>(a.k), ncand));
  const bool kd = a.keep_diagonal != 0;
  const int32_t need = kd ? krow - 1 : krow;
  const bool high = a.select_high != 0;
  const uint64_t lt_mask = lanemask_lt();
  __shared__ __attribute__((aligned(16))) uint32_t hist_all[4][256 * HSUB];
  uint32_t* hist = hist_all[wv];
  const int Mi = static_cast<int>(a.M), nch = (Mi + 63) / 64;
  const int ncand_i = static_cast<int>(ncand), i_i = static_cast<int>(i);
  auto is_cand = [&](int c) {
    const int j = 64 * c + lane;
    return j < ncand_i && !(kd && j == i_i);
  };
  // Keys through one buffer descriptor per row (columns past M read as zero;
  // they are never candidates), by the three-instruction map; a key outside
  // [KEY_LO, KEY_HI] comes from a NaN score and takes NaN's key (the row is
  // not held, so every load is tested).
  auto load_key = [&](const brsrc_t& rs, int c, float sgn, uint32_t nan_key) {
    const uint32_t u = static_cast<uint32_t>(
        __builtin_amdgcn_raw_buffer_load_b32(rs, 4u * (64u * c + lane), 0u, 0));
    const uint32_t kk = order_key_fast(u, sgn);
    return kk - KEY_LO > KEY_HI - KEY_LO ? nan_key : kk;
  };
  const brsrc_t frs = make_rsrc(a.frc + row * a.M, static_cast<uint32_t>(a.M * 4));
  const float fsgn = high ? -1.0f : 1.0f;
  const uint32_t fnan = high ? ~0xffc00000u : 0xffc00000u;
  auto fkey = [&](int c) { return load_key(frs, c, fsgn, fnan); };
  const brsrc_t mrs = make_rsrc(HYB ? a.mag + row * a.M : nullptr, HYB ? static_cast<uint32_t>(a.M * 4) : 0u);
  auto mkey = [&](int c) { return load_key(mrs, c, -1.0f, ~0xffc00000u); };

  int32_t need_m = 0;
  uint32_t mtheta = 0u;
  int jm_last = -1;  // the last tie at mtheta (in j) the quota keeps
  if constexpr (HYB) {
    need_m = min(a.kmag, need);
    int32_t meq = 0;
    mtheta = kth_key_stream(mkey, is_cand, nch, need_m, meq, hist);
    if (need_m > 0 && meq > 0) {
      int32_t seen = 0;
      for (int c = 0; c < nch && jm_last < 0; ++c) {  // uniform: ballots only
        const bool eq = is_cand(c) && mkey(c) == mtheta;
        const uint64_t eqb = ballot64(eq);
        const int32_t r = meq - 1 - seen;  // its rank among this chunk's ties
        if (r < __popcll(eqb)) {
          const uint64_t hit = ballot64(eq && __popcll(eqb & lt_mask) == r);
          jm_last = 64 * c + __builtin_ctzll(hit);
        }
        seen += __popcll(eqb);
      }
    }
  }
  auto taken = [&](int c) {
    if (!HYB || need_m <= 0 || !is_cand(c)) return false;
    const uint32_t mk = mkey(c);
    return mk < mtheta || (mk == mtheta && 64 * c + lane <= jm_last);
  };
  auto is_cand_f = [&](int c) { return is_cand(c) && !taken(c); };

  const int32_t need_f = need - need_m;
  int32_t need_eq = 0;
  const uint32_t theta = kth_key_stream(fkey, is_cand_f, nch, need_f, need_eq, hist);

  // Output as in topk_kernel: list stores from the selected lanes, the dense
  // row through a descriptor that drops columns past M.
  uint32_t pos = 0;
  int32_t eq_seen = 0;
  int32_t* out = a.kv_idx + row * a.k;
  const brsrc_t ors = make_rsrc(out, static_cast<uint32_t>(a.k * 4));
  const bool dense = a.dense != nullptr;
  const brsrc_t drs = make_rsrc(dense ? a.dense + row * a.M : nullptr, dense ? static_cast<uint32_t>(a.M) : 0u);
  for (int c = 0; c < nch; ++c) {
    const uint32_t j = 64u * c + lane;
    const bool tk = taken(c);
    const bool cand = need_f > 0 && is_cand(c) && !tk;
    const uint32_t kc = cand ? fkey(c) : KEY_NONE;
    const bool eq = cand && kc == theta;
    const uint64_t eqb = ballot64(eq);
    const int32_t eq_rank = eq_seen + static_cast<int32_t>(rank_below(eqb));
    const bool sel = (cand && kc < theta) || (eq && eq_rank < need_eq) || tk || (kd && static_cast<int>(j) == i_i);
    const uint64_t selb = ballot64(sel);
    if (sel) __builtin_amdgcn_raw_buffer_store_b32(j, ors, 4u * (pos + rank_below(selb)), 0u, 0);
    if (dense) __builtin_amdgcn_raw_buffer_store_b8(static_cast<unsigned char>(sel ? 1 : 0), drs, j, 0u, CPOL_NT);
    pos += static_cast<uint32_t>(__popcll(selb));
    eq_seen += __popcll(eqb);
  }
  for (int64_t p = pos + lane; p < a.k; p += 64) out[p] = -1;
  if (lane == 0) a.kv_cnt[row] = static_cast<int32_t>(pos);
}

template <bool HYB>
void launch_topk(const TopkArgs& a, dim3 grid, hipStream_t s) {
  const int64_t nch = ceil_div(a.M, 64);
  if (nch <= 1) topk_kernel<1, HYB><<<grid, 256, 0, s>>>(a);
  else if (nch <= 2) topk_kernel<2, HYB><<<grid, 256, 0, s>>>(a);
  else if (nch <= 4) topk_kernel<4, HYB><<<grid, 256, 0, s>>>(a);
  else if (nch <= 8) topk_kernel<8, HYB><<<grid, 256, 0, s>>>(a);
  else if (nch <= 16) topk_kernel<16, HYB><<<grid, 256, 0, s>>>(a);
  else if (nch <= 32) topk_kernel<32, HYB><<<grid, 256, 0, s>>>(a);
  else if (nch <= 64) topk_kernel<64, HYB><<<grid, 256, 0, s>>>(a);
  else if (nch <= 128) topk_kernel<128, HYB><<<grid, 256, 0, s>>>(a);
  else topk_stream_kernel<HYB><<<grid, 256, 0, s>>>(a);
}

cab_status_t topk_common(const char* fn, const float* frc, const float* mag, int64_t B, int64_t H,
                         int64_t M, int32_t k, int32_t kmag, int select_high, int keep_diagonal,
                         int causal, int32_t* kv_idx, int32_t* kv_cnt, uint8_t* dense_mask,
                         void* stream, bool hybrid) {
  clear_error();
  CAB_REQUIRE(B >= 0 && H >= 0 && M >= 0, CAB_ESHAPE, "%s: negative size", fn);
  CAB_REQUIRE(M <= 32768, CAB_ESHAPE, "%s: M=%lld exceeds 32768", fn, (long long)M);
  CAB_REQUIRE(k >= 1, CAB_EINVAL, "%s: k=%d must be >= 1", fn, (int)k);
  CAB_REQUIRE(M == 0 || k <= M, CAB_EINVAL, "%s: k=%d exceeds M=%lld", fn, (int)k, (long long)M);
  CAB_REQUIRE(!hybrid || (kmag >= 0 && kmag <= k), CAB_EINVAL,
              "%s: magnitude quota %d outside [0, k=%d]", fn, (int)kmag, (int)k);
  const int64_t rows = B * H * M;
  if (rows == 0) return CAB_OK;
  CAB_REQUIRE(frc && kv_idx && kv_cnt, CAB_EINVAL, "%s: null tensor pointer", fn);
  CAB_REQUIRE(!hybrid || mag, CAB_EINVAL, "%s: null magnitude scores", fn);
  const int64_t blocks = ceil_div(rows, 4);
  CAB_REQUIRE(blocks <= INT32_MAX, CAB_ESHAPE, "%s: problem too large", fn);
  TopkArgs a;
  a.frc = frc;
  a.mag = mag;
  a.kv_idx = kv_idx;
  a.kv_cnt = kv_cnt;
  a.dense = dense_mask;
  a.rows = rows;
  a.M = M;
  a.k = k;
  a.kmag = kmag;
  a.select_high = select_high;
  a.keep_diagonal = keep_diagonal;
  a.causal = causal;
  const dim3 grid(static_cast<unsigned>(blocks));
  if (hybrid)
    launch_topk<true>(a, grid, static_cast<hipStream_t>(stream));
  else
    launch_topk<false>(a, grid, static_cast<hipStream_t>(stream));
  return launch_status(fn);
}

}  // namespace
}  // namespace cab

using namespace cab;

extern "C" cab_status_t cab_block_topk(const float* frc, int64_t B, int64_t H, int64_t M,
                                       int32_t k, int select_high, int keep_diagonal, int causal,
                                       int32_t* kv_idx, int32_t* kv_cnt, uint8_t* dense_mask,
                                       void* stream) {
  return topk_common("cab_block_topk", frc, nullptr, B, H, M, k, 0, select_high, keep_diagonal,
                     causal, kv_idx, kv_cnt, dense_mask, stream, false);
}

extern "C" cab_status_t cab_block_topk_hybrid(const float* frc, const float* magnitude, int64_t B,
                                              int64_t H, int64_t M, int32_t k, int32_t k_mag,
                                              int select_high, int keep_diagonal, int causal,
                                              int32_t* kv_idx, int32_t* kv_cnt,
                                              uint8_t* dense_mask, void* stream) {
  return topk_common("cab_block_topk_hybrid", frc, magnitude, B, H, M, k, k_mag, select_high,
                     keep_diagonal, causal, kv_idx, kv_cnt, dense_mask, stream, true);
}
