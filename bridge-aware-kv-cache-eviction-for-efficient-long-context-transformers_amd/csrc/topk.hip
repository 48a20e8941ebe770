// Per-row block selection (cab_block_topk).
//
// One wave64 per FRC row. The row's M scores are read once (coalesced, lane l
// holds columns j = 64 c + l) and mapped to order-preserving uint32 keys in
// registers. The k-th smallest key is found by a 32-step bitwise search: each
// step counts the candidates below a trial threshold with one ballot +
// popcount per register, so all lanes agree on every decision without LDS.
// A last pass in ascending j keeps every key below the threshold and the
// first (in j) keys equal to it, assigns output slots with a prefix
// popcount, and writes the compact ascending index list and, optionally, the
// dense 0/1 row.
//
// HBM traffic per row: 4 M bytes read; 4 k + 4 (+ M for the dense mask)
// bytes written. Bound by HBM bandwidth.
#include "cab_internal.h"

namespace cab {
namespace {

struct TopkArgs {
  const float* frc;
  int32_t* kv_idx;
  int32_t* kv_cnt;
  uint8_t* dense;
  int64_t rows, M;
  int32_t k;
  int select_high, keep_diagonal, causal;
};

// Ascending key order == selection order: float order with -0 == +0 and NaN
// above +inf, inverted when the highest scores are wanted.
__device__ __forceinline__ uint32_t order_key(float f, bool high) {
  uint32_t u = __float_as_uint(f);
  if (f == 0.f) u = 0u;
  if (isnan(f)) u = 0x7fc00000u;
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return high ? ~u : u;
}

template <int NCH>
__global__ __launch_bounds__(256) void topk_kernel(TopkArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // uniform per wave
  const int lane = lane_id();
  const int64_t i = row % a.M;
  const int64_t ncand = a.causal ? i + 1 : a.M;
  const int64_t krow = min(static_cast<int64_t>(a.k), ncand);
  const bool kd = a.keep_diagonal != 0;
  const int64_t need = kd ? krow - 1 : krow;
  const float* f = a.frc + row * a.M;
  const bool high = a.select_high != 0;

  uint32_t key[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t j = 64 * c + lane;
    key[c] = j < a.M ? order_key(f[j], high) : 0xffffffffu;
  }
  auto is_cand = [&](int c) {
    const int64_t j = 64 * c + lane;
    return j < ncand && !(kd && j == i);
  };

  // theta = need-th smallest candidate key (largest theta with
  // count(key < theta) < need).
  uint32_t theta = 0u;
  int64_t need_eq = 0;
  if (need > 0) {
    for (int b = 31; b >= 0; --b) {
      const uint32_t trial = theta | (1u << b);
      int64_t cnt = 0;
#pragma unroll
      for (int c = 0; c < NCH; ++c) cnt += __popcll(ballot64(is_cand(c) && key[c] < trial));
      if (cnt < need) theta = trial;
    }
    int64_t below = 0;
#pragma unroll
    for (int c = 0; c < NCH; ++c) below += __popcll(ballot64(is_cand(c) && key[c] < theta));
    need_eq = need - below;
  }

  int64_t pos = 0, eq_seen = 0;
  const uint64_t lt_mask = lanemask_lt();
  int32_t* out = a.kv_idx + row * a.k;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t j = 64 * c + lane;
    const bool cand = is_cand(c);
    const bool eq = cand && need > 0 && key[c] == theta;
    const uint64_t eqb = ballot64(eq);
    const int64_t eq_rank = eq_seen + __popcll(eqb & lt_mask);
    const bool sel = (cand && need > 0 && key[c] < theta) || (eq && eq_rank < need_eq) ||
                     (kd && j == i);
    const uint64_t selb = ballot64(sel);
    if (sel) out[pos + __popcll(selb & lt_mask)] = static_cast<int32_t>(j);
    if (a.dense && j < a.M) a.dense[row * a.M + j] = sel ? 1 : 0;
    pos += __popcll(selb);
    eq_seen += __popcll(eqb);
  }
  for (int64_t p = pos + lane; p < a.k; p += 64) out[p] = -1;
  if (lane == 0) a.kv_cnt[row] = static_cast<int32_t>(pos);
}

}  // namespace
}  // namespace cab

using namespace cab;

extern "C" cab_status_t cab_block_topk(const float* frc, int64_t B, int64_t H, int64_t M,
                                       int32_t k, int select_high, int keep_diagonal, int causal,
                                       int32_t* kv_idx, int32_t* kv_cnt, uint8_t* dense_mask,
                                       void* stream) {
  clear_error();
  CAB_REQUIRE(B >= 0 && H >= 0 && M >= 0, CAB_ESHAPE, "cab_block_topk: negative size");
  CAB_REQUIRE(M <= 8192, CAB_ESHAPE, "cab_block_topk: M=%lld exceeds 8192", (long long)M);
  CAB_REQUIRE(k >= 1, CAB_EINVAL, "cab_block_topk: k=%d must be >= 1", (int)k);
  CAB_REQUIRE(M == 0 || k <= M, CAB_EINVAL, "cab_block_topk: k=%d exceeds M=%lld", (int)k,
              (long long)M);
  const int64_t rows = B * H * M;
  if (rows == 0) return CAB_OK;
  CAB_REQUIRE(frc && kv_idx && kv_cnt, CAB_EINVAL, "cab_block_topk: null tensor pointer");
  const int64_t blocks = ceil_div(rows, 4);
  CAB_REQUIRE(blocks <= INT32_MAX, CAB_ESHAPE, "cab_block_topk: problem too large");
  TopkArgs a;
  a.frc = frc;
  a.kv_idx = kv_idx;
  a.kv_cnt = kv_cnt;
  a.dense = dense_mask;
  a.rows = rows;
  a.M = M;
  a.k = k;
  a.select_high = select_high;
  a.keep_diagonal = keep_diagonal;
  a.causal = causal;
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(blocks));
  const int64_t nch = ceil_div(M, 64);
  if (nch <= 1) topk_kernel<1><<<grid, 256, 0, s>>>(a);
  else if (nch <= 2) topk_kernel<2><<<grid, 256, 0, s>>>(a);
  else if (nch <= 4) topk_kernel<4><<<grid, 256, 0, s>>>(a);
  else if (nch <= 8) topk_kernel<8><<<grid, 256, 0, s>>>(a);
  else if (nch <= 16) topk_kernel<16><<<grid, 256, 0, s>>>(a);
  else if (nch <= 32) topk_kernel<32><<<grid, 256, 0, s>>>(a);
  else if (nch <= 64) topk_kernel<64><<<grid, 256, 0, s>>>(a);
  else topk_kernel<128><<<grid, 256, 0, s>>>(a);
  return launch_status("cab_block_topk");
}
