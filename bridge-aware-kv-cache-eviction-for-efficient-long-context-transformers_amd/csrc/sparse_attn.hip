// Block-sparse attention forward (cab_block_sparse_attn_fwd), D = 128,
// block_size = 64.
//
// One workgroup (4 waves) per (b, h, query block i); wave w owns queries
// 16 w .. 16 w + 15 of the block. The workgroup walks the kept key blocks
// kv_idx[b, h, i, :cnt] and, per 64-key block, every wave computes
//   S^T = K Q^T   (16 MFMA 16x16x32: A = K from LDS, B = Q in registers)
//   online softmax in the log2 domain, fp32
//   O^T += V^T P^T (16 MFMA 16x16x32: A = V^T from LDS, B = P in registers)
// Computing the transposed products keeps one query per lane (lane l owns
// query l % 16) in S, P and O alike, so the softmax statistics never cross
// lanes except for the 4-lane row reductions, and P feeds the second MFMA
// straight from the first one's accumulators: the k-slots of P^T are the
// keys {32 s + 4 g + r, 32 s + 16 + 4 g + r} (g = lane / 16, r = 0..3) and V^T
// is staged in LDS in the same key order.
//
// Both operand tiles sit in LDS in MFMA order (16 bytes per lane and slot),
// so every operand read is one contiguous 1 KB wave access. The next block's
// K and V are loaded into registers while the current block is computed
// (two LDS stages, one barrier per block). Workgroups are mapped so that one
// XCD runs consecutive query blocks of the same heads (their K/V share L2),
// longest rows first.
//
// Algorithmic work per kept tile: 4 * 64 * 64 * 128 flops (2 * 64 * 65 * 128
// on a causal diagonal tile). Bound: MFMA.
#include "cab_internal.h"

namespace cab {
namespace {

constexpr int BS = 64;   // tokens per block
constexpr int HD = 128;  // head dim

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t qs[3], ks[3], vs[3], os[3];  // b, h, token strides (elements)
  const int32_t* kv_idx;
  const int32_t* kv_cnt;
  int64_t B, H, N, M;
  int32_t kmax;
  float scale_log2;
  int causal;
};

template <bool BF16>
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (BF16) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};  // v_cvt_pk_bf16_f32, RNE
    return __builtin_bit_cast(uint32_t, v);
  } else {
    return static_cast<uint32_t>(f32_to_f16(lo)) | (static_cast<uint32_t>(f32_to_f16(hi)) << 16);
  }
}

// Global -> register staging of one key block (rows beyond N read as 0).
struct KVRegs {
  u32x4 k[4];  // K[16 w + l % 16][32 r + 8 (l / 16) .. +8] for wave w, lane l, r = 0..3
  u32x4 v[4];  // V rows 4 kq + r at d = 8 c, kq = tid / 16, c = tid % 16
};

__device__ __forceinline__ void load_kv(const AttnArgs& a, const uint16_t* kb, const uint16_t* vb,
                                        int64_t j, KVRegs& R) {
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int64_t tok0 = j * BS;
  const int64_t tk = tok0 + 16 * w + (l & 15);
#pragma unroll
  for (int r = 0; r < 4; ++r)
    R.k[r] = tk < a.N ? *reinterpret_cast<const u32x4*>(kb + tk * a.ks[2] + 32 * r + 8 * (l >> 4))
                      : u32x4{0u, 0u, 0u, 0u};
  const int kq = tid >> 4, c = tid & 15;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t t = tok0 + 4 * kq + r;
    R.v[r] = t < a.N ? *reinterpret_cast<const u32x4*>(vb + t * a.vs[2] + 8 * c) : u32x4{0u, 0u, 0u, 0u};
  }
}

// Register -> LDS in MFMA operand order.
//  K slot (tt, ds, lane'): key 16 tt + lane' % 16, d = 32 ds + 8 (lane' / 16) .. +8. Wave w
//    writes block tt = w, so every store is one linear 1 KB wave access.
//  V^T slot (dt, s, lane'): d = 16 dt + lane' % 16; 8 bytes per half:
//    half 0 = keys 32 s + 4 g + 0..3, half 1 = keys 32 s + 16 + 4 g + 0..3, g = lane' / 16.
//    Stored at lane' ^ dt within its 64-slot row: the transposing 8-byte stores of one
//    wave then spread over 16 bank groups instead of 2, and a row read stays a
//    permutation of one contiguous 1 KB block (conflict-free).
__device__ __forceinline__ void store_kv(u32x4* ks, u32x4* vts, const KVRegs& R) {
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
#pragma unroll
  for (int r = 0; r < 4; ++r) ks[(w * 4 + r) * 64 + l] = R.k[r];
  const int kq = tid >> 4, c = tid & 15;
  const int key0 = 4 * kq;
  const int s = key0 >> 5, rem = key0 & 31;
  const int hf = rem >> 4, g = (rem & 15) >> 2;
  char* vbytes = reinterpret_cast<char*>(vts);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int wd = e >> 1;
    uint32_t x0, x1;
    if ((e & 1) == 0) {
      x0 = (R.v[0][wd] & 0xffffu) | (R.v[1][wd] << 16);
      x1 = (R.v[2][wd] & 0xffffu) | (R.v[3][wd] << 16);
    } else {
      x0 = (R.v[0][wd] >> 16) | (R.v[1][wd] & 0xffff0000u);
      x1 = (R.v[2][wd] >> 16) | (R.v[3][wd] & 0xffff0000u);
    }
    const int d = 8 * c + e;
    const int dt = d >> 4, lanep = ((d & 15) + 16 * g) ^ dt;
    *reinterpret_cast<u32x2*>(vbytes + ((dt * 2 + s) * 64 + lanep) * 16 + hf * 8) = u32x2{x0, x1};
  }
}

template <bool BF16>
__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnArgs a) {
  __shared__ u32x4 lds[2][2][1024];  // [stage][K, V^T][slot]: 64 KB

  const int64_t total = a.B * a.H * a.M;
  const int64_t logical = xcd_remap(blockIdx.x, total);
  const int64_t bh = logical / a.M;
  const int64_t i = a.M - 1 - (logical - bh * a.M);  // longest causal rows first
  const int64_t b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int w = threadIdx.x >> 6, lane = lane_id();
  const int g = lane >> 4;
  const int qi = lane & 15;
  const int64_t qtok = i * BS + 16 * w + qi;

  const uint16_t* qb = a.q + b * a.qs[0] + h * a.qs[1];
  const uint16_t* kb = a.k + b * a.ks[0] + h * a.ks[1];
  const uint16_t* vb = a.v + b * a.vs[0] + h * a.vs[1];

  // Q^T as the B operand: lane holds Q[qtok][32 ds + 8 g .. +8].
  u32x4 qreg[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds)
    qreg[ds] = qtok < a.N ? *reinterpret_cast<const u32x4*>(qb + qtok * a.qs[2] + 32 * ds + 8 * g)
                          : u32x4{0u, 0u, 0u, 0u};

  const int64_t row = bh * a.M + i;
  int cnt = a.kv_cnt[row];
  cnt = cnt < 0 ? 0 : (cnt > a.kmax ? a.kmax : cnt);
  const int32_t* list = a.kv_idx + row * a.kmax;

  f32x4 acc_o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc_o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  int stage = 0;

  auto fetch = [&](int n, KVRegs& R) {
    const int64_t j = list[n];
    if (j >= 0 && j < a.M) load_kv(a, kb, vb, j, R);
  };

  auto compute = [&](int64_t j, const u32x4* ks, const u32x4* vts) {
    // S^T[key][query] for the block's 64 keys.
    f32x4 sc[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) acc = mfma16<BF16>(ks[(tt * 4 + ds) * 64 + lane], qreg[ds], acc);
      sc[tt] = acc;
    }
    const bool need_mask = (a.causal && j >= i) || (j + 1) * BS > a.N;
    float mx = -INFINITY;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float sv = sc[tt][r] * a.scale_log2;
        if (need_mask) {
          const int64_t ktok = j * BS + 16 * tt + 4 * g + r;
          if (ktok >= a.N || (a.causal && ktok > qtok)) sv = -INFINITY;
        }
        sc[tt][r] = sv;
        mx = fmaxf(mx, sv);
      }
    mx = fmaxf(mx, shfl_xor_f32(mx, 16));
    mx = fmaxf(mx, shfl_xor_f32(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float psum = 0.f;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = __builtin_amdgcn_exp2f(sc[tt][r] - m_use);
        sc[tt][r] = p;
        psum += p;
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc_o[dt] *= alpha;

    // P^T as the B operand, k-slots {32 s + 4 g + r, 32 s + 16 + 4 g + r}.
    u32x4 pb[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      pb[s][0] = pack2<BF16>(sc[2 * s][0], sc[2 * s][1]);
      pb[s][1] = pack2<BF16>(sc[2 * s][2], sc[2 * s][3]);
      pb[s][2] = pack2<BF16>(sc[2 * s + 1][0], sc[2 * s + 1][1]);
      pb[s][3] = pack2<BF16>(sc[2 * s + 1][2], sc[2 * s + 1][3]);
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        acc_o[dt] = mfma16<BF16>(vts[(dt * 2 + s) * 64 + (lane ^ dt)], pb[s], acc_o[dt]);
  };

  // Two blocks in flight in registers: block n is stored to LDS while block
  // n + 1 is still arriving; block n + 2 is requested as soon as n's
  // registers are free.
  auto step = [&](int n, KVRegs& R) {
    const int64_t j = list[n];
    const bool valid = j >= 0 && j < a.M;  // uniform over the workgroup
    if (valid) {
      store_kv(lds[stage][0], lds[stage][1], R);
      __syncthreads();
    }
    if (n + 2 < cnt) fetch(n + 2, R);
    if (valid) {
      compute(j, lds[stage][0], lds[stage][1]);
      stage ^= 1;
    }
  };

  KVRegs R0, R1;
  if (cnt > 0) fetch(0, R0);
  if (cnt > 1) fetch(1, R1);
  for (int n = 0; n < cnt; n += 2) {
    step(n, R0);
    if (n + 1 < cnt) step(n + 1, R1);
  }

  float l_tot = l_run + shfl_xor_f32(l_run, 16);
  l_tot = l_tot + shfl_xor_f32(l_tot, 32);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (qtok < a.N) {
    uint16_t* ob = a.o + b * a.os[0] + h * a.os[1] + qtok * a.os[2];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const u32x2 pk = {pack2<BF16>(acc_o[dt][0] * inv, acc_o[dt][1] * inv),
                        pack2<BF16>(acc_o[dt][2] * inv, acc_o[dt][3] * inv)};
      *reinterpret_cast<u32x2*>(ob + 16 * dt + 4 * g) = pk;
    }
    if (a.lse && g == 0) {
      a.lse[bh * a.N + qtok] =
          l_tot > 0.f ? (m_run + __log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
    }
  }
}

}  // namespace
}  // namespace cab

using namespace cab;

extern "C" cab_status_t cab_block_sparse_attn_fwd(
    const void* q, const void* k, const void* v, cab_dtype_t dtype, int64_t B, int64_t H,
    int64_t N, int64_t D, const int64_t q_strides[4], const int64_t k_strides[4],
    const int64_t v_strides[4], const int64_t o_strides[4], int32_t block_size,
    const int32_t* kv_idx, const int32_t* kv_cnt, int32_t kmax, float scale, int causal,
    void* out, float* lse, void* stream) {
  clear_error();
  CAB_REQUIRE(dtype == CAB_BF16 || dtype == CAB_F16, CAB_EDTYPE,
              "cab_block_sparse_attn_fwd: dtype %d unsupported (bf16 or fp16)", (int)dtype);
  CAB_REQUIRE(B >= 0 && H >= 0 && N >= 0, CAB_ESHAPE, "cab_block_sparse_attn_fwd: negative size");
  CAB_REQUIRE(D == HD, CAB_ESHAPE, "cab_block_sparse_attn_fwd: head dim %lld unsupported (128)",
              (long long)D);
  CAB_REQUIRE(block_size == BS, CAB_ESHAPE,
              "cab_block_sparse_attn_fwd: block_size %d unsupported (64)", (int)block_size);
  CAB_REQUIRE(kmax >= 1, CAB_EINVAL, "cab_block_sparse_attn_fwd: kmax=%d must be >= 1", (int)kmax);
  CAB_REQUIRE(std::isfinite(scale), CAB_EINVAL, "cab_block_sparse_attn_fwd: scale not finite");
  CAB_REQUIRE(q_strides && k_strides && v_strides && o_strides, CAB_EINVAL,
              "cab_block_sparse_attn_fwd: null stride array");
  const int64_t M = ceil_div(N, BS);
  if (B == 0 || H == 0 || M == 0) return CAB_OK;
  CAB_REQUIRE(q && k && v && out && kv_idx && kv_cnt, CAB_EINVAL,
              "cab_block_sparse_attn_fwd: null tensor pointer");
  const void* ptrs[4] = {q, k, v, out};
  const int64_t* strides[4] = {q_strides, k_strides, v_strides, o_strides};
  const char* names[4] = {"q", "k", "v", "out"};
  for (int t = 0; t < 4; ++t) {
    CAB_REQUIRE(strides[t][3] == 1, CAB_ESHAPE,
                "cab_block_sparse_attn_fwd: %s last-dim stride must be 1", names[t]);
    CAB_REQUIRE(reinterpret_cast<uintptr_t>(ptrs[t]) % 16 == 0, CAB_ESHAPE,
                "cab_block_sparse_attn_fwd: %s not 16-byte aligned", names[t]);
    for (int d = 0; d < 3; ++d)
      CAB_REQUIRE(strides[t][d] >= 0 && (strides[t][d] * 2) % 16 == 0, CAB_ESHAPE,
                  "cab_block_sparse_attn_fwd: %s stride[%d]=%lld must keep rows 16-byte aligned",
                  names[t], d, (long long)strides[t][d]);
  }
  const int64_t total = B * H * M;
  CAB_REQUIRE(total <= INT32_MAX, CAB_ESHAPE, "cab_block_sparse_attn_fwd: problem too large");
  AttnArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<uint16_t*>(out);
  a.lse = lse;
  for (int d = 0; d < 3; ++d) {
    a.qs[d] = q_strides[d];
    a.ks[d] = k_strides[d];
    a.vs[d] = v_strides[d];
    a.os[d] = o_strides[d];
  }
  a.kv_idx = kv_idx;
  a.kv_cnt = kv_cnt;
  a.B = B;
  a.H = H;
  a.N = N;
  a.M = M;
  a.kmax = kmax;
  a.scale_log2 = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
  a.causal = causal ? 1 : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(total));
  if (dtype == CAB_BF16)
    attn_fwd_kernel<true><<<grid, 256, 0, s>>>(a);
  else
    attn_fwd_kernel<false><<<grid, 256, 0, s>>>(a);
  return launch_status("cab_block_sparse_attn_fwd");
}
