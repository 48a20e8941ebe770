// Block-sparse attention forward (cab_block_sparse_attn_fwd), D = 128,
// block_size = 64.
//
// Two kernels:
//  1. pack_vt_kernel: V [B, H, N, D] -> V^T tiles in MFMA operand order
//     (16 KB per (b, h, key block), zero past N), in the caller's workspace.
//     One streaming pass; it moves the transposition MFMA needs for P V out
//     of the attention loop.
//  2. attn_fwd_kernel: one workgroup (4 waves) per (b, h, query block i);
//     wave w owns queries 16 w .. 16 w + 15 of the block. For every kept key
//     block the workgroup stages K and V^T in LDS with gfx950 direct-to-LDS
//     loads (global_load_lds_dwordx4: each lane supplies its own global
//     address, the data lands at LDS base + 16 * lane, so K is gathered
//     straight into MFMA order and staging costs no VALU work), then every
//     wave computes
//       S^T = K Q^T    (16 MFMA 16x16x32: A = K from LDS, B = Q in registers)
//       online softmax in the log2 domain, fp32
//       O^T += V^T P^T (16 MFMA 16x16x32: A = V^T from LDS, B = P in registers)
// Computing the transposed products keeps one query per lane (lane l owns
// query l % 16) in S, P and O alike, so softmax statistics only cross the 4
// lanes of a query, and P feeds the second MFMA straight from the first
// one's accumulators: the k-slots of P^T are the keys
// {32 s + 4 g + r, 32 s + 16 + 4 g + r} (g = lane / 16, r = 0..3), the order
// pack_vt_kernel writes V^T in.
// The accumulator is rescaled only when some query's running maximum grows
// by more than 2^8 (P stays below 256, exact in fp32, the final division by
// the row sum is unchanged). Two LDS stages, one barrier per block; the next
// block's loads are issued right after the barrier and land while the
// current block is computed. Workgroups are mapped so that one XCD runs
// consecutive query blocks of the same heads (their K/V share L2), longest
// causal rows first.
//
// Algorithmic work per kept tile: 4 * 64 * 64 * 128 flops (2 * 64 * 65 * 128
// on a causal diagonal tile). Bound: MFMA.
#include "cab_internal.h"

namespace cab {
namespace {

constexpr int BS = 64;                       // tokens per block
constexpr int HD = 128;                      // head dim
constexpr int TILE_SLOTS = 1024;             // 16-byte slots per operand tile
constexpr size_t TILE_BYTES = TILE_SLOTS * 16;
constexpr float RESCALE_LOG2 = 8.0f;         // lazy rescale threshold (2^8)

typedef __attribute__((address_space(3))) void lds_void;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;  // packed V^T tiles [B*H][M][TILE_SLOTS] x 16 bytes
  uint16_t* o;
  float* lse;
  int64_t qs[3], ks[3], os[3];  // b, h, token strides (elements)
  const int32_t* kv_idx;
  const int32_t* kv_cnt;
  int64_t B, H, N, M;
  int32_t kmax;
  float scale_log2;
  int causal;
};

struct PackArgs {
  const uint16_t* v;
  uint16_t* vt;
  int64_t vs[3];
  int64_t H, N, M;
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

// V^T tile slot (dt, s, L) (index (2 dt + s) * 64 + L) holds, for d = 16 dt + L % 16
// and g = L / 16, the 8 values V[32 s + 4 g + r][d] (r = 0..3) followed by
// V[32 s + 16 + 4 g + r][d] (r = 0..3).
__global__ __launch_bounds__(256) void pack_vt_kernel(PackArgs a) {
  __shared__ uint16_t vs[BS][HD + 8];  // padded rows
  const int64_t bh = blockIdx.y, j = blockIdx.x;
  const int64_t b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const uint16_t* vb = a.v + b * a.vs[0] + h * a.vs[1];
  const int tid = threadIdx.x;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int cid = tid + 256 * r;  // 1024 chunks of 8 values
    const int key = cid >> 4, c = cid & 15;
    const int64_t t = j * BS + key;
    const u32x4 x = t < a.N ? *reinterpret_cast<const u32x4*>(vb + t * a.vs[2] + 8 * c)
                            : u32x4{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x2*>(&vs[key][8 * c]) = u32x2{x[0], x[1]};
    *reinterpret_cast<u32x2*>(&vs[key][8 * c + 4]) = u32x2{x[2], x[3]};
  }
  __syncthreads();
  u32x4* out = reinterpret_cast<u32x4*>(a.vt) + (bh * a.M + j) * TILE_SLOTS;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int slot = tid + 256 * r;
    const int row = slot >> 6, L = slot & 63;
    const int dt = row >> 1, s = row & 1, g = L >> 4;
    const int d = 16 * dt + (L & 15);
    const int k0 = 32 * s + 4 * g;
    u32x4 x;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      x[2 * p + 0] = static_cast<uint32_t>(vs[k0 + 16 * p + 0][d]) |
                     (static_cast<uint32_t>(vs[k0 + 16 * p + 1][d]) << 16);
      x[2 * p + 1] = static_cast<uint32_t>(vs[k0 + 16 * p + 2][d]) |
                     (static_cast<uint32_t>(vs[k0 + 16 * p + 3][d]) << 16);
    }
    out[slot] = x;
  }
}

// Issues the direct-to-LDS loads of key block j into one stage: wave w
// fetches K slot rows (tt = w, ds = 0..3) and V^T slot rows 4 w .. 4 w + 3.
// K slot (tt, ds, L) = K[16 tt + L % 16][32 ds + 8 (L / 16) .. +8]; rows past N
// are clamped to N - 1 (their scores are masked).
__device__ __forceinline__ void issue_tile(const AttnArgs& a, const uint16_t* kb, const u32x4* vtb,
                                           int64_t j, u32x4* kst, u32x4* vst) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  int64_t tk = j * BS + 16 * w + (l & 15);
  tk = tk < a.N ? tk : a.N - 1;
  const uint16_t* kp = kb + tk * a.ks[2] + 8 * (l >> 4);
  const u32x4* vp = vtb + j * TILE_SLOTS + w * 256 + l;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    __builtin_amdgcn_global_load_lds(kp + 32 * r, (lds_void*)(kst + (w * 4 + r) * 64), 16, 0, 0);
#pragma unroll
  for (int r = 0; r < 4; ++r)
    __builtin_amdgcn_global_load_lds(vp + 64 * r, (lds_void*)(vst + (w * 4 + r) * 64), 16, 0, 0);
}

// Pulls key block j's 256 cache lines (128 of K rows, 128 of its V^T tile)
// into L2 ahead of its staging loads: one 16-byte load per lane, each lane a
// different 128-byte line, landing in a scratch LDS row nobody reads.
__device__ __forceinline__ void prefetch_tile(const AttnArgs& a, const uint16_t* kb,
                                              const u32x4* vtb, int64_t j, u32x4* junk) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int line = 64 * w + l;
  const void* p;
  if (line < 128) {
    int64_t tk = j * BS + (line >> 1);
    tk = tk < a.N ? tk : a.N - 1;
    p = kb + tk * a.ks[2] + 64 * (line & 1);
  } else {
    p = vtb + j * TILE_SLOTS + 8 * (line - 128);
  }
  __builtin_amdgcn_global_load_lds(p, (lds_void*)junk, 16, 0, 0);
}

// Waits until at most n of this wave's vector-memory operations are pending.
__device__ __forceinline__ void wait_vmcnt(int n) {
  if (n <= 0)
    __builtin_amdgcn_s_waitcnt(0x0f70);
  else if (n == 1)
    __builtin_amdgcn_s_waitcnt(0x0f71);
  else
    __builtin_amdgcn_s_waitcnt(0x0f72);
}

constexpr int LIST_MAX = 2048;  // kv lists up to this length are staged in LDS
constexpr int PREFETCH = 3;     // L2 prefetch distance in key blocks

template <bool BF16, bool LIST_LDS>
__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnArgs a) {
  // One LDS object: [stage 0: K, V^T][stage 1: K, V^T][prefetch landing row][list].
  __shared__ u32x4 smem[4 * TILE_SLOTS + 64 + LIST_MAX / 4];
  auto stage_k = [&](int s) { return smem + 2 * s * TILE_SLOTS; };
  auto stage_v = [&](int s) { return smem + (2 * s + 1) * TILE_SLOTS; };
  u32x4* junk = smem + 4 * TILE_SLOTS;
  int32_t* slist = reinterpret_cast<int32_t*>(smem + 4 * TILE_SLOTS + 64);

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
  const u32x4* vtb = reinterpret_cast<const u32x4*>(a.vt) + bh * a.M * TILE_SLOTS;

  const int64_t row = bh * a.M + i;
  int cnt = a.kv_cnt[row];
  cnt = cnt < 0 ? 0 : (cnt > a.kmax ? a.kmax : cnt);
  const int32_t* glist = a.kv_idx + row * a.kmax;
  if constexpr (LIST_LDS) {
    for (int p = threadIdx.x; p < cnt; p += 256) slist[p] = glist[p];
    __syncthreads();
  }
  // Entry p of the list; an entry outside [0, M) becomes block 0 with every
  // score masked, so the pipeline below never branches on validity.
  auto entry = [&](int p) -> int64_t {
    if constexpr (LIST_LDS)
      return slist[p];
    else
      return glist[p];
  };
  auto block_of = [&](int64_t j) -> int64_t { return (j >= 0 && j < a.M) ? j : 0; };

  // Q^T as the B operand: lane holds Q[qtok][32 ds + 8 g .. +8]. Issue order:
  // block 0's staging loads, Q, then the first prefetches; the empty asm makes
  // Q ready here (it waits past the prefetches only), so no wait for Q is left
  // inside the loop where it would also stall on the next block's loads.
  u32x4 qreg[4];
  int pre = 0;  // prefetches issued before the loop, after block 0's loads
  if (cnt > 0) issue_tile(a, kb, vtb, block_of(entry(0)), stage_k(0), stage_v(0));
#pragma unroll
  for (int ds = 0; ds < 4; ++ds)
    qreg[ds] = qtok < a.N ? *reinterpret_cast<const u32x4*>(qb + qtok * a.qs[2] + 32 * ds + 8 * g)
                          : u32x4{0u, 0u, 0u, 0u};
  for (int p = 1; p < PREFETCH && p < cnt; ++p, ++pre)
    prefetch_tile(a, kb, vtb, block_of(entry(p)), junk);
  asm volatile("" ::"v"(qreg[0]), "v"(qreg[1]), "v"(qreg[2]), "v"(qreg[3]));

  f32x4 acc_o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc_o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float c = a.scale_log2;
  float m_run = -INFINITY;  // running max of the raw scores this lane's query saw
  float l_run = 0.f;        // partial row sum of exp2((s - m_run) c) over this lane's keys
  // One key block; ST (compile-time) is the LDS stage holding it, so the
  // compiler sees that the loads into stage ST ^ 1 cannot alias its reads.
  auto step = [&](int p, auto stage_tag) {
    constexpr int ST = decltype(stage_tag)::value;
    const int64_t jraw = entry(p);
    const bool valid = jraw >= 0 && jraw < a.M;
    const int64_t j = valid ? jraw : 0;
    // Block p's loads were followed by the prefetches issued after them.
    wait_vmcnt(p == 0 ? pre : (p + PREFETCH - 1 < cnt ? 1 : 0));
    __builtin_amdgcn_s_barrier();  // every wave's loads of block p landed; stage ST^1 is free
    if (p + 1 < cnt) issue_tile(a, kb, vtb, block_of(entry(p + 1)), stage_k(ST ^ 1), stage_v(ST ^ 1));
    if (p + PREFETCH < cnt) prefetch_tile(a, kb, vtb, block_of(entry(p + PREFETCH)), junk);
    const u32x4* ks = stage_k(ST);
    const u32x4* vts = stage_v(ST);
    // S^T[key][query] for the block's 64 keys: lane holds keys 16 tt + 4 g + r.
    f32x4 sc[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) acc = mfma16<BF16>(ks[(tt * 4 + ds) * 64 + lane], qreg[ds], acc);
      sc[tt] = acc;
    }
    if (!valid || (a.causal && j >= i) || (j + 1) * BS > a.N) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t ktok = j * BS + 16 * tt + 4 * g + r;
          if (!valid || ktok >= a.N || (a.causal && ktok > qtok)) sc[tt][r] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sc[tt][r]);
    mx = fmaxf(mx, shfl_xor_f32(mx, 16));
    mx = fmaxf(mx, shfl_xor_f32(mx, 32));
    // Raise the reference point only when P would exceed 2^8 (or on first sight).
    const bool grow = mx > m_run && (m_run == -INFINITY || (mx - m_run) * c > RESCALE_LOG2);
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float m_new = grow ? mx : m_run;
      const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m_run - m_new) * c);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc_o[dt] *= alpha;
      m_run = m_new;
    }
    const float mc = m_run == -INFINITY ? 0.f : m_run * c;
    float psum = 0.f;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[tt][r], c, -mc));
        sc[tt][r] = pv;
        psum += pv;
      }
    l_run += psum;

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
        acc_o[dt] = mfma16<BF16>(vts[(dt * 2 + s) * 64 + lane], pb[s], acc_o[dt]);
  };
  for (int p = 0; p < cnt; p += 2) {
    step(p, std::integral_constant<int, 0>{});
    if (p + 1 < cnt) step(p + 1, std::integral_constant<int, 1>{});
  }
  wait_vmcnt(0);  // drain the scratch prefetches before the workgroup exits

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
          l_tot > 0.f ? (m_run * c + __log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
    }
  }
}

}  // namespace
}  // namespace cab

using namespace cab;

extern "C" size_t cab_block_sparse_attn_workspace_bytes(int64_t B, int64_t H, int64_t N,
                                                        int64_t D, int32_t block_size) {
  if (B <= 0 || H <= 0 || N <= 0 || D != HD || block_size != BS) return 0;
  return static_cast<size_t>(B * H * ceil_div(N, BS)) * TILE_BYTES;
}

extern "C" cab_status_t cab_block_sparse_attn_fwd(
    const void* q, const void* k, const void* v, cab_dtype_t dtype, int64_t B, int64_t H,
    int64_t N, int64_t D, const int64_t q_strides[4], const int64_t k_strides[4],
    const int64_t v_strides[4], const int64_t o_strides[4], int32_t block_size,
    const int32_t* kv_idx, const int32_t* kv_cnt, int32_t kmax, float scale, int causal,
    void* out, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  CAB_REQUIRE(dtype == CAB_BF16 || dtype == CAB_F16, CAB_EDTYPE,
              "cab_block_sparse_attn_fwd: dtype %d unsupported (bf16 or fp16)", (int)dtype);
  CAB_REQUIRE(B >= 0 && H >= 0 && N >= 0, CAB_ESHAPE, "cab_block_sparse_attn_fwd: negative size");
  CAB_REQUIRE(D == HD, CAB_ESHAPE, "cab_block_sparse_attn_fwd: head dim %lld unsupported (128)",
              (long long)D);
  CAB_REQUIRE(block_size == BS, CAB_ESHAPE,
              "cab_block_sparse_attn_fwd: block_size %d unsupported (64)", (int)block_size);
  CAB_REQUIRE(kmax >= 1, CAB_EINVAL, "cab_block_sparse_attn_fwd: kmax=%d must be >= 1", (int)kmax);
  CAB_REQUIRE(std::isfinite(scale) && scale > 0.f, CAB_EINVAL,
              "cab_block_sparse_attn_fwd: scale must be finite and > 0");
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
  const size_t need = static_cast<size_t>(B * H * M) * TILE_BYTES;
  CAB_REQUIRE(workspace != nullptr && workspace_bytes >= need, CAB_EWORKSPACE,
              "cab_block_sparse_attn_fwd: workspace of %zu bytes given, %zu needed",
              workspace_bytes, need);
  CAB_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, CAB_EWORKSPACE,
              "cab_block_sparse_attn_fwd: workspace not 16-byte aligned");
  const int64_t total = B * H * M;
  CAB_REQUIRE(total <= INT32_MAX && B * H <= 65535, CAB_ESHAPE,
              "cab_block_sparse_attn_fwd: problem too large (B*H <= 65535, B*H*M < 2^31)");
  hipStream_t s = static_cast<hipStream_t>(stream);

  PackArgs p;
  p.v = static_cast<const uint16_t*>(v);
  p.vt = static_cast<uint16_t*>(workspace);
  for (int d = 0; d < 3; ++d) p.vs[d] = v_strides[d];
  p.H = H;
  p.N = N;
  p.M = M;
  pack_vt_kernel<<<dim3(static_cast<unsigned>(M), static_cast<unsigned>(B * H)), 256, 0, s>>>(p);
  cab_status_t st = launch_status("cab_block_sparse_attn_fwd/pack_vt");
  if (st != CAB_OK) return st;

  AttnArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.vt = static_cast<const uint16_t*>(workspace);
  a.o = static_cast<uint16_t*>(out);
  a.lse = lse;
  for (int d = 0; d < 3; ++d) {
    a.qs[d] = q_strides[d];
    a.ks[d] = k_strides[d];
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
  dim3 grid(static_cast<unsigned>(total));
  const bool list_lds = kmax <= LIST_MAX;
  if (dtype == CAB_BF16) {
    if (list_lds)
      attn_fwd_kernel<true, true><<<grid, 256, 0, s>>>(a);
    else
      attn_fwd_kernel<true, false><<<grid, 256, 0, s>>>(a);
  } else {
    if (list_lds)
      attn_fwd_kernel<false, true><<<grid, 256, 0, s>>>(a);
    else
      attn_fwd_kernel<false, false><<<grid, 256, 0, s>>>(a);
  }
  return launch_status("cab_block_sparse_attn_fwd");
}
