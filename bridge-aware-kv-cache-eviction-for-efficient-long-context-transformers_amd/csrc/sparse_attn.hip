// Block-sparse attention forward (cab_block_sparse_attn_fwd), head dim
// D = 64 or 128 (a template parameter of every kernel below), block_size = 64.
// The comments give the D = 128 sizes; D = 64 halves every per-block byte
// count, the k-steps of S^T and the O^T tiles.
//
// Two kernels:
//  1. pack_vt_kernel: V [B, H, N, D] -> V^T tiles in MFMA operand order
//     (16 KB per (b, h, key block), zero past N), in the caller's workspace.
//     One streaming pass; it moves the transposition MFMA needs for P V out
//     of the attention loop.
//  2. attn_fwd_kernel: one workgroup of 4 waves per (b, h, query block i),
//     two workgroups per CU. Wave (kh, qh) owns key half kh (keys 32 kh ..
//     32 kh + 31) of every kept key block and query half qh (32 queries).
//     The 4 waves stage each kept key block (K rows and the packed V^T tile,
//     32 KB) into one of two LDS stages with 16-byte buffer loads to LDS,
//     one block ahead: the loads of block p + 1 are issued two at a time
//     between the score MFMAs of block p (a load waits for a free slot in the
//     CU's 64 B/clk load path; spread out, the wait does not hold MFMAs back).
//     Per block each wave reads its K half and V^T half from LDS and computes
//       S^T = K_kh Q^T    (16 MFMA 16x16x32: A = K rows, B = Q in registers)
//       online softmax over its 32 keys, fp32, log2 domain
//       O^T += V_kh^T P^T (16 MFMA 16x16x32: A = packed V^T, B = P)
//       row sums = 1 P^T  (2 MFMA: the sums of exactly the bf16 P used above)
//     The two key halves keep separate running maxima, sums and accumulators
//     (a split of the key dimension), merged once at the end through LDS.
//     One barrier per block hands a stage from the waves that read it to
//     the waves that refill it.
// Transposed products keep the query on the lane axis: lane l holds queries
// 32 qh + 16 qt + l % 16 (qt = 0, 1) in S, P and O alike. S^T's accumulator already
// is the P^T B operand with k-slots {4 g + r, 16 + 4 g + r} (g = lane / 16,
// r = 0..3), the key order pack_vt_kernel writes V^T in. Column maxima use
// gfx950's lane swaps (v_permlane16/32_swap), not LDS.
// The accumulator is rescaled only when a query's running maximum grows by
// more than 2^8 (P stays below 256; the final division by the row sum is
// unchanged).
// Workgroups are mapped so that one XCD runs consecutive query blocks of the
// same heads (their K/V share L2), longest causal rows first.
//
// fp32 inputs run the same kernel on bf16 MFMA with every operand split in
// two, x = hi + lo (hi = bf16(x), lo = bf16(x - hi), RNE), and three products
// per MFMA site: a b ~ a_hi b_hi + a_lo b_hi + a_hi b_lo (the dropped
// a_lo b_lo and the rounding of lo leave a relative error near 2^-16 per
// product). pack_split_kernel writes each key block's K and V^T halves as
// one 64 KB image (the exact LDS layout of a stage); the attention kernel
// then runs one workgroup per CU with 64 KB stages and writes fp32 output.
//
// Algorithmic work per kept tile: 4 * 64 * 64 * 128 flops (2 * 64 * 65 * 128
// on a causal diagonal tile). Bound: MFMA.
#include <cstdlib>

#include "cab_internal.h"

namespace cab {
namespace {

constexpr int BS = 64;                       // tokens per block
constexpr float RESCALE_LOG2 = 8.0f;         // lazy rescale threshold (2^8)
constexpr int LIST_MAX = 2048;               // kv lists up to this length are staged in LDS

// Sizes that follow from the head dim HD (64 or 128).
template <int HD>
struct Dims {
  static_assert(HD == 64 || HD == 128, "head dim 64 or 128");
  static constexpr int CPR = HD / 8;                // 16-byte chunks per 16-bit K row
  static constexpr int ROW_BYTES = 2 * HD;          // one 16-bit K row
  static constexpr int NDS = HD / 32;               // 32-deep k-steps of S^T = K Q^T
  static constexpr int NDT = HD / 16;               // 16-row tiles of O^T
  static constexpr int TILE_SLOTS = BS * HD / 8;    // 16-byte slots of a K block or V^T tile
  static constexpr int TILE_BYTES = TILE_SLOTS * 16;
  static constexpr int NI = TILE_BYTES / 4096;      // 1 KB staging loads per wave and tile
  static constexpr int ROWS_PER_LOAD = 1024 / ROW_BYTES;  // K rows one 1 KB load covers
  // Merge buffer of one query half: O^T partials, running maxima, row sums.
  static constexpr int XCHG_FLOATS = NDT * 2 * 4 * 64 + 2 * 2 * 64;
  // Chunk c of K row R sits at chunk position c ^ kswz(R): the 16 rows one
  // operand read touches then fall into 16 distinct 16-byte bank groups
  // (a 128-byte row pairs rows R, R + 1 in one 256-byte bank cycle).
  __host__ __device__ static constexpr int kswz(int R) {
    return HD == 128 ? (R & 15) : ((R >> 1) & 7);
  }
};

// Bytes of packed data per (b, h, key block) for an input dtype: the V^T tile,
// or for fp32 the block image [K hi rows][K lo rows][V^T hi][V^T lo].
constexpr size_t block_bytes(cab_dtype_t dt, int hd) {
  return static_cast<size_t>(dt == CAB_F32 ? 4 : 1) * BS * hd * 2;
}

struct AttnArgs {
  const void* q;       // bf16 / fp16 / fp32 [B, H, N, D]
  const uint16_t* k;   // bf16 / fp16 K (unused for fp32: K is in the block images)
  const uint16_t* vt;  // per (b, h, key block): V^T tile (16 KB) or fp32 block image (64 KB)
  void* o;             // same dtype as q
  float* lse;
  int64_t qs[3], ks[3], os[3];  // b, h, token strides (elements)
  const int32_t* kv_idx;
  const int32_t* kv_cnt;
  int32_t BH, H, N, M;  // B * H, query heads, query tokens, query blocks (all < 2^31)
  int32_t Nk, Mk;       // key tokens, key blocks
  int32_t group;        // query heads per K / V head
  int32_t qoff;         // causal: query token t sees keys <= t + qoff
  int32_t kmax;
  float scale_log2;
  int causal;
  // Block sizes below 64: per list entry, the 64-bit mask of the (bs x bs)
  // sub-tiles of its 64 x 64 tile that are kept (bit (q / bs) * (64 / bs) +
  // k / bs for query q and key k of the tile); null when every tile is whole.
  const uint64_t* submask;
  int sub_shift;  // log2(block_size) when submask is set
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

// fp32 -> bf16 pair split of two values: {hi, lo} with hi = bf16(x) and
// lo = bf16(x - hi), both round-to-nearest-even (x - hi is exact in fp32).
__device__ __forceinline__ u32x2 split2(float x0, float x1) {
  const uint32_t hi = pack2<true>(x0, x1);
  const float h0 = __builtin_bit_cast(float, hi << 16);
  const float h1 = __builtin_bit_cast(float, hi & 0xffff0000u);
  return u32x2{hi, pack2<true>(x0 - h0, x1 - h1)};
}

// Eight consecutive fp32 values (x0, x1) -> bf16x8 hi and lo operands.
__device__ __forceinline__ void split8(const f32x4& x0, const f32x4& x1, u32x4& hi, u32x4& lo) {
  const u32x2 a = split2(x0[0], x0[1]), b = split2(x0[2], x0[3]);
  const u32x2 e = split2(x1[0], x1[1]), f = split2(x1[2], x1[3]);
  hi = u32x4{a[0], b[0], e[0], f[0]};
  lo = u32x4{a[1], b[1], e[1], f[1]};
}

// One block of V rows in LDS, padded.
template <int HD>
using VRows = uint16_t[HD + 8];

// V^T tile slot (dt, s, L) (index (2 dt + s) * 64 + L) holds, for d = 16 dt + L % 16
// and g = L / 16, the 8 values V[32 s + 4 g + r][d] (r = 0..3) followed by
// V[32 s + 16 + 4 g + r][d] (r = 0..3).
template <int HD>
__device__ __forceinline__ u32x4 vt_slot(const VRows<HD>* vs, int slot) {
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
  return x;
}

template <int HD>
__device__ __forceinline__ void vrows_put(VRows<HD>* vs, int key, int c, const u32x4& x) {
  *reinterpret_cast<u32x2*>(&vs[key][8 * c]) = u32x2{x[0], x[1]};
  *reinterpret_cast<u32x2*>(&vs[key][8 * c + 4]) = u32x2{x[2], x[3]};
}

template <int HD>
__global__ __launch_bounds__(256) void pack_vt_kernel(PackArgs a) {
  using G = Dims<HD>;
  __shared__ VRows<HD> vs[BS];
  const int64_t bh = blockIdx.y, j = blockIdx.x;
  const int64_t b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const uint16_t* vb = a.v + b * a.vs[0] + h * a.vs[1];
  const int tid = threadIdx.x;
#pragma unroll
  for (int r = 0; r < G::TILE_SLOTS / 256; ++r) {
    const int cid = tid + 256 * r;  // TILE_SLOTS chunks of 8 values
    const int key = cid / G::CPR, c = cid % G::CPR;
    const int64_t t = j * BS + key;
    // V is read once: non-temporal loads (the pass 4 % faster)
    const u32x4 x = t < a.N ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vb + t * a.vs[2] + 8 * c))
                            : u32x4{0u, 0u, 0u, 0u};
    vrows_put<HD>(vs, key, c, x);
  }
  __syncthreads();
  u32x4* out = reinterpret_cast<u32x4*>(a.vt) + (bh * a.M + j) * G::TILE_SLOTS;
#pragma unroll
  for (int r = 0; r < G::TILE_SLOTS / 256; ++r) out[tid + 256 * r] = vt_slot<HD>(vs, tid + 256 * r);
}

struct SplitPackArgs {
  const float* k;
  const float* v;
  uint16_t* img;  // [B*H][M] block images of SPLIT_BLOCK_BYTES
  int64_t ks[3], vs[3];
  int64_t H, N, M;
};

// fp32 K and V of key block j -> its block image (64 KB at D = 128; zero
// past N):
//   K hi / K lo: 64 rows x 2 D bytes, the 16-byte chunks of row R stored at
//     position c ^ kswz(R) (the LDS layout the K operand reads expect);
//   V^T hi / V^T lo: pack_vt_kernel's tile layout.
template <int HD>
__global__ __launch_bounds__(256) void pack_split_kernel(SplitPackArgs a) {
  using G = Dims<HD>;
  constexpr int TILE_SLOTS = G::TILE_SLOTS;
  __shared__ VRows<HD> vh[BS], vl[BS];
  const int64_t bh = blockIdx.y, j = blockIdx.x;
  const int64_t b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const float* kb = a.k + b * a.ks[0] + h * a.ks[1];
  const float* vb = a.v + b * a.vs[0] + h * a.vs[1];
  const int tid = threadIdx.x;
  u32x4* out = reinterpret_cast<u32x4*>(a.img) + (bh * a.M + j) * (4 * TILE_SLOTS);
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < TILE_SLOTS / 256; ++r) {
    const int cid = tid + 256 * r;  // TILE_SLOTS chunks of 8 values
    const int key = cid / G::CPR, c = cid % G::CPR;
    const int64_t t = j * BS + key;
    const bool in = t < a.N;
    const float* kp = kb + t * a.ks[2] + 8 * c;
    const float* vp = vb + t * a.vs[2] + 8 * c;
    const f32x4 k0 = in ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(kp)) : zero;
    const f32x4 k1 = in ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(kp + 4)) : zero;
    const f32x4 v0 = in ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(vp)) : zero;
    const f32x4 v1 = in ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(vp + 4)) : zero;
    u32x4 hi, lo;
    split8(k0, k1, hi, lo);
    const int pos = G::CPR * key + (c ^ G::kswz(key));
    out[pos] = hi;
    out[TILE_SLOTS + pos] = lo;
    split8(v0, v1, hi, lo);
    vrows_put<HD>(vh, key, c, hi);
    vrows_put<HD>(vl, key, c, lo);
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < TILE_SLOTS / 256; ++r) {
    const int slot = tid + 256 * r;
    out[2 * TILE_SLOTS + slot] = vt_slot<HD>(vh, slot);
    out[3 * TILE_SLOTS + slot] = vt_slot<HD>(vl, slot);
  }
}

// 16-byte direct-to-LDS load per lane: global g + OFF, LDS l + OFF + 16 * lane.
// OFF is the instruction's immediate, a 13-bit signed field: the compiler
// wraps larger constants without a diagnostic, so they are refused here.
template <int OFF>
__device__ __forceinline__ void dma16(const char* g, char* l) {
  static_assert(OFF >= 0 && OFF < 4096, "global_load_lds immediate offset must be in [0, 4096)");
  __builtin_amdgcn_global_load_lds(g, (lds_void*)l, 16, OFF, 0);
}

// gfx950 lane swaps between the two halves of two registers (v_permlane32_swap:
// 32-lane halves; v_permlane16_swap: odd and even 16-lane rows), written as
// inline asm because the compiler's builtins return the first result twice.
// The s_nop gives the two wait states a swap needs after a VALU write of
// its operands.
__device__ __forceinline__ void lane_swap32(uint32_t& a, uint32_t& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void lane_swap16(uint32_t& a, uint32_t& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// Maxima over the four lane groups (lanes c + 16 g, g = 0..3) of two
// registers at once, without an LDS round trip. In: x0, x1 hold per-lane
// partial maxima of query column c = lane % 16 for query tiles 0 and 1.
// Out: each holds its tile's full column maximum in every lane.
__device__ __forceinline__ void colmax2(float& x0, float& x1) {
  uint32_t a = __builtin_bit_cast(uint32_t, x0), b = __builtin_bit_cast(uint32_t, x1);
  lane_swap32(a, b);  // one register holds both tiles' lower halves, the other the upper
  float y = __builtin_fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
  // y: tile 0 merged over g and g ^ 2 in one 32-lane half, tile 1 in the other.
  a = b = __builtin_bit_cast(uint32_t, y);
  lane_swap16(a, b);  // rows g and g ^ 1 side by side
  y = __builtin_fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
  a = b = __builtin_bit_cast(uint32_t, y);
  lane_swap32(a, b);  // each half broadcast to all 64 lanes
  x0 = __builtin_bit_cast(float, a);
  x1 = __builtin_bit_cast(float, b);
}

// Running-max sentinel: a finite stand-in for -inf, so that -max * c stays
// finite and exp2(s * c - max * c) of a masked score (-inf) is exactly 0.
constexpr float M_EMPTY = -1.0e30f;

// Softmax modes of one block step.
//  SM_ONLINE: online softmax with the lazy rescale (the maximum may grow).
//  SM_FIRST:  first block of a fixed-maximum walk: each query's maximum is
//             set to its largest score in this block (the accumulators are
//             still zero, so nothing is rescaled); queries with no finite
//             score keep M_EMPTY.
//  SM_FIXED:  later blocks of that walk: p = exp2(s c - m c) with the
//             maximum of the first block, no maxima, no rescale. A score
//             far above that maximum makes p (and the row sum) large or
//             infinite; the walk's end check (row_sums_ok) then sends the
//             row through an SM_ONLINE walk instead.
constexpr int SM_ONLINE = 0, SM_FIRST = 1, SM_FIXED = 2;
// Largest row sum a fixed-maximum walk may end with (2^64): every p is then
// at most 2^64, far inside fp32 and bf16 range, and the first block's
// maximum gives each query with a finite score a p of exactly 1, so no p
// that matters underflows.
constexpr uint32_t FIXED_SUM_MAX_BITS = 0x5f800000u;

// Online-softmax state of one wave: 32 queries (two tiles of 16, query on
// the lane axis) against one key half of every kept block.
template <int HD>
struct WaveAcc {
  static constexpr int NDS = Dims<HD>::NDS, NDT = Dims<HD>::NDT;
  u32x4 qreg[2][NDS];  // Q^T B operand: qreg[qt][ds] = Q[q0 + 16 qt + l % 16][32 ds + 8 g .. +8]
  u32x4 qlo[2][NDS];   // fp32 inputs: the lo halves of qreg (unused otherwise)
  f32x4 oacc[NDT][2];  // O^T[16 dt + 4 g + r][q0 + 16 qt + l % 16]
  f32x4 lacc[2];       // row sums (all four r equal)
  float m_run[2];      // running maximum of the raw scores
  float nmc[2];        // -m_run * c
};

// A wave's place in its group of four: key half kh, query half qh.
template <int HD>
struct WaveGeo {
  int kh, qh, lane, g, l16;
  uint32_t kread[Dims<HD>::NDS];  // K operand byte offsets inside a K stage
};

template <int HD>
__device__ __forceinline__ WaveGeo<HD> wave_geo(int w4) {
  using G = Dims<HD>;
  WaveGeo<HD> ge;
  ge.kh = w4 & 1;
  ge.qh = (w4 >> 1) & 1;
  ge.lane = lane_id();
  ge.g = ge.lane >> 4;
  ge.l16 = ge.lane & 15;
  // K operand (key 32 kh + 16 tt + l % 16, dims 32 ds + 8 g .. +8) inside a
  // stage: row R = 32 kh + 16 tt + l % 16, chunk 4 ds + g, stored
  // XOR-swizzled at chunk position (4 ds + g) ^ kswz(R); kswz(R) depends on
  // l % 16 only, so tt adds a fixed 16 rows (the caller's offset).
#pragma unroll
  for (int ds = 0; ds < G::NDS; ++ds)
    ge.kread[ds] = G::ROW_BYTES * (32 * ge.kh + ge.l16) + 16 * ((4 * ds + ge.g) ^ G::kswz(ge.l16));
  return ge;
}

// Loads the wave's 32 queries (from token q0; rows at or past N are zero;
// fp32 queries split into qreg / qlo) and clears the accumulators.
template <cab_dtype_t DT, int HD>
__device__ __forceinline__ void acc_init(WaveAcc<HD>& s, const WaveGeo<HD>& ge, const void* qv,
                                         int64_t qs2, int q0, int N, float c) {
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qtok = q0 + 16 * qt + ge.l16;
    const bool in = q0 >= 0 && qtok < N;
#pragma unroll
    for (int ds = 0; ds < Dims<HD>::NDS; ++ds) {
      if constexpr (DT == CAB_F32) {
        const float* qp = static_cast<const float*>(qv) + qtok * qs2 + 32 * ds + 8 * ge.g;
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        const f32x4 x0 = in ? *reinterpret_cast<const f32x4*>(qp) : zero;
        const f32x4 x1 = in ? *reinterpret_cast<const f32x4*>(qp + 4) : zero;
        split8(x0, x1, s.qreg[qt][ds], s.qlo[qt][ds]);
      } else {
        const uint16_t* qp = static_cast<const uint16_t*>(qv) + qtok * qs2 + 32 * ds + 8 * ge.g;
        s.qreg[qt][ds] = in ? *reinterpret_cast<const u32x4*>(qp) : u32x4{0u, 0u, 0u, 0u};
      }
    }
    s.lacc[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < Dims<HD>::NDT; ++dt) s.oacc[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    s.m_run[qt] = M_EMPTY;
    s.nmc[qt] = -M_EMPTY * c;
  }
}

// Clears the accumulators and maxima (the queries stay loaded).
template <int HD>
__device__ __forceinline__ void acc_reset(WaveAcc<HD>& s, float c) {
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    s.lacc[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < Dims<HD>::NDT; ++dt) s.oacc[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    s.m_run[qt] = M_EMPTY;
    s.nmc[qt] = -M_EMPTY * c;
  }
}

// Whether a fixed-maximum walk left this lane's state usable: both row sums
// finite and at most 2^64, and the accumulators finite (their sum is; an
// overflow of the sum alone only costs a needless online walk). Tested on
// the bits: the file's device code is compiled without NaN semantics.
template <int HD>
__device__ __forceinline__ bool row_sums_ok(const WaveAcc<HD>& s) {
  float t = 0.f;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int dt = 0; dt < Dims<HD>::NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) t += s.oacc[dt][qt][r];
  const uint32_t l0 = __builtin_bit_cast(uint32_t, s.lacc[0][0]) & 0x7fffffffu;
  const uint32_t l1 = __builtin_bit_cast(uint32_t, s.lacc[1][0]) & 0x7fffffffu;
  const uint32_t te = __builtin_bit_cast(uint32_t, t) & 0x7f800000u;
  return l0 <= FIXED_SUM_MAX_BITS && l1 <= FIXED_SUM_MAX_BITS && te != 0x7f800000u;
}

// Marks the queries as loaded: later waits in the block loop then never
// have to cover the Q loads.
template <cab_dtype_t DT, int HD>
__device__ __forceinline__ void acc_q_ready(WaveAcc<HD>& s) {
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int ds = 0; ds < Dims<HD>::NDS; ++ds) {
      asm volatile("" ::"v"(s.qreg[qt][ds]));
      if constexpr (DT == CAB_F32) asm volatile("" ::"v"(s.qlo[qt][ds]));
    }
}

// Whether key block j needs per-key masks for query block i: an invalid
// list entry, keys past Nk, or (causal) a key after some query of the block.
__device__ __forceinline__ bool block_needs_mask(int j, int i, bool valid, int Nk, bool causal,
                                                 int qoff) {
  return !valid || (j + 1) * BS > Nk || (causal && j * BS + BS - 1 > i * BS + qoff);
}

// One key block j (staged at ks / vts) for the wave's queries of query block i:
//   S^T = K_kh Q^T (16 MFMA), masks, online softmax (fp32, log2 domain),
//   O^T += V_kh^T P^T (16 MFMA), row sums = 1 P^T (2 MFMA).
// fp32 (split operands, the lo halves 16 KB past the hi ones in LDS):
// 48 + 48 + 4 MFMA. Keys at or past Nk and (causal) keys after t + qoff for
// query t are dropped.
template <cab_dtype_t DT, int HD, int SM, typename Stager>
__device__ __forceinline__ void acc_block(WaveAcc<HD>& s, const WaveGeo<HD>& ge, const char* ks,
                                          const u32x4* vts, int j, int i, bool valid, int Nk,
                                          bool causal, int qoff, float c, uint64_t sm,
                                          int sub_shift, const Stager& stg) {
  using G = Dims<HD>;
  constexpr int NDS = G::NDS, NDT = G::NDT;
  constexpr int TT_BYTES = 16 * G::ROW_BYTES;  // 16 K rows
  constexpr bool BF16 = DT != CAB_F16;
  constexpr bool SPLIT = DT == CAB_F32;
  const uint32_t one2 = BF16 ? 0x3f803f80u : 0x3c003c00u;
  const u32x4 ones = {one2, one2, one2, one2};
  u32x4 kop[NDS][2], vop[NDT];
  u32x4 klo[NDS][2], vlo[NDT];  // SPLIT only
#pragma unroll
  for (int ds = 0; ds < NDS; ++ds)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      kop[ds][tt] = *reinterpret_cast<const u32x4*>(ks + ge.kread[ds] + TT_BYTES * tt);
      if constexpr (SPLIT)
        klo[ds][tt] =
            *reinterpret_cast<const u32x4*>(ks + G::TILE_BYTES + ge.kread[ds] + TT_BYTES * tt);
    }
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    vop[dt] = vts[(dt * 2 + ge.kh) * 64 + ge.lane];
    if constexpr (SPLIT) vlo[dt] = vts[G::TILE_SLOTS + (dt * 2 + ge.kh) * 64 + ge.lane];
  }

  // sc[tt][qt][r] = score(key 32 kh + 16 tt + 4 g + r, query 32 qh + 16 qt + l % 16)
  f32x4 sc[2][2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) sc[tt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ds = 0; ds < NDS; ++ds) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        if constexpr (SPLIT) {
          sc[tt][qt] = mfma16<true>(klo[ds][tt], s.qreg[qt][ds], sc[tt][qt]);
          sc[tt][qt] = mfma16<true>(kop[ds][tt], s.qlo[qt][ds], sc[tt][qt]);
        }
        sc[tt][qt] = mfma16<BF16>(kop[ds][tt], s.qreg[qt][ds], sc[tt][qt]);
      }
    if constexpr (!SPLIT) {
      // the next block's staging loads, spread between the score MFMAs
      __builtin_amdgcn_sched_barrier(0);
      stg(ds);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  const bool subm = sm != ~0ull;  // a tile of smaller blocks, some of them dropped
  if (block_needs_mask(j, i, valid, Nk, causal, qoff) || subm) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kl = 32 * ge.kh + 16 * tt + 4 * ge.g + r, ql = 32 * ge.qh + 16 * qt + ge.l16;
          const int ktok = j * BS + kl, qtok = i * BS + ql;
          bool drop = !valid || ktok >= Nk || (causal && ktok > qtok + qoff);
          if (subm)
            drop = drop || ((sm >> (((ql >> sub_shift) << (6 - sub_shift)) | (kl >> sub_shift))) &
                            1ull) == 0;
          if (drop) sc[tt][qt][r] = -INFINITY;
        }
  }
  float mx[2];
  if constexpr (SM != SM_FIXED) {
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const float m0 = __builtin_fmaxf(__builtin_fmaxf(sc[0][qt][0], sc[0][qt][1]),
                                       __builtin_fmaxf(sc[0][qt][2], sc[0][qt][3]));
      const float m1 = __builtin_fmaxf(__builtin_fmaxf(sc[1][qt][0], sc[1][qt][1]),
                                       __builtin_fmaxf(sc[1][qt][2], sc[1][qt][3]));
      mx[qt] = __builtin_fmaxf(m0, m1);
    }
  }
  if constexpr (SM == SM_FIRST) {
    colmax2(mx[0], mx[1]);
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      s.m_run[qt] = mx[qt] > M_EMPTY ? mx[qt] : M_EMPTY;
      s.nmc[qt] = -s.m_run[qt] * c;
    }
  }
  // Rescale only when a query's maximum grew by more than 2^RESCALE_LOG2
  // in exp2 units (always on its first non-empty block). A query's keys sit
  // in the four lane groups l16 + 16 g: the lane-local maxima tell whether
  // any query can have grown, and only then are the column maxima formed.
  if (SM == SM_ONLINE &&
      __builtin_amdgcn_ballot_w64(__builtin_fmaf(mx[0], c, s.nmc[0]) > RESCALE_LOG2 ||
                                  __builtin_fmaf(mx[1], c, s.nmc[1]) > RESCALE_LOG2)) {
    colmax2(mx[0], mx[1]);
    const bool grow[2] = {__builtin_fmaf(mx[0], c, s.nmc[0]) > RESCALE_LOG2,
                          __builtin_fmaf(mx[1], c, s.nmc[1]) > RESCALE_LOG2};
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const float m_new = grow[qt] ? mx[qt] : s.m_run[qt];
      const float alpha = __builtin_amdgcn_exp2f((s.m_run[qt] - m_new) * c);
      s.lacc[qt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) s.oacc[dt][qt] *= alpha;
      s.m_run[qt] = m_new;
      s.nmc[qt] = -m_new * c;
    }
  }
  u32x4 pb[2], pl[2];  // pl: SPLIT only
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    float pv[2][4];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        pv[tt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[tt][qt][r], c, s.nmc[qt]));
    if constexpr (SPLIT) {
      const f32x4 p0 = {pv[0][0], pv[0][1], pv[0][2], pv[0][3]};
      const f32x4 p1 = {pv[1][0], pv[1][1], pv[1][2], pv[1][3]};
      split8(p0, p1, pb[qt], pl[qt]);
    } else {
      pb[qt][0] = pack2<BF16>(pv[0][0], pv[0][1]);
      pb[qt][1] = pack2<BF16>(pv[0][2], pv[0][3]);
      pb[qt][2] = pack2<BF16>(pv[1][0], pv[1][1]);
      pb[qt][3] = pack2<BF16>(pv[1][2], pv[1][3]);
    }
  }
  // The P V products run at raised wave priority: the other wave of the SIMD
  // then fills the MFMA gaps with its own softmax work, not the reverse.
  if constexpr (!SPLIT) __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      if constexpr (SPLIT) {
        s.oacc[dt][qt] = mfma16<true>(vlo[dt], pb[qt], s.oacc[dt][qt]);
        s.oacc[dt][qt] = mfma16<true>(vop[dt], pl[qt], s.oacc[dt][qt]);
      }
      s.oacc[dt][qt] = mfma16<BF16>(vop[dt], pb[qt], s.oacc[dt][qt]);
    }
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    if constexpr (SPLIT) s.lacc[qt] = mfma16<true>(ones, pl[qt], s.lacc[qt]);
    s.lacc[qt] = mfma16<BF16>(ones, pb[qt], s.lacc[qt]);
  }
  if constexpr (!SPLIT) __builtin_amdgcn_s_setprio(0);
}

// Merge of the two key halves of a query half through LDS: the kh = 1 wave
// exports (acc_export), and after a workgroup barrier the kh = 0 wave
// combines and writes out, lse (acc_store). Dims<HD>::XCHG_FLOATS per query half.
template <int HD>
__device__ __forceinline__ void acc_export(const WaveAcc<HD>& s, const WaveGeo<HD>& ge, float* xo) {
  constexpr int NDT = Dims<HD>::NDT;
  float* xm = xo + NDT * 2 * 4 * 64;
  float* xl = xm + 2 * 64;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    xm[qt * 64 + ge.lane] = s.m_run[qt];
    xl[qt * 64 + ge.lane] = s.lacc[qt][0];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) xo[((dt * 2 + qt) * 4 + r) * 64 + ge.lane] = s.oacc[dt][qt][r];
  }
}

template <cab_dtype_t DT, int HD>
__device__ __forceinline__ void acc_store(const WaveAcc<HD>& s, const WaveGeo<HD>& ge,
                                          const float* xo, void* obase, int64_t os2,
                                          float* lse_row, int q0, int N, float c) {
  constexpr bool BF16 = DT != CAB_F16;
  constexpr int NDT = Dims<HD>::NDT;
  const float* xm = xo + NDT * 2 * 4 * 64;
  const float* xl = xm + 2 * 64;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float m1 = xm[qt * 64 + ge.lane], l1 = xl[qt * 64 + ge.lane];
    const float m = fmaxf(s.m_run[qt], m1);
    const float a0 = __builtin_amdgcn_exp2f((s.m_run[qt] - m) * c);
    const float a1 = __builtin_amdgcn_exp2f((m1 - m) * c);
    const float l = s.lacc[qt][0] * a0 + l1 * a1;
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    const int qtok = q0 + 16 * qt + ge.l16;
    if (qtok < N) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          o[r] = (s.oacc[dt][qt][r] * a0 + xo[((dt * 2 + qt) * 4 + r) * 64 + ge.lane] * a1) * inv;
        if constexpr (DT == CAB_F32) {
          float* ob = static_cast<float*>(obase) + qtok * os2;
          *reinterpret_cast<f32x4*>(ob + 16 * dt + 4 * ge.g) = f32x4{o[0], o[1], o[2], o[3]};
        } else {
          uint16_t* ob = static_cast<uint16_t*>(obase) + qtok * os2;
          *reinterpret_cast<u32x2*>(ob + 16 * dt + 4 * ge.g) = u32x2{pack2<BF16>(o[0], o[1]),
                                                                     pack2<BF16>(o[2], o[3])};
        }
      }
      if (lse_row && ge.g == 0)
        lse_row[qtok] = l > 0.f ? (m * c + __log2f(l)) * 0.69314718055994531f : -INFINITY;
    }
  }
}

// K staging offsets. K lands row-major, 64 rows x 2 D bytes, the 16-byte
// chunks of row R XOR-swizzled (chunk c at position c ^ kswz(R)) so that the
// operand reads are bank-conflict free; one instruction fetches 1 KB of
// whole rows (4 rows at D = 128, 8 at D = 64; full 128-byte lines): lane L
// takes row RPL x + L / CPR (x = the instruction's row group), chunk
// position L % CPR, i.e. source chunk (L % CPR) ^ kswz(row).
template <int HD>
__device__ __forceinline__ uint32_t k_lane_off(int group, int lane, int64_t krow_bytes) {
  using G = Dims<HD>;
  const int row = G::ROWS_PER_LOAD * group + lane / G::CPR;
  return static_cast<uint32_t>(row * krow_bytes + 16 * ((lane % G::CPR) ^ G::kswz(row)));
}



// ---------------------------------------------------------------------------
// attn_fwd_kernel: one query block per workgroup of 4 waves, two LDS stages;
// two workgroups per CU (bf16 / fp16: 32 KB stages) or one (fp32: 64 KB
// stages of split operands).
// ---------------------------------------------------------------------------
// Key-block lists of a query block: the caller's kv_idx staged in LDS, read
// from global memory (lists longer than LIST_MAX), or dense (every key block
// up to the causal limit, in order).
constexpr int LIST_LDS = 0, LIST_GLOBAL = 1, LIST_DENSE = 2;

template <cab_dtype_t DT, int LIST, int HD>
__global__ __launch_bounds__(256, DT == CAB_F32 ? 1 : 2) void attn_fwd_kernel(AttnArgs a) {
  using G = Dims<HD>;
  constexpr bool SPLIT = DT == CAB_F32;
  constexpr int TILE_SLOTS = G::TILE_SLOTS;
  constexpr int TILE_BYTES = G::TILE_BYTES;
  constexpr int NI = G::NI;
  constexpr int STAGE_SLOTS = (SPLIT ? 4 : 2) * TILE_SLOTS;
  constexpr int64_t BLOCK_BYTES = static_cast<int64_t>(block_bytes(DT, HD));
  // One LDS object: [stage 0][stage 1][list], a stage being [K][V^T] or
  // [K hi][K lo][V^T hi][V^T lo]; the merge at the end reuses the stages.
  __shared__ u32x4 smem[2 * STAGE_SLOTS + LIST_MAX / 4];
  auto stage_k = [&](int s) { return smem + s * STAGE_SLOTS; };
  auto stage_v = [&](int s) { return smem + s * STAGE_SLOTS + STAGE_SLOTS / 2; };
  int32_t* slist = reinterpret_cast<int32_t*>(smem + 2 * STAGE_SLOTS);

  const int M = a.M, N = a.N, Mk = a.Mk, Nk = a.Nk;
  const int logical = static_cast<int>(xcd_remap(blockIdx.x, static_cast<int64_t>(a.BH) * M));
  const int bh = logical / M;
  const int i = M - 1 - (logical - bh * M);  // longest causal rows first
  const int b = bh / a.H, hh = bh - (bh / a.H) * a.H;
  const int hk = hh / a.group;                        // K / V head
  const int64_t bhk = static_cast<int64_t>(b) * (a.H / a.group) + hk;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const WaveGeo<HD> ge = wave_geo<HD>(w);
  const float c = a.scale_log2;

  const void* qb = SPLIT ? static_cast<const void*>(static_cast<const float*>(a.q) + b * a.qs[0] +
                                                      hh * a.qs[1])
                         : static_cast<const void*>(static_cast<const uint16_t*>(a.q) +
                                                    b * a.qs[0] + hh * a.qs[1]);
  const char* kbytes = SPLIT ? nullptr
                             : reinterpret_cast<const char*>(a.k + b * a.ks[0] + hk * a.ks[1]);
  const char* vtbytes = reinterpret_cast<const char*>(a.vt) + bhk * Mk * BLOCK_BYTES;

  int cnt;
  const int32_t* glist = nullptr;
  if constexpr (LIST == LIST_DENSE) {
    // Key blocks 0 .. the last one holding a key some query of block i sees.
    const int last = i * BS + BS - 1 + a.qoff;
    cnt = !a.causal ? Mk : (last < 0 ? 0 : (last / BS + 1 < Mk ? last / BS + 1 : Mk));
  } else {
    cnt = a.kv_cnt[bh * static_cast<int64_t>(M) + i];
    cnt = cnt < 0 ? 0 : (cnt > a.kmax ? a.kmax : cnt);
    glist = a.kv_idx + (static_cast<int64_t>(bh) * M + i) * a.kmax;
  }
  if constexpr (LIST == LIST_LDS) {
    for (int p = threadIdx.x; p < cnt; p += 256) slist[p] = glist[p];
    __syncthreads();
  }
  auto entry = [&](int p) -> int {
    if constexpr (LIST == LIST_LDS)
      return __builtin_amdgcn_readfirstlane(slist[p]);
    else if constexpr (LIST == LIST_GLOBAL)
      return glist[p];
    else
      return p;
  };

  // Staging of key block j by the 4 waves: wave w fetches its NI KB of K
  // rows (rows 16 w .. +15 at D = 128) and of the V^T tile, one 1 KB buffer
  // load each, through descriptors based at the block (K: its valid rows, so
  // rows at or past Nk read as zero; V^T: the whole tile). fp32: the block
  // image is a copy of the stage; wave w copies its quarter w (one tile's
  // bytes).
  const int64_t krow_bytes = a.ks[2] * 2;
  const int64_t kblk_bytes = BS * krow_bytes;
  uint32_t koff[NI];
#pragma unroll
  for (int r = 0; r < NI; ++r) koff[r] = k_lane_off<HD>(NI * w + r, ge.lane, krow_bytes);
  const int voff = w * NI * 1024 + 16 * ge.lane;
  // Loads 2 NI / NDS of the 2 NI staging loads of block j (part ds of NDS).
  auto stage_part = [&](int j, u32x4* kst, u32x4* vst, int ds) {
    constexpr int PER = 2 * NI / G::NDS;
    char* kl = reinterpret_cast<char*>(kst) + w * NI * 1024;
    const int rows = Nk - j * BS < BS ? Nk - j * BS : BS;
    const brsrc_t krs = make_rsrc(kbytes + j * kblk_bytes, static_cast<uint32_t>(rows * krow_bytes));
    const brsrc_t vrs = make_rsrc(vtbytes + static_cast<int64_t>(j) * TILE_BYTES, TILE_BYTES);
    char* vl = reinterpret_cast<char*>(vst) + w * NI * 1024;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int r = ds * PER + q;
      if (r < NI)
        bdma16(krs, koff[r], 0, kl + 1024 * r);
      else
        bdma16(vrs, voff, 1024 * (r - NI), vl + 1024 * (r - NI));
    }
  };
  auto stage = [&](int j, u32x4* kst, u32x4* vst) {
    if constexpr (SPLIT) {
      const char* gp = vtbytes + j * BLOCK_BYTES + w * TILE_BYTES + 16 * ge.lane;
      char* lp = reinterpret_cast<char*>(kst) + w * TILE_BYTES;
#pragma unroll
      for (int r = 0; r < TILE_BYTES / 4096; ++r) {
        dma16<0>(gp + 4096 * r, lp + 4096 * r);
        dma16<1024>(gp + 4096 * r, lp + 4096 * r);
        dma16<2048>(gp + 4096 * r, lp + 4096 * r);
        dma16<3072>(gp + 4096 * r, lp + 4096 * r);
      }
      return;
    }
    char* kl = reinterpret_cast<char*>(kst) + w * NI * 1024;
    const int rows = Nk - j * BS < BS ? Nk - j * BS : BS;
    const brsrc_t krs = make_rsrc(kbytes + j * kblk_bytes, static_cast<uint32_t>(rows * krow_bytes));
#pragma unroll
    for (int r = 0; r < NI; ++r) bdma16(krs, koff[r], 0, kl + 1024 * r);
    const brsrc_t vrs = make_rsrc(vtbytes + static_cast<int64_t>(j) * TILE_BYTES, TILE_BYTES);
    char* vl = reinterpret_cast<char*>(vst) + w * NI * 1024;
#pragma unroll
    for (int r = 0; r < NI; ++r) bdma16(vrs, voff, 1024 * r, vl + 1024 * r);
  };

  WaveAcc<HD> st;
  acc_init<DT, HD>(st, ge, qb, a.qs[2], i * BS + 32 * ge.qh, N, c);
  __shared__ int wave_bad[4];
  auto block_of = [&](int j) { return (j >= 0 && j < Mk) ? j : 0; };

  // One walk over the row's blocks. FAST: the first block sets each query's
  // maximum and the rest use it unchanged (SM_FIRST, then SM_FIXED);
  // otherwise the online softmax with the lazy rescale (SM_ONLINE).
  auto walk = [&](auto fast_tag) {
    constexpr bool FAST = decltype(fast_tag)::value;
    int jraw = entry(0);
    stage(block_of(jraw), stage_k(0), stage_v(0));
    acc_q_ready<DT, HD>(st);

    // Block p lives in LDS stage PAR = p % 2 (compile time, so the compiler
    // sees the staging of block p + 1 into the other stage cannot alias).
    auto step = [&](int p, auto par_tag, auto sm_tag) {
      constexpr int PAR = decltype(par_tag)::value;
      constexpr int SM = decltype(sm_tag)::value;
      const bool valid = jraw >= 0 && jraw < Mk;
      const int j = valid ? jraw : 0;
      const uint64_t sm = a.submask ? a.submask[(static_cast<int64_t>(bh) * M + i) * a.kmax + p]
                                    : ~0ull;
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's staging of block p landed
      __builtin_amdgcn_s_barrier();        // ... and every wave's; stage PAR ^ 1 is free
      int jnext = 0;
      if constexpr (SPLIT) {
        if (p + 1 < cnt) {
          jnext = entry(p + 1);
          stage(block_of(jnext), stage_k(PAR ^ 1), stage_v(PAR ^ 1));
        }
        acc_block<DT, HD, SM>(st, ge, reinterpret_cast<const char*>(stage_k(PAR)), stage_v(PAR),
                              j, i, valid, Nk, a.causal, a.qoff, c, sm, a.sub_shift, [](int) {});
      } else {
        // unconditional (the last step re-stages a valid block into the free
        // stage; waited for after the loop) so that the loads sit between the MFMAs
        const int e = entry(p + 1 < cnt ? p + 1 : cnt - 1);
        jnext = p + 1 < cnt ? e : 0;
        const int js = block_of(jnext);
        acc_block<DT, HD, SM>(st, ge, reinterpret_cast<const char*>(stage_k(PAR)), stage_v(PAR),
                              j, i, valid, Nk, a.causal, a.qoff, c, sm, a.sub_shift,
                              [&](int ds) { stage_part(js, stage_k(PAR ^ 1), stage_v(PAR ^ 1), ds); });
      }
      jraw = jnext;
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    if constexpr (FAST) {
      step(0, P0{}, std::integral_constant<int, SM_FIRST>{});
      for (int p = 1; p < cnt; p += 2) {
        step(p, P1{}, std::integral_constant<int, SM_FIXED>{});
        if (p + 1 < cnt) step(p + 1, P0{}, std::integral_constant<int, SM_FIXED>{});
      }
    } else {
      for (int p = 0; p < cnt; p += 2) {
        step(p, P0{}, std::integral_constant<int, SM_ONLINE>{});
        if (p + 1 < cnt) step(p + 1, P1{}, std::integral_constant<int, SM_ONLINE>{});
      }
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the last step's staging landed
  };

  if (cnt > 0) {
    walk(std::true_type{});
    // Every wave reports whether its fixed-maximum state is usable; if any
    // is not, the whole row is walked again with the online softmax (the
    // barrier also frees both stages for that walk's first loads).
    const bool bad = __builtin_amdgcn_ballot_w64(!row_sums_ok<HD>(st)) != 0;
    if (threadIdx.x % 64 == 0) wave_bad[w] = bad ? 1 : 0;
    __syncthreads();
    if ((wave_bad[0] | wave_bad[1] | wave_bad[2] | wave_bad[3]) != 0) {
      acc_reset<HD>(st, c);
      walk(std::false_type{});
    }
  }

  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the last step's staging landed
  __syncthreads();
  static_assert(2 * G::XCHG_FLOATS * 4 <= 2 * STAGE_SLOTS * 16, "merge buffer fits the stages");
  float* xo = reinterpret_cast<float*>(smem) + ge.qh * G::XCHG_FLOATS;
  if (ge.kh == 1) acc_export<HD>(st, ge, xo);
  __syncthreads();
  void* ob = SPLIT ? static_cast<void*>(static_cast<float*>(a.o) + b * a.os[0] + hh * a.os[1])
                   : static_cast<void*>(static_cast<uint16_t*>(a.o) + b * a.os[0] + hh * a.os[1]);
  if (ge.kh == 0)
    acc_store<DT, HD>(st, ge, xo, ob, a.os[2],
                    a.lse ? a.lse + static_cast<int64_t>(bh) * N : nullptr, i * BS + 32 * ge.qh,
                    N, c);
}

// ---------------------------------------------------------------------------
// attn_pair_kernel: two adjacent query blocks (rows i = 2 p and 2 p + 1 of
// the block mask) per workgroup of 4 waves, two workgroups per CU.
//
// Adjacent rows keep most of the same key blocks (about 62 % at config 4),
// so the workgroup walks the union of the two rows' lists and stages each
// block once for both rows: 0.62 staged blocks per kept tile there instead
// of 1. Wave w owns queries 16 w .. 16 w + 15 of each row, so every wave has
// the same work in every step (both rows' 16-query tiles for a block both
// rows keep, one tile otherwise) and keeps its own queries' softmax state
// for all 64 keys: no split of the key dimension and no merge at the end.
// Per union entry and wave:
//   S^T_r = K Q_r^T    (16 MFMA 16x16x32 per present row r; each K operand
//                       read from LDS once and used for both rows)
//   softmax of the row's 16 x 64 scores (fixed-maximum walk, as above)
//   O^T_r += V^T P_r^T (16 MFMA per row; each V^T operand read once)
//   row sums = 1 P_r^T (2 MFMA per row)
// The union walk is built in the prologue from the rows' lists: entries
// outside [0, Mk) are dropped, and two strictly ascending lists are merged
// (each entry tagged with the rows that keep it); other lists (unsorted or
// with repeats, whose blocks count once per occurrence) are walked one
// after the other, untagged for the other row. 16-bit inputs, lists of at
// most PAIR_KMAX entries.
// ---------------------------------------------------------------------------
constexpr int PAIR_KMAX = 512;
constexpr uint32_t TAG_A = 1u << 30, TAG_B = 1u << 31, TAG_BLOCK = TAG_A - 1u;

template <int HD>
struct PairAcc {
  static constexpr int NDS = Dims<HD>::NDS, NDT = Dims<HD>::NDT;
  u32x4 qreg[2][NDS];  // row r: Q[q0_r + l % 16][32 ds + 8 g .. +8]
  f32x4 oacc[2][NDT];  // row r: O^T[16 dt + 4 g + r'][q0_r + l % 16]
  f32x4 lacc[2];       // row sums (all four entries equal)
  float m_run[2];      // each lane's query maximum (raw scores)
  float nmc[2];        // -m_run * c
};

template <int HD>
__device__ __forceinline__ void pair_reset(PairAcc<HD>& s, float c) {
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    s.lacc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < Dims<HD>::NDT; ++dt) s.oacc[r][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    s.m_run[r] = M_EMPTY;
    s.nmc[r] = -M_EMPTY * c;
  }
}

// The fixed-maximum walk's end check for both rows of a lane (row_sums_ok).
template <int HD>
__device__ __forceinline__ bool pair_sums_ok(const PairAcc<HD>& s) {
  float t = 0.f;
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int dt = 0; dt < Dims<HD>::NDT; ++dt)
#pragma unroll
      for (int q = 0; q < 4; ++q) t += s.oacc[r][dt][q];
  const uint32_t l0 = __builtin_bit_cast(uint32_t, s.lacc[0][0]) & 0x7fffffffu;
  const uint32_t l1 = __builtin_bit_cast(uint32_t, s.lacc[1][0]) & 0x7fffffffu;
  const uint32_t te = __builtin_bit_cast(uint32_t, t) & 0x7f800000u;
  return l0 <= FIXED_SUM_MAX_BITS && l1 <= FIXED_SUM_MAX_BITS && te != 0x7f800000u;
}

// Softmax of one row's 16 x 64 score tile held by a wave (lane: query
// l % 16, keys 16 kt + 4 g + r') into its P^T operands. FAST: fixed maximum,
// set from the first block the row meets (mset); otherwise the online
// softmax with the lazy rescale.
template <bool FAST, bool BF16, int HD>
__device__ __forceinline__ void pair_softmax(PairAcc<HD>& s, int r, f32x4 (&sc)[4], float c,
                                             bool& mset, u32x4 (&pb)[2]) {
  constexpr int NDT = Dims<HD>::NDT;
  if (!FAST || !mset) {
    float mx = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(sc[0][0], sc[0][1]),
                                               __builtin_fmaxf(sc[0][2], sc[0][3])),
                               __builtin_fmaxf(__builtin_fmaxf(sc[1][0], sc[1][1]),
                                               __builtin_fmaxf(sc[1][2], sc[1][3])));
    mx = __builtin_fmaxf(mx, __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(sc[2][0], sc[2][1]),
                                                             __builtin_fmaxf(sc[2][2], sc[2][3])),
                                             __builtin_fmaxf(__builtin_fmaxf(sc[3][0], sc[3][1]),
                                                             __builtin_fmaxf(sc[3][2], sc[3][3]))));
    if constexpr (FAST) {
      float m2 = mx;
      colmax2(mx, m2);
      s.m_run[r] = mx > M_EMPTY ? mx : M_EMPTY;
      s.nmc[r] = -s.m_run[r] * c;
      mset = true;
    } else if (__builtin_amdgcn_ballot_w64(__builtin_fmaf(mx, c, s.nmc[r]) > RESCALE_LOG2)) {
      float m2 = mx;
      colmax2(mx, m2);
      const bool grow = __builtin_fmaf(mx, c, s.nmc[r]) > RESCALE_LOG2;
      const float m_new = grow ? mx : s.m_run[r];
      const float alpha = __builtin_amdgcn_exp2f((s.m_run[r] - m_new) * c);
      s.lacc[r] *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) s.oacc[r][dt] *= alpha;
      s.m_run[r] = m_new;
      s.nmc[r] = -m_new * c;
    }
  }
  float p[4][4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int q = 0; q < 4; ++q) p[kt][q] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kt][q], c, s.nmc[r]));
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    pb[ks][0] = pack2<BF16>(p[2 * ks][0], p[2 * ks][1]);
    pb[ks][1] = pack2<BF16>(p[2 * ks][2], p[2 * ks][3]);
    pb[ks][2] = pack2<BF16>(p[2 * ks + 1][0], p[2 * ks + 1][1]);
    pb[ks][3] = pack2<BF16>(p[2 * ks + 1][2], p[2 * ks + 1][3]);
  }
}

template <cab_dtype_t DT, int LIST, int HD>
__global__ __launch_bounds__(256, 2) void attn_pair_kernel(AttnArgs a) {
  static_assert(DT != CAB_F32, "16-bit inputs only");
  static_assert(LIST == LIST_LDS || LIST == LIST_DENSE, "lists staged in LDS, or dense");
  constexpr bool DENSE = LIST == LIST_DENSE;
  using G = Dims<HD>;
  constexpr int NDS = G::NDS, NDT = G::NDT;
  constexpr int TILE_SLOTS = G::TILE_SLOTS, TILE_BYTES = G::TILE_BYTES, NI = G::NI;
  constexpr int STAGE_SLOTS = 2 * TILE_SLOTS;
  constexpr int TT_BYTES = 16 * G::ROW_BYTES;  // 16 K rows
  constexpr bool BF16 = DT == CAB_BF16;
  __shared__ u32x4 smem[2 * STAGE_SLOTS];  // [stage 0: K, V^T][stage 1: K, V^T]
  constexpr int LISTN = DENSE ? 1 : PAIR_KMAX;  // dense rows need no list in LDS
  __shared__ int32_t lst[2][LISTN];        // each row's valid entries, in list order
  __shared__ uint32_t uni[2 * LISTN];      // the walk: block | TAG_A | TAG_B
  __shared__ int meta[8];                  // n_A, n_B, sorted_A, sorted_B, U, -, -, -
  __shared__ int wave_bad[4];
  auto stage_k = [&](int st) { return smem + st * STAGE_SLOTS; };
  auto stage_v = [&](int st) { return smem + st * STAGE_SLOTS + TILE_SLOTS; };

  const int M = a.M, N = a.N, Mk = a.Mk, Nk = a.Nk;
  const int MP = (M + 1) / 2;
  const int logical = static_cast<int>(xcd_remap(blockIdx.x, static_cast<int64_t>(a.BH) * MP));
  const int bh = logical / MP;
  const int pr = MP - 1 - (logical - bh * MP);  // longest causal pairs first
  const int irow[2] = {2 * pr, 2 * pr + 1};     // irow[1] == M: no second row
  const int b = bh / a.H, hh = bh - (bh / a.H) * a.H;
  const int hk = hh / a.group;                                  // K / V head
  const int64_t bhk = static_cast<int64_t>(b) * (a.H / a.group) + hk;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int lane = lane_id(), g = lane >> 4, l16 = lane & 15;
  const float c = a.scale_log2;

  const uint16_t* qb = static_cast<const uint16_t*>(a.q) + b * a.qs[0] + hh * a.qs[1];
  const char* kbytes = reinterpret_cast<const char*>(a.k + b * a.ks[0] + hk * a.ks[1]);
  const char* vtbytes = reinterpret_cast<const char*>(a.vt) + bhk * Mk * TILE_BYTES;

  // Queries (issued first; they land while the walk is built).
  PairAcc<HD> st;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int qtok = 64 * irow[r] + 16 * w + l16;
    const bool in = irow[r] < M && qtok < N;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
      st.qreg[r][ds] = in ? *reinterpret_cast<const u32x4*>(qb + qtok * a.qs[2] + 32 * ds + 8 * g)
                          : u32x4{0u, 0u, 0u, 0u};
  }
  pair_reset<HD>(st, c);

  // The walk. Dense rows: key blocks 0 .. dcnt[r] - 1 of each row (up to the
  // last block holding a key some query of the row sees), so the union is
  // 0 .. max - 1, tagged arithmetically. Lists: waves 0 and 1 each compact
  // one row's list (valid entries, in order) and test it for strict ascent;
  // then each places its row's entries: merged by rank when both lists
  // ascend, else one after the other.
  int dcnt[2] = {0, 0};
  int U = 0;
  if constexpr (DENSE) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int last = irow[r] * BS + BS - 1 + a.qoff;
      dcnt[r] = irow[r] >= M ? 0
                : !a.causal ? Mk
                            : (last < 0 ? 0 : (last / BS + 1 < Mk ? last / BS + 1 : Mk));
    }
    U = dcnt[0] > dcnt[1] ? dcnt[0] : dcnt[1];
  } else {
    if (w < 2) {
      const int r = w;
      int cnt = 0;
      if (irow[r] < M) {
        cnt = a.kv_cnt[static_cast<int64_t>(bh) * M + irow[r]];
        cnt = cnt < 0 ? 0 : (cnt > a.kmax ? a.kmax : cnt);
      }
      const int32_t* gl = a.kv_idx + (static_cast<int64_t>(bh) * M + irow[r]) * a.kmax;
      int n = 0;
      for (int base = 0; base < cnt; base += 64) {
        const int x = base + lane < cnt ? gl[base + lane] : -1;
        const bool valid = x >= 0 && x < Mk;
        const uint64_t bal = ballot64(valid);
        if (valid) lst[r][n + static_cast<int>(rank_below64(bal))] = x;
        n += __popcll(bal);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's list writes landed
      bool asc = true;
      for (int base = 0; base + 1 < n; base += 64) {
        const int i = base + lane;
        const bool ok = i + 1 >= n || lst[r][i] < lst[r][i + 1 < n ? i + 1 : i];
        asc = asc && ballot64(!ok) == 0;
      }
      if (lane == 0) {
        meta[r] = n;
        meta[2 + r] = asc ? 1 : 0;
      }
    }
    __syncthreads();
    const int nrow[2] = {meta[0], meta[1]};
    const bool merge = meta[2] != 0 && meta[3] != 0;
    if (w < 2) {
      const int r = w, n = nrow[r], no = nrow[r ^ 1];
      const int32_t* other = lst[r ^ 1];
      const uint32_t tag = r == 0 ? TAG_A : TAG_B;
      int common = 0;  // entries of this row below the chunk that the other row keeps too
      for (int base = 0; base < n; base += 64) {
        const int i = base + lane;
        const int x = i < n ? lst[r][i] : 0;
        int pos = r == 0 ? i : nrow[0] + i;
        bool shared = false;
        if (merge) {
          int lo = 0, hi = no;  // lower bound of x in the other row's list
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (other[mid] < x) lo = mid + 1; else hi = mid;
          }
          shared = lo < no && other[lo] == x;
          const uint64_t sb = ballot64(i < n && shared);
          pos = i + lo - common - static_cast<int>(rank_below64(sb));
          common += __popcll(sb);
        }
        if (i < n && !(r == 1 && shared))
          uni[pos] = static_cast<uint32_t>(x) | tag | (shared ? TAG_B : 0u);
      }
      if (r == 0 && lane == 0) meta[4] = nrow[0] + nrow[1] - (merge ? common : 0);
    }
    __syncthreads();
    U = meta[4];
  }

  // Staging (as in attn_fwd_kernel): wave w fetches its NI KB of K rows and
  // of the V^T tile of a block, one 1 KB buffer load each.
  const int64_t krow_bytes = a.ks[2] * 2;
  const int64_t kblk_bytes = BS * krow_bytes;
  uint32_t koff[NI];
#pragma unroll
  for (int r = 0; r < NI; ++r) koff[r] = k_lane_off<HD>(NI * w + r, lane, krow_bytes);
  const int voff = w * NI * 1024 + 16 * lane;
  // Loads 2 NI / NDS of the wave's 2 NI staging loads of block j (part
  // 0 .. NDS - 1).
  auto stage_part = [&](int j, u32x4* kst, u32x4* vst, int part) {
    constexpr int PER = 2 * NI / NDS;
    static_assert(NDS % 2 == 0 && NDT % (NDS / 2) == 0, "staging parts split over S and P V");
    char* kl = reinterpret_cast<char*>(kst) + w * NI * 1024;
    char* vl = reinterpret_cast<char*>(vst) + w * NI * 1024;
    const int rows = Nk - j * BS < BS ? Nk - j * BS : BS;
    const sgpr_rsrc_t krs =
        make_sgpr_rsrc(kbytes + j * kblk_bytes, static_cast<uint32_t>(rows * krow_bytes));
    const sgpr_rsrc_t vrs = make_sgpr_rsrc(vtbytes + static_cast<int64_t>(j) * TILE_BYTES, TILE_BYTES);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int r = part * PER + q;
      if (r < NI)
        bdma16_untracked(krs, koff[r], 0u, kl + 1024 * r);
      else
        bdma16_untracked(vrs, voff + 1024u * (r - NI), 0u, vl + 1024 * (r - NI));
    }
  };
  // K operand offset of (key tile kt, k-step ds) inside a K stage.
  uint32_t kread[NDS];
#pragma unroll
  for (int ds = 0; ds < NDS; ++ds)
    kread[ds] = G::ROW_BYTES * l16 + 16 * ((4 * ds + g) ^ G::kswz(l16));
  const uint32_t one2 = BF16 ? 0x3f803f80u : 0x3c003c00u;
  const u32x4 ones = {one2, one2, one2, one2};

  // One union entry (block j, rows ROWS: bit 0 row A, bit 1 row B) from LDS
  // stage PAR, with the next entry's staging spread between its S MFMAs.
  auto entry_step = [&](int j, auto rows_tag, auto par_tag, auto fast_tag, int jn, bool (&mset)[2]) {
    constexpr int ROWS = decltype(rows_tag)::value;
    constexpr int PAR = decltype(par_tag)::value;
    constexpr bool FAST = decltype(fast_tag)::value;
    const char* ks = reinterpret_cast<const char*>(stage_k(PAR));
    const u32x4* vts = stage_v(PAR);
    f32x4 sc[2][4];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) sc[r][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // K operands one k-step ahead of their MFMAs (two register sets), so an
    // LDS read's latency overlaps the previous k-step's products.
    u32x4 kf[2][4];
    auto read_k = [&](int ds, u32x4 (&dst)[4]) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
        dst[kt] = *reinterpret_cast<const u32x4*>(ks + kread[ds] + TT_BYTES * kt);
    };
    read_k(0, kf[0]);
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      if (ds + 1 < NDS) read_k(ds + 1, kf[(ds + 1) & 1]);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 2; ++r)
          if (ROWS & (1 << r)) sc[r][kt] = mfma16<BF16>(kf[ds & 1][kt], st.qreg[r][ds], sc[r][kt]);
      // the next entry's staging: the first half of its loads here, between
      // the S MFMAs, the second half between the P V MFMAs below
      if (ds % 2 == 0) {
        __builtin_amdgcn_sched_barrier(0);
        stage_part(jn, stage_k(PAR ^ 1), stage_v(PAR ^ 1), ds / 2);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // The first V^T operands are read before the softmax, the rest four
    // O^T tiles ahead of their MFMAs.
    constexpr int VAHEAD = 4;
    constexpr int PV_PART_EVERY = NDT / (NDS / 2);  // O^T tiles per staging part
    u32x4 vf[NDT][2];
    auto read_v = [&](int dt) {
      vf[dt][0] = vts[(2 * dt + 0) * 64 + lane];
      vf[dt][1] = vts[(2 * dt + 1) * 64 + lane];
    };
#pragma unroll
    for (int dt = 0; dt < VAHEAD; ++dt) read_v(dt);
    u32x4 pb[2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      if (!(ROWS & (1 << r))) continue;
      if (block_needs_mask(j, irow[r], true, Nk, a.causal, a.qoff)) {
        const int qtok = 64 * irow[r] + 16 * w + l16;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int ktok = j * BS + 16 * kt + 4 * g + q;
            if (ktok >= Nk || (a.causal && ktok > qtok + a.qoff)) sc[r][kt][q] = -INFINITY;
          }
      }
      pair_softmax<FAST, BF16, HD>(st, r, sc[r], c, mset[r], pb[r]);
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      if (dt + VAHEAD < NDT) read_v(dt + VAHEAD);
      if (dt % PV_PART_EVERY == 0) {
        __builtin_amdgcn_sched_barrier(0);
        stage_part(jn, stage_k(PAR ^ 1), stage_v(PAR ^ 1), NDS / 2 + dt / PV_PART_EVERY);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int r = 0; r < 2; ++r)
        if (ROWS & (1 << r)) {
          st.oacc[r][dt] = mfma16<BF16>(vf[dt][0], pb[r][0], st.oacc[r][dt]);
          st.oacc[r][dt] = mfma16<BF16>(vf[dt][1], pb[r][1], st.oacc[r][dt]);
        }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r)
      if (ROWS & (1 << r)) {
        st.lacc[r] = mfma16<BF16>(ones, pb[r][0], st.lacc[r]);
        st.lacc[r] = mfma16<BF16>(ones, pb[r][1], st.lacc[r]);
      }
    __builtin_amdgcn_s_setprio(0);
  };

  auto walk = [&](auto fast_tag) {
    bool mset[2] = {false, false};
    auto ent = [&](int u) -> uint32_t {
      if constexpr (DENSE)
        return static_cast<uint32_t>(u) | (u < dcnt[0] ? TAG_A : 0u) | (u < dcnt[1] ? TAG_B : 0u);
      else
        return __builtin_amdgcn_readfirstlane(uni[u]);
    };
    uint32_t e = ent(0);
    {
      const int j0 = static_cast<int>(e & TAG_BLOCK);
#pragma unroll
      for (int part = 0; part < NDS; ++part) stage_part(j0, stage_k(0), stage_v(0), part);
    }
    auto step = [&](int u, auto par_tag) {
      const uint32_t en = ent(u + 1 < U ? u + 1 : U - 1);  // the last step re-stages its own block
      const int j = static_cast<int>(e & TAG_BLOCK), jn = static_cast<int>(en & TAG_BLOCK);
      // vmcnt(0): this wave's staging of entry u landed; the barrier: every
      // wave's did, and the other stage is free. Written as one asm statement
      // with a memory clobber, so no LDS access moves across it.
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      if ((e & TAG_A) && (e & TAG_B))
        entry_step(j, std::integral_constant<int, 3>{}, par_tag, fast_tag, jn, mset);
      else if (e & TAG_A)
        entry_step(j, std::integral_constant<int, 1>{}, par_tag, fast_tag, jn, mset);
      else
        entry_step(j, std::integral_constant<int, 2>{}, par_tag, fast_tag, jn, mset);
      e = en;
    };
    for (int u = 0; u < U; u += 2) {
      step(u, std::integral_constant<int, 0>{});
      if (u + 1 < U) step(u + 1, std::integral_constant<int, 1>{});
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last step's staging landed
  };

  if (U > 0) {
    walk(std::true_type{});
    const bool bad = ballot64(!pair_sums_ok<HD>(st)) != 0;
    if (lane == 0) wave_bad[w] = bad ? 1 : 0;
    __syncthreads();
    if ((wave_bad[0] | wave_bad[1] | wave_bad[2] | wave_bad[3]) != 0) {
      pair_reset<HD>(st, c);
      walk(std::false_type{});
    }
  }

  // Each wave writes its own queries: O = O^T / l, lse = (m c + log2 l) ln 2.
  uint16_t* ob = static_cast<uint16_t*>(a.o) + b * a.os[0] + hh * a.os[1];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int qtok = 64 * irow[r] + 16 * w + l16;
    if (irow[r] >= M || qtok >= N) continue;
    const float l = st.lacc[r][0];
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const f32x4 o = st.oacc[r][dt] * inv;
      *reinterpret_cast<u32x2*>(ob + qtok * a.os[2] + 16 * dt + 4 * g) =
          u32x2{pack2<BF16>(o[0], o[1]), pack2<BF16>(o[2], o[3])};
    }
    if (a.lse && g == 0)
      a.lse[static_cast<int64_t>(bh) * N + qtok] =
          l > 0.f ? (st.m_run[r] * c + __log2f(l)) * 0.69314718055994531f : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// Block sizes other than 64: the caller's lists over bs-token blocks become
// lists over 64-token tiles, which the executors walk.
//  relist_expand_kernel (bs = 64 r): entry jb of bs-row ib gives tiles
//    jb r .. jb r + r - 1 to each of the r 64-rows of ib, in that order
//    (entries outside [0, Mb) and tiles past the last key block stay -1,
//    which the executors skip).
//  relist_merge_kernel (bs = 64 / r): the r bs-rows of a 64-row give their
//    entries jb as (tile jb / r, sub-tile bit u r + jb % r) for sub-row u.
//    One wave merges them in list order: a pair joins the first entry of
//    its tile that lacks its bit, or starts a new entry. A block listed
//    twice therefore counts twice, as in the caller's lists. Each entry
//    carries its 64-bit sub-tile mask (AttnArgs::submask).
// ---------------------------------------------------------------------------
struct RelistArgs {
  const int32_t* idx;  // [BH, Mb, kmax]
  const int32_t* cnt;  // [BH, Mb]
  int32_t* idx64;      // [BH, M64, K64]
  int32_t* cnt64;      // [BH, M64]
  uint64_t* sub64;     // [BH, M64, K64] (merge only)
  int32_t Mb, M64, Mk64, kmax, K64, r;
};

__global__ __launch_bounds__(64) void relist_expand_kernel(RelistArgs a) {
  const int64_t row = blockIdx.x;  // bh * M64 + i64
  const int64_t bh = row / a.M64, i64 = row - bh * a.M64;
  const int64_t ib = i64 / a.r;
  int cnt = a.cnt[bh * a.Mb + ib];
  cnt = cnt < 0 ? 0 : (cnt > a.kmax ? a.kmax : cnt);
  const int32_t* src = a.idx + (bh * a.Mb + ib) * a.kmax;
  int32_t* dst = a.idx64 + row * a.K64;
  for (int e = threadIdx.x; e < cnt * a.r; e += 64) {
    const int jb = src[e / a.r];
    const int64_t j64 = static_cast<int64_t>(jb) * a.r + e % a.r;
    dst[e] = jb >= 0 && jb < a.Mb && j64 < a.Mk64 ? static_cast<int32_t>(j64) : -1;
  }
  if (threadIdx.x == 0) a.cnt64[row] = cnt * a.r;
}

__global__ __launch_bounds__(64) void relist_merge_kernel(RelistArgs a) {
  extern __shared__ __align__(16) unsigned char relist_lds[];
  uint64_t* lsub = reinterpret_cast<uint64_t*>(relist_lds);        // [K64]
  int32_t* lidx = reinterpret_cast<int32_t*>(lsub + a.K64);         // [K64]
  const int64_t row = blockIdx.x;
  const int64_t bh = row / a.M64, i64 = row - bh * a.M64;
  const int lane = lane_id();
  int n = 0;  // entries so far (uniform)
  for (int u = 0; u < a.r; ++u) {
    const int64_t ib = i64 * a.r + u;
    if (ib >= a.Mb) break;
    int cnt = a.cnt[bh * a.Mb + ib];
    cnt = cnt < 0 ? 0 : (cnt > a.kmax ? a.kmax : cnt);
    const int32_t* src = a.idx + (bh * a.Mb + ib) * a.kmax;
    for (int base = 0; base < cnt; base += 64) {
      const int x = base + lane < cnt ? src[base + lane] : -1;
      uint64_t vb = ballot64(x >= 0 && x < a.Mb);
      while (vb) {
        const int t = __builtin_ctzll(vb);
        vb &= vb - 1;
        const int jb = __builtin_amdgcn_readlane(x, t);
        const int j64 = jb / a.r;
        const uint64_t bit = 1ull << (u * a.r + jb % a.r);
        int found = -1;
        for (int ob = 0; ob < n && found < 0; ob += 64) {
          const int e = ob + lane;
          const bool hit = e < n && lidx[e] == j64 && (lsub[e] & bit) == 0;
          const uint64_t hb = ballot64(hit);
          if (hb) found = ob + __builtin_ctzll(hb);
        }
        if (lane == 0) {
          if (found >= 0) {
            lsub[found] |= bit;
          } else {
            lidx[n] = j64;
            lsub[n] = bit;
          }
        }
        n += found < 0 ? 1 : 0;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // visible to the next search
      }
    }
  }
  int32_t* didx = a.idx64 + row * a.K64;
  uint64_t* dsub = a.sub64 + row * a.K64;
  for (int e = lane; e < n; e += 64) {
    didx[e] = lidx[e];
    dsub[e] = lsub[e];
  }
  if (lane == 0) a.cnt64[row] = n;
}

// ---------------------------------------------------------------------------
// key_score_kernel: per-key attention totals (cab_attn_key_scores).
// score[k] = sum over queries t of softmax_t(k) = exp(s_tk - lse_t), with
// the natural-log lse of attn_fwd_kernel's rows. One workgroup of 4 waves per
// (b, h, group of 4 key blocks); wave w holds block 4 g + w's 64 keys as the
// B operand of S = Q K^T (K^T tiles in 16 registers x 4). The four waves walk
// the same 16-query tiles, last to first: each tile's Q (4 KB, MFMA operand order) and lse
// (16 floats, one copy per wave) are staged once per workgroup into a ring
// of 4 LDS stages by global_load_lds, three tiles ahead, so the texture path
// carries a quarter of the bytes per MFMA of one wave per key block. Per
// tile and wave:
//   S (16 queries x 64 keys) = 16 MFMA 16x16x32,
//   P = exp2(S c - lse log2 e) (fp32, masked entries 0),
//   column sums over the tile's queries, kept per lane.
// The lane partials are added once at the end in a fixed order (no
// atomics) and written to, or added into, score[b, h, keys of the block].
// fp32 inputs: the Q tile is staged in fp32 (two loads per stager lane) and
// every operand is split into bf16 hi / lo halves in registers; S takes
// three bf16 products per site, q_hi k_hi + q_lo k_hi + q_hi k_lo, as the
// executor's fp32 path does.
// ---------------------------------------------------------------------------
struct KeyScoreArgs {
  const void* q;
  const void* k;
  const float* lse;  // [B, H, Nq] contiguous
  float* score;      // score[b * ss0 + h * ss1 + token]
  int64_t qs[3], ks[3], ss[2];
  int32_t BH, H, group, Nq, Nk, Mk, Mkg, qoff, causal, accumulate;
  float scale_log2;
};

constexpr int KS_STAGES = 4;
constexpr int KS_WAVES = 4;  // key blocks (waves) sharing each staged query tile (8 measured slower)

// One ring stage: the Q tile (16 queries x D, 2 or 4 bytes per value), then
// one 64-float lse copy per wave.
template <int HD, bool F32>
constexpr int ks_q_bytes() { return (F32 ? 64 : 32) * HD; }
template <int HD, bool F32>
constexpr int ks_stage_bytes() { return ks_q_bytes<HD, F32>() + 4 * 256; }

template <cab_dtype_t DT, int NW, int HD>
__global__ __launch_bounds__(64 * NW) void key_score_kernel(KeyScoreArgs a) {
  constexpr int NDS = Dims<HD>::NDS;
  constexpr bool F32 = DT == CAB_F32;
  constexpr bool BF16 = DT != CAB_F16;
  constexpr int KS_STAGE_BYTES = ks_stage_bytes<HD, F32>();
  constexpr int QB = ks_q_bytes<HD, F32>();
  constexpr int ESZ = F32 ? 4 : 2;
  __shared__ __attribute__((aligned(16))) char ring[KS_STAGES * KS_STAGE_BYTES];
  const int logical = static_cast<int>(xcd_remap(blockIdx.x, static_cast<int64_t>(a.BH) * a.Mkg));
  const int bh = logical / a.Mkg;
  const int jg = logical - bh * a.Mkg;  // causal: group 0 sees the most queries, first
  const int b = bh / a.H, hh = bh - (bh / a.H) * a.H;
  const int hk = hh / a.group;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int lane = lane_id(), l16 = lane & 15, g = lane >> 4;
  const int j = NW * jg + w;  // this wave's key block (none when j >= Mk)
  const float c = a.scale_log2;
  constexpr float LOG2E = 1.4426950408889634f;

  const char* qb = static_cast<const char*>(a.q) + (b * a.qs[0] + hh * a.qs[1]) * ESZ;
  const char* kb = static_cast<const char*>(a.k) + (b * a.ks[0] + hk * a.ks[1]) * ESZ;
  const float* lb = a.lse + static_cast<int64_t>(bh) * a.Nq;

  // K^T operand: kop[kt][ds] = K[16 kt + l16][32 ds + 8 g .. +8] (zero past
  // Nk); fp32: its hi half, klo the lo half.
  u32x4 kop[4][NDS];
  u32x4 klo[4][F32 ? NDS : 1];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    const int key = j * BS + 16 * kt + l16;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      const char* kp = kb + (key * a.ks[2] + 32 * ds + 8 * g) * ESZ;
      if constexpr (F32) {
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        const f32x4 x0 = key < a.Nk ? *reinterpret_cast<const f32x4*>(kp) : zero;
        const f32x4 x1 = key < a.Nk ? *reinterpret_cast<const f32x4*>(kp + 16) : zero;
        split8(x0, x1, kop[kt][ds], klo[kt][ds]);
      } else {
        kop[kt][ds] = key < a.Nk ? *reinterpret_cast<const u32x4*>(kp) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  // Query tiles that see the group's first block, and this wave's first.
  auto first_tile = [&](int blk) {
    const int t_first = a.causal ? blk * BS - a.qoff : 0;
    return t_first <= 0 ? 0 : t_first / 16;
  };
  const int tile0 = first_tile(NW * jg);
  const int my0 = first_tile(j);
  const int ntiles = (a.Nq + 15) / 16;
  const int nt = ntiles > tile0 ? ntiles - tile0 : 0;

  // Tiles are walked from the last one down, so the workgroups of a head,
  // which start together, read the same tiles at about the same time (L2).
  auto tile_of = [&](int it) { return ntiles - 1 - it; };
  // Staging of tile tile_of(it): wave w < NDS moves Q dims 32 w .. 32 w + 31
  // of the tile's 16 queries (lane L: query L % 16, dims 32 w + 8 (L / 16)
  // .. + 7, landing at 16 L: the A operand of MFMA k-step w; fp32: dims
  // .. + 3 at 2048 w + 16 L and .. + 4 .. + 7 at 1024 bytes past them); waves
  // w < 4 move lse copy w (one load per tile for waves NDS .. 3); waves
  // 4 .. 7 (NW = 8) stage nothing and read lse copy w % 4.
  // The loads go through a buffer descriptor per tile (its 16 rows; rows
  // past N_q read as zero and are masked below), so a lane's offsets are the
  // same for every tile and the staging costs no vector instructions.
  const bool stager = w < 4;
  const bool qstager = w < NDS;
  const uint32_t qrow = static_cast<uint32_t>(a.qs[2] * ESZ);  // below 2^27 (host check)
  const uint32_t q_voff = static_cast<uint32_t>(l16) * qrow + static_cast<uint32_t>((32 * w + 8 * g) * ESZ);
  auto issue = [&](int it) {
    if (!stager) return;
    char* st = ring + (it % KS_STAGES) * KS_STAGE_BYTES;
    const int q0 = 16 * tile_of(it);
    const uint32_t rows = static_cast<uint32_t>(min(16, a.Nq - q0));
    if (qstager) {
      const brsrc_t qrs = make_rsrc(qb + static_cast<int64_t>(q0) * a.qs[2] * ESZ, rows * qrow);
      if constexpr (F32) {
        bdma16(qrs, q_voff, 0, st + 2048 * w);
        bdma16(qrs, q_voff + 16u, 0, st + 2048 * w + 1024);
      } else {
        bdma16(qrs, q_voff, 0, st + 1024 * w);
      }
    }
    const brsrc_t lrs = make_rsrc(lb + q0, 4u * rows);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(lrs, (lds_void*)(st + QB + 256 * w), 4, 4u * l16, 0, 0, 0);
  };

  float colsum[4] = {0.f, 0.f, 0.f, 0.f};
  const bool has_keys = j < a.Mk;
  for (int it = 0; it < KS_STAGES - 1 && it < nt; ++it) issue(it);
  // Tile it lives in stage it % 4, a compile-time constant below, so the
  // compiler sees the staging of tile it + 3 cannot alias this tile's reads.
  auto step = [&](int it, auto stage_tag) {
    constexpr int S = decltype(stage_tag)::value;
    const int ahead = stager ? nt - 1 - it : 0;  // tiles it + 1, it + 2 may be in flight
    // A Q stager has two loads per tile in flight (fp32: three), an
    // lse-only stager one.
    if (ahead >= 2) {
      if (qstager)
        __builtin_amdgcn_s_waitcnt(F32 ? 0x0f76 : 0x0f74);  // vmcnt(6) / vmcnt(4)
      else
        __builtin_amdgcn_s_waitcnt(0x0f72);  // vmcnt(2)
    } else if (ahead == 1) {
      if (qstager)
        __builtin_amdgcn_s_waitcnt(F32 ? 0x0f73 : 0x0f72);  // vmcnt(3) / vmcnt(2)
      else
        __builtin_amdgcn_s_waitcnt(0x0f71);  // vmcnt(1)
    } else {
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    }
    __builtin_amdgcn_s_barrier();  // every wave's part of tile it landed; stage (S + 3) % 4 is free
    if (it + KS_STAGES - 1 < nt) issue(it + KS_STAGES - 1);
    const int tile = tile_of(it);
    if (!has_keys || tile < my0) return;
    const char* st = ring + S * KS_STAGE_BYTES;
    u32x4 qop[NDS];
    u32x4 qlo[F32 ? NDS : 1];
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      if constexpr (F32) {
        const f32x4 x0 = reinterpret_cast<const f32x4*>(st + 2048 * ds)[lane];
        const f32x4 x1 = reinterpret_cast<const f32x4*>(st + 2048 * ds + 1024)[lane];
        split8(x0, x1, qop[ds], qlo[ds]);
      } else {
        qop[ds] = reinterpret_cast<const u32x4*>(st + 1024 * ds)[lane];
      }
    }
    const f32x4 lv = reinterpret_cast<const f32x4*>(st + QB + 256 * (w & 3))[g];
    float nl[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) nl[r] = -lv[r] * LOG2E;
    f32x4 sc[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      sc[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < NDS; ++ds) {
        if constexpr (F32) {
          sc[kt] = mfma16<true>(qlo[ds], kop[kt][ds], sc[kt]);
          sc[kt] = mfma16<true>(qop[ds], klo[kt][ds], sc[kt]);
        }
        sc[kt] = mfma16<BF16>(qop[ds], kop[kt][ds], sc[kt]);
      }
    }
    // sc[kt][r]: query 16 tile + 4 g + r, key j BS + 16 kt + l16.
    const int t0 = 16 * tile + 4 * g;
    const bool edge = 16 * tile + 15 >= a.Nq || (j + 1) * BS > a.Nk ||
                      (a.causal && j * BS + BS - 1 > 16 * tile + a.qoff);
    // Two loops behind one uniform branch: written as one loop with the
    // edge test inside, the compiler branched around every element.
    if (!edge) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) colsum[kt] += __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kt][r], c, nl[r]));
    } else {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const int key = j * BS + 16 * kt + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = t0 + r;
          const bool drop = t >= a.Nq || key >= a.Nk || (a.causal && key > t + a.qoff);
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kt][r], c, nl[r]));
          colsum[kt] += drop ? 0.f : p;
        }
      }
    }
  };
  for (int it = 0; it < nt; it += KS_STAGES) {
    step(it, std::integral_constant<int, 0>{});
    if (it + 1 < nt) step(it + 1, std::integral_constant<int, 1>{});
    if (it + 2 < nt) step(it + 2, std::integral_constant<int, 2>{});
    if (it + 3 < nt) step(it + 3, std::integral_constant<int, 3>{});
  }
  // Key 16 kt + l16: add the four query-lane groups (lanes l16 + 16 g) in a
  // fixed order; lane l writes key l of the block.
  float mine = 0.f;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    float sum = colsum[kt];
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    if (g == kt) mine = sum;
  }
  const int key = j * BS + lane;
  if (has_keys && key < a.Nk) {
    float* dst = a.score + b * a.ss[0] + hh * a.ss[1] + key;
    *dst = a.accumulate ? *dst + mine : mine;
  }
}

}  // namespace
}  // namespace cab

using namespace cab;

namespace {

// Shape and scalar checks shared by the three entry points. fp32 is accepted
// by cab_block_sparse_attn_fwd only (its packed form holds K as well as V).
// Block sizes the executor takes: 64, its multiples 128 and 256 (lists
// expanded to 64-token tiles) and 8, 16, 32 (tiles with sub-tile masks).
bool executor_block_size(int64_t bs) {
  return bs == 8 || bs == 16 || bs == 32 || bs == 64 || bs == 128 || bs == 256;
}
constexpr int64_t MERGE_K64_MAX = 4096;  // merged 64-tile entries per row (LDS of the merge)

cab_status_t check_common(const char* fn, cab_dtype_t dtype, int64_t B, int64_t H, int64_t N,
                          int64_t D, int32_t block_size, bool allow_f32, bool any_bs = false) {
  if (allow_f32)
    CAB_REQUIRE(dtype == CAB_BF16 || dtype == CAB_F16 || dtype == CAB_F32, CAB_EDTYPE,
                "%s: dtype %d unsupported (bf16, fp16 or fp32)", fn, (int)dtype);
  else
    CAB_REQUIRE(dtype == CAB_BF16 || dtype == CAB_F16, CAB_EDTYPE,
                "%s: dtype %d unsupported (bf16 or fp16; fp32 runs through "
                "cab_block_sparse_attn_fwd)", fn, (int)dtype);
  CAB_REQUIRE(B >= 0 && H >= 0 && N >= 0, CAB_ESHAPE, "%s: negative size", fn);
  CAB_REQUIRE(D == 64 || D == 128, CAB_ESHAPE, "%s: head dim %lld unsupported (64 or 128)", fn,
              (long long)D);
  if (any_bs)
    CAB_REQUIRE(executor_block_size(block_size), CAB_ESHAPE,
                "%s: block_size %d unsupported (8, 16, 32, 64, 128 or 256)", fn, (int)block_size);
  else
    CAB_REQUIRE(block_size == BS, CAB_ESHAPE, "%s: block_size %d unsupported (64)", fn,
                (int)block_size);
  const int64_t M = ceil_div(N, BS);
  CAB_REQUIRE(B * H * M <= INT32_MAX && B * H <= 65535 && N <= INT32_MAX - BS, CAB_ESHAPE,
              "%s: problem too large (B*H <= 65535, B*H*M < 2^31, N < 2^31 - 64)", fn);
  return CAB_OK;
}

cab_status_t check_tensor(const char* fn, const char* name, const void* ptr,
                          const int64_t* strides, int64_t esize) {
  CAB_REQUIRE(ptr != nullptr, CAB_EINVAL, "%s: null %s", fn, name);
  CAB_REQUIRE(strides != nullptr, CAB_EINVAL, "%s: null %s strides", fn, name);
  CAB_REQUIRE(strides[3] == 1, CAB_ESHAPE, "%s: %s last-dim stride must be 1", fn, name);
  CAB_REQUIRE(reinterpret_cast<uintptr_t>(ptr) % 16 == 0, CAB_ESHAPE,
              "%s: %s not 16-byte aligned", fn, name);
  for (int d = 0; d < 3; ++d)
    CAB_REQUIRE(strides[d] >= 0 && (strides[d] * esize) % 16 == 0, CAB_ESHAPE,
                "%s: %s stride[%d]=%lld must keep rows 16-byte aligned", fn, name, d,
                (long long)strides[d]);
  return CAB_OK;
}

cab_status_t check_packed(const char* fn, const void* vt, size_t bytes, int64_t B, int64_t H,
                          int64_t M, cab_dtype_t dtype, int64_t D) {
  const size_t need = static_cast<size_t>(B * H * M) * block_bytes(dtype, static_cast<int>(D));
  CAB_REQUIRE(vt != nullptr && bytes >= need, CAB_EWORKSPACE,
              "%s: workspace of %zu bytes given, %zu needed", fn, bytes, need);
  CAB_REQUIRE(reinterpret_cast<uintptr_t>(vt) % 16 == 0, CAB_EWORKSPACE,
              "%s: workspace not 16-byte aligned", fn);
  return CAB_OK;
}

cab_status_t check_attn(const char* fn, const void* q, const void* k, const int64_t* q_strides,
                        const int64_t* k_strides, const int64_t* o_strides, void* out,
                        const int32_t* kv_idx, const int32_t* kv_cnt, int32_t kmax, float scale,
                        int64_t esize) {
  CAB_REQUIRE(kmax >= 1, CAB_EINVAL, "%s: kmax=%d must be >= 1", fn, (int)kmax);
  CAB_REQUIRE(std::isfinite(scale) && scale > 0.f, CAB_EINVAL, "%s: scale must be finite and > 0",
              fn);
  CAB_REQUIRE(kv_idx != nullptr && kv_cnt != nullptr, CAB_EINVAL, "%s: null block list", fn);
  cab_status_t st;
  if ((st = check_tensor(fn, "q", q, q_strides, esize)) != CAB_OK) return st;
  if ((st = check_tensor(fn, "k", k, k_strides, esize)) != CAB_OK) return st;
  if ((st = check_tensor(fn, "out", out, o_strides, esize)) != CAB_OK) return st;
  CAB_REQUIRE(k_strides[2] <= (int64_t{1} << 24), CAB_ESHAPE,
              "%s: k token stride %lld too large (<= 2^24 elements)", fn, (long long)k_strides[2]);
  return CAB_OK;
}

cab_status_t launch_pack(const char* fn, const void* v, const int64_t* v_strides, int64_t B,
                         int64_t H, int64_t N, int64_t D, void* vt, hipStream_t s) {
  PackArgs p;
  p.v = static_cast<const uint16_t*>(v);
  p.vt = static_cast<uint16_t*>(vt);
  for (int d = 0; d < 3; ++d) p.vs[d] = v_strides[d];
  p.H = H;
  p.N = N;
  p.M = ceil_div(N, BS);
  const dim3 grid(static_cast<unsigned>(p.M), static_cast<unsigned>(B * H));
  if (D == 64)
    pack_vt_kernel<64><<<grid, 256, 0, s>>>(p);
  else
    pack_vt_kernel<128><<<grid, 256, 0, s>>>(p);
  return launch_status(fn);
}

cab_status_t launch_pack_split(const char* fn, const void* k, const int64_t* k_strides,
                               const void* v, const int64_t* v_strides, int64_t B, int64_t H,
                               int64_t N, int64_t D, void* img, hipStream_t s) {
  SplitPackArgs p;
  p.k = static_cast<const float*>(k);
  p.v = static_cast<const float*>(v);
  p.img = static_cast<uint16_t*>(img);
  for (int d = 0; d < 3; ++d) {
    p.ks[d] = k_strides[d];
    p.vs[d] = v_strides[d];
  }
  p.H = H;
  p.N = N;
  p.M = ceil_div(N, BS);
  const dim3 grid(static_cast<unsigned>(p.M), static_cast<unsigned>(B * H));
  if (D == 64)
    pack_split_kernel<64><<<grid, 256, 0, s>>>(p);
  else
    pack_split_kernel<128><<<grid, 256, 0, s>>>(p);
  return launch_status(fn);
}

// Whether the row-pair kernel may run (development switch: CAB_ATTN_PAIR=0
// keeps every call on attn_fwd_kernel).
bool pair_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("CAB_ATTN_PAIR");
    return !(e && e[0] == '0');
  }();
  return on;
}

template <cab_dtype_t DT, int HD>
void launch_attn_kernel(int list, dim3 grid, hipStream_t s, const AttnArgs& a) {
  if (list == LIST_LDS)
    attn_fwd_kernel<DT, LIST_LDS, HD><<<grid, 256, 0, s>>>(a);
  else if (list == LIST_GLOBAL)
    attn_fwd_kernel<DT, LIST_GLOBAL, HD><<<grid, 256, 0, s>>>(a);
  else
    attn_fwd_kernel<DT, LIST_DENSE, HD><<<grid, 256, 0, s>>>(a);
}

// Problem geometry of one executor call: query heads H over Hkv K / V heads,
// Nq query and Nk key tokens, head dim D, the causal offset and the list mode.
struct AttnGeom {
  int64_t B, H, Hkv, Nq, Nk, D;
  int64_t qoff;
  int list;
};

cab_status_t launch_attn(const char* fn, const void* q, const void* k, const void* vt,
                         cab_dtype_t dtype, const AttnGeom& g, const int64_t* q_strides,
                         const int64_t* k_strides, const int64_t* o_strides,
                         const int32_t* kv_idx, const int32_t* kv_cnt, int32_t kmax, float scale,
                         int causal, void* out, float* lse, hipStream_t s,
                         const uint64_t* submask = nullptr, int sub_shift = 0) {
  const int64_t M = ceil_div(g.Nq, BS);
  AttnArgs a;
  a.q = q;
  a.k = static_cast<const uint16_t*>(k);
  a.vt = static_cast<const uint16_t*>(vt);
  a.o = out;
  a.lse = lse;
  for (int d = 0; d < 3; ++d) {
    a.qs[d] = q_strides[d];
    a.ks[d] = k_strides[d];
    a.os[d] = o_strides[d];
  }
  a.kv_idx = kv_idx;
  a.kv_cnt = kv_cnt;
  a.BH = static_cast<int32_t>(g.B * g.H);
  a.H = static_cast<int32_t>(g.H);
  a.N = static_cast<int32_t>(g.Nq);
  a.M = static_cast<int32_t>(M);
  a.Nk = static_cast<int32_t>(g.Nk);
  a.Mk = static_cast<int32_t>(ceil_div(g.Nk, BS));
  a.group = static_cast<int32_t>(g.H / g.Hkv);
  a.qoff = static_cast<int32_t>(g.qoff);
  a.kmax = kmax;
  a.scale_log2 = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
  a.causal = causal ? 1 : 0;
  a.submask = submask;
  a.sub_shift = sub_shift;
  if (dtype != CAB_F32 && submask == nullptr && pair_enabled() &&
      ((g.list == LIST_LDS && kmax <= PAIR_KMAX) || g.list == LIST_DENSE)) {
    const dim3 pgrid(static_cast<unsigned>(g.B * g.H * ((M + 1) / 2)));
    auto go = [&](auto dt_tag, auto hd_tag) {
      constexpr cab_dtype_t DT = decltype(dt_tag)::value;
      constexpr int HD = decltype(hd_tag)::value;
      if (g.list == LIST_DENSE)
        attn_pair_kernel<DT, LIST_DENSE, HD><<<pgrid, 256, 0, s>>>(a);
      else
        attn_pair_kernel<DT, LIST_LDS, HD><<<pgrid, 256, 0, s>>>(a);
    };
    using BF = std::integral_constant<cab_dtype_t, CAB_BF16>;
    using FH = std::integral_constant<cab_dtype_t, CAB_F16>;
    using D64 = std::integral_constant<int, 64>;
    using D128 = std::integral_constant<int, 128>;
    if (g.D == 64) {
      if (dtype == CAB_BF16) go(BF{}, D64{}); else go(FH{}, D64{});
    } else {
      if (dtype == CAB_BF16) go(BF{}, D128{}); else go(FH{}, D128{});
    }
    return launch_status(fn);
  }
  const dim3 grid(static_cast<unsigned>(g.B * g.H * M));
  if (g.D == 64) {
    if (dtype == CAB_BF16)
      launch_attn_kernel<CAB_BF16, 64>(g.list, grid, s, a);
    else if (dtype == CAB_F16)
      launch_attn_kernel<CAB_F16, 64>(g.list, grid, s, a);
    else
      launch_attn_kernel<CAB_F32, 64>(g.list, grid, s, a);
  } else {
    if (dtype == CAB_BF16)
      launch_attn_kernel<CAB_BF16, 128>(g.list, grid, s, a);
    else if (dtype == CAB_F16)
      launch_attn_kernel<CAB_F16, 128>(g.list, grid, s, a);
    else
      launch_attn_kernel<CAB_F32, 128>(g.list, grid, s, a);
  }
  return launch_status(fn);
}

// The sparse entry points: one K / V head per query head, Nq = Nk = N.
AttnGeom sparse_geom(int64_t B, int64_t H, int64_t N, int64_t D, int32_t kmax) {
  return AttnGeom{B, H, H, N, N, D, 0, kmax <= LIST_MAX ? LIST_LDS : LIST_GLOBAL};
}

// The 64-tile lists of a block size other than 64, in the workspace after
// the packed V: idx64 [BH, M64, K64], cnt64 [BH, M64], and for sizes below
// 64 the sub-tile masks [BH, M64, K64], each part 256-byte aligned.
struct TileLists {
  int64_t r, K64, M64;
  size_t off_idx, off_cnt, off_sub, end;
};
TileLists tile_lists(int64_t B, int64_t H, int64_t N, int32_t bs, int32_t kmax, size_t base) {
  TileLists t;
  t.r = bs >= BS ? bs / BS : BS / bs;
  t.K64 = static_cast<int64_t>(kmax) * t.r;
  t.M64 = ceil_div(N, BS);
  const int64_t rows = B * H * t.M64;
  t.off_idx = static_cast<size_t>(round_up(static_cast<int64_t>(base), 256));
  t.off_cnt = t.off_idx + static_cast<size_t>(round_up(rows * t.K64 * 4, 256));
  t.off_sub = t.off_cnt + static_cast<size_t>(round_up(rows * 4, 256));
  t.end = t.off_sub + (bs < BS ? static_cast<size_t>(rows * t.K64 * 8) : 0);
  return t;
}

}  // namespace

extern "C" size_t cab_block_sparse_attn_workspace_bytes_k(cab_dtype_t dtype, int64_t B, int64_t H,
                                                          int64_t N, int64_t D, int32_t block_size,
                                                          int32_t kmax) {
  if (dtype != CAB_BF16 && dtype != CAB_F16 && dtype != CAB_F32) return 0;
  if (B <= 0 || H <= 0 || N <= 0 || (D != 64 && D != 128) || !executor_block_size(block_size) ||
      kmax < 1)
    return 0;
  const size_t packed =
      static_cast<size_t>(B * H * ceil_div(N, BS)) * block_bytes(dtype, static_cast<int>(D));
  if (block_size == BS) return packed;
  return tile_lists(B, H, N, block_size, kmax, packed).end;
}

extern "C" size_t cab_block_sparse_attn_workspace_bytes(cab_dtype_t dtype, int64_t B, int64_t H,
                                                        int64_t N, int64_t D, int32_t block_size) {
  if (dtype != CAB_BF16 && dtype != CAB_F16 && dtype != CAB_F32) return 0;
  if (B <= 0 || H <= 0 || N <= 0 || (D != 64 && D != 128) || block_size != BS) return 0;
  return static_cast<size_t>(B * H * ceil_div(N, BS)) * block_bytes(dtype, static_cast<int>(D));
}

extern "C" cab_status_t cab_block_sparse_attn_pack_v(const void* v, cab_dtype_t dtype, int64_t B,
                                                     int64_t H, int64_t N, int64_t D,
                                                     const int64_t v_strides[4],
                                                     int32_t block_size, void* workspace,
                                                     size_t workspace_bytes, void* stream) {
  const char* fn = "cab_block_sparse_attn_pack_v";
  clear_error();
  cab_status_t st = check_common(fn, dtype, B, H, N, D, block_size, false);
  if (st != CAB_OK) return st;
  const int64_t M = ceil_div(N, BS);
  if (B == 0 || H == 0 || M == 0) return CAB_OK;
  if ((st = check_tensor(fn, "v", v, v_strides, 2)) != CAB_OK) return st;
  if ((st = check_packed(fn, workspace, workspace_bytes, B, H, M, dtype, D)) != CAB_OK) return st;
  return launch_pack(fn, v, v_strides, B, H, N, D, workspace, static_cast<hipStream_t>(stream));
}

extern "C" cab_status_t cab_block_sparse_attn_fwd_packed(
    const void* q, const void* k, const void* vt, cab_dtype_t dtype, int64_t B, int64_t H,
    int64_t N, int64_t D, const int64_t q_strides[4], const int64_t k_strides[4],
    const int64_t o_strides[4], int32_t block_size, const int32_t* kv_idx,
    const int32_t* kv_cnt, int32_t kmax, float scale, int causal, void* out, float* lse,
    size_t vt_bytes, void* stream) {
  const char* fn = "cab_block_sparse_attn_fwd_packed";
  clear_error();
  cab_status_t st = check_common(fn, dtype, B, H, N, D, block_size, false);
  if (st != CAB_OK) return st;
  const int64_t M = ceil_div(N, BS);
  if (B == 0 || H == 0 || M == 0) return CAB_OK;
  if ((st = check_attn(fn, q, k, q_strides, k_strides, o_strides, out, kv_idx, kv_cnt, kmax,
                       scale, 2)) != CAB_OK)
    return st;
  if ((st = check_packed(fn, vt, vt_bytes, B, H, M, dtype, D)) != CAB_OK) return st;
  return launch_attn(fn, q, k, vt, dtype, sparse_geom(B, H, N, D, kmax), q_strides, k_strides,
                     o_strides, kv_idx, kv_cnt, kmax, scale, causal, out, lse,
                     static_cast<hipStream_t>(stream));
}

extern "C" cab_status_t cab_block_sparse_attn_fwd(
    const void* q, const void* k, const void* v, cab_dtype_t dtype, int64_t B, int64_t H,
    int64_t N, int64_t D, const int64_t q_strides[4], const int64_t k_strides[4],
    const int64_t v_strides[4], const int64_t o_strides[4], int32_t block_size,
    const int32_t* kv_idx, const int32_t* kv_cnt, int32_t kmax, float scale, int causal,
    void* out, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "cab_block_sparse_attn_fwd";
  clear_error();
  cab_status_t st = check_common(fn, dtype, B, H, N, D, block_size, true, true);
  if (st != CAB_OK) return st;
  CAB_REQUIRE(kmax >= 1, CAB_EINVAL, "%s: kmax=%d must be >= 1", fn, (int)kmax);
  if (block_size < BS)
    CAB_REQUIRE(static_cast<int64_t>(kmax) * (BS / block_size) <= MERGE_K64_MAX, CAB_ESHAPE,
                "%s: block_size %d takes lists of at most %lld entries (kmax=%d)", fn,
                (int)block_size, (long long)(MERGE_K64_MAX / (BS / block_size)), (int)kmax);
  if (block_size > BS)
    CAB_REQUIRE(static_cast<int64_t>(kmax) * (block_size / BS) <= INT32_MAX / 2, CAB_ESHAPE,
                "%s: kmax=%d too large for block_size %d", fn, (int)kmax, (int)block_size);
  CAB_REQUIRE(std::isfinite(scale) && scale > 0.f, CAB_EINVAL, "%s: scale must be finite and > 0",
              fn);
  CAB_REQUIRE(q_strides && k_strides && v_strides && o_strides, CAB_EINVAL,
              "%s: null stride array", fn);
  const int64_t M = ceil_div(N, BS);
  if (B == 0 || H == 0 || M == 0) return CAB_OK;
  const int64_t esize = dtype == CAB_F32 ? 4 : 2;
  if ((st = check_attn(fn, q, k, q_strides, k_strides, o_strides, out, kv_idx, kv_cnt, kmax,
                       scale, esize)) != CAB_OK)
    return st;
  if ((st = check_tensor(fn, "v", v, v_strides, esize)) != CAB_OK) return st;
  if ((st = check_packed(fn, workspace, workspace_bytes, B, H, M, dtype, D)) != CAB_OK) return st;
  const size_t packed = static_cast<size_t>(B * H * M) * block_bytes(dtype, static_cast<int>(D));
  TileLists tl{};
  if (block_size != BS) {
    tl = tile_lists(B, H, N, block_size, kmax, packed);
    CAB_REQUIRE(workspace_bytes >= tl.end, CAB_EWORKSPACE,
                "%s: workspace of %zu bytes given, %zu needed for block_size %d and kmax %d "
                "(cab_block_sparse_attn_workspace_bytes_k)", fn, workspace_bytes, tl.end,
                (int)block_size, (int)kmax);
    CAB_REQUIRE(B * H * tl.M64 * tl.K64 <= INT64_C(1) << 40, CAB_ESHAPE, "%s: lists too large", fn);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (block_size != BS) {
    char* ws = static_cast<char*>(workspace);
    RelistArgs ra;
    ra.idx = kv_idx;
    ra.cnt = kv_cnt;
    ra.idx64 = reinterpret_cast<int32_t*>(ws + tl.off_idx);
    ra.cnt64 = reinterpret_cast<int32_t*>(ws + tl.off_cnt);
    ra.sub64 = block_size < BS ? reinterpret_cast<uint64_t*>(ws + tl.off_sub) : nullptr;
    ra.Mb = static_cast<int32_t>(ceil_div(N, block_size));
    ra.M64 = static_cast<int32_t>(tl.M64);
    ra.Mk64 = static_cast<int32_t>(tl.M64);
    ra.kmax = kmax;
    ra.K64 = static_cast<int32_t>(tl.K64);
    ra.r = static_cast<int32_t>(tl.r);
    const dim3 rgrid(static_cast<unsigned>(B * H * tl.M64));
    if (block_size > BS) {
      relist_expand_kernel<<<rgrid, 64, 0, s>>>(ra);
    } else {
      const size_t lds = static_cast<size_t>(tl.K64) * 12;
      relist_merge_kernel<<<rgrid, 64, lds, s>>>(ra);
    }
    if ((st = launch_status("cab_block_sparse_attn_fwd/relist")) != CAB_OK) return st;
  }
  if (dtype == CAB_F32)
    st = launch_pack_split("cab_block_sparse_attn_fwd/pack_split", k, k_strides, v, v_strides, B,
                           H, N, D, workspace, s);
  else
    st = launch_pack("cab_block_sparse_attn_fwd/pack_v", v, v_strides, B, H, N, D, workspace, s);
  if (st != CAB_OK) return st;
  if (block_size != BS) {
    const char* ws = static_cast<const char*>(workspace);
    int sh = 0;
    while ((1 << sh) < block_size) ++sh;
    return launch_attn(fn, q, k, workspace, dtype,
                       sparse_geom(B, H, N, D, static_cast<int32_t>(tl.K64)), q_strides,
                       k_strides, o_strides, reinterpret_cast<const int32_t*>(ws + tl.off_idx),
                       reinterpret_cast<const int32_t*>(ws + tl.off_cnt),
                       static_cast<int32_t>(tl.K64), scale, causal, out, lse, s,
                       block_size < BS ? reinterpret_cast<const uint64_t*>(ws + tl.off_sub) : nullptr,
                       sh);
  }
  return launch_attn(fn, q, k, workspace, dtype, sparse_geom(B, H, N, D, kmax), q_strides, k_strides,
                     o_strides, kv_idx, kv_cnt, kmax, scale, causal, out, lse, s);
}

// ---------------------------------------------------------------------------
// Dense attention with per-key scores (the eviction path's fused kernel).
// ---------------------------------------------------------------------------

namespace {

// Shape checks of the dense entry points: H query heads over H_kv K / V
// heads (H % H_kv == 0), N_q queries, N_k keys, D = 64 or 128.
cab_status_t check_dense(const char* fn, cab_dtype_t dtype, bool allow_f32, int64_t B, int64_t H,
                         int64_t H_kv, int64_t N_q, int64_t N_k, int64_t D) {
  if (allow_f32)
    CAB_REQUIRE(dtype == CAB_BF16 || dtype == CAB_F16 || dtype == CAB_F32, CAB_EDTYPE,
                "%s: dtype %d unsupported (bf16, fp16 or fp32)", fn, (int)dtype);
  else
    CAB_REQUIRE(dtype == CAB_BF16 || dtype == CAB_F16, CAB_EDTYPE,
                "%s: dtype %d unsupported (bf16 or fp16)", fn, (int)dtype);
  CAB_REQUIRE(B >= 0 && H >= 0 && H_kv >= 0 && N_q >= 0 && N_k >= 0, CAB_ESHAPE,
              "%s: negative size", fn);
  CAB_REQUIRE(D == 64 || D == 128, CAB_ESHAPE, "%s: head dim %lld unsupported (64 or 128)", fn,
              (long long)D);
  CAB_REQUIRE(H_kv > 0 ? H % H_kv == 0 : H == 0, CAB_ESHAPE,
              "%s: %lld query heads are not a multiple of %lld K/V heads", fn, (long long)H,
              (long long)H_kv);
  CAB_REQUIRE(B * H * ceil_div(N_q, BS) <= INT32_MAX && B * H * ceil_div(N_k, BS) <= INT32_MAX &&
                  N_q <= INT32_MAX - BS && N_k <= INT32_MAX - BS,
              CAB_ESHAPE, "%s: problem too large (B*H*blocks < 2^31, N < 2^31 - 64)", fn);
  return CAB_OK;
}

}  // namespace

extern "C" size_t cab_flash_attn_workspace_bytes(cab_dtype_t dtype, int64_t B, int64_t H_kv,
                                                 int64_t N_k, int64_t D) {
  if (dtype != CAB_BF16 && dtype != CAB_F16 && dtype != CAB_F32) return 0;
  if (B <= 0 || H_kv <= 0 || N_k <= 0 || (D != 64 && D != 128)) return 0;
  return static_cast<size_t>(B * H_kv * ceil_div(N_k, BS)) * block_bytes(dtype, static_cast<int>(D));
}

extern "C" cab_status_t cab_flash_attn_fwd(
    const void* q, const void* k, const void* v, cab_dtype_t dtype, int64_t B, int64_t H,
    int64_t H_kv, int64_t N_q, int64_t N_k, int64_t D, const int64_t q_strides[4],
    const int64_t k_strides[4], const int64_t v_strides[4], const int64_t o_strides[4],
    float scale, int causal, void* out, float* lse, void* workspace, size_t workspace_bytes,
    void* stream) {
  const char* fn = "cab_flash_attn_fwd";
  clear_error();
  cab_status_t st = check_dense(fn, dtype, true, B, H, H_kv, N_q, N_k, D);
  if (st != CAB_OK) return st;
  CAB_REQUIRE(std::isfinite(scale) && scale > 0.f, CAB_EINVAL, "%s: scale must be finite and > 0",
              fn);
  CAB_REQUIRE(q_strides && k_strides && v_strides && o_strides, CAB_EINVAL,
              "%s: null stride array", fn);
  if (B == 0 || H == 0 || N_q == 0) return CAB_OK;
  const int64_t esize = dtype == CAB_F32 ? 4 : 2;
  if ((st = check_tensor(fn, "q", q, q_strides, esize)) != CAB_OK) return st;
  if ((st = check_tensor(fn, "out", out, o_strides, esize)) != CAB_OK) return st;
  CAB_REQUIRE(lse == nullptr || reinterpret_cast<uintptr_t>(lse) % 4 == 0, CAB_ESHAPE,
              "%s: lse not 4-byte aligned", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (N_k == 0 || H_kv == 0) {
    // No keys: every row attends to nothing (output 0, lse -inf); K, V and
    // the workspace are not read (q stands in for their addresses).
    const AttnGeom g{B, H, H_kv > 0 ? H_kv : H, N_q, 0, D, -N_q, LIST_DENSE};
    return launch_attn(fn, q, q, q, dtype, g, q_strides, q_strides, o_strides, nullptr, nullptr,
                       1, scale, causal, out, lse, s);
  }
  if ((st = check_tensor(fn, "k", k, k_strides, esize)) != CAB_OK) return st;
  if ((st = check_tensor(fn, "v", v, v_strides, esize)) != CAB_OK) return st;
  CAB_REQUIRE(k_strides[2] <= (int64_t{1} << 24), CAB_ESHAPE,
              "%s: k token stride %lld too large (<= 2^24 elements)", fn, (long long)k_strides[2]);
  const int64_t Mk = ceil_div(N_k, BS);
  const size_t need = static_cast<size_t>(B * H_kv * Mk) * block_bytes(dtype, static_cast<int>(D));
  CAB_REQUIRE(workspace != nullptr && workspace_bytes >= need, CAB_EWORKSPACE,
              "%s: workspace of %zu bytes given, %zu needed", fn, workspace_bytes, need);
  CAB_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, CAB_EWORKSPACE,
              "%s: workspace not 16-byte aligned", fn);
  if (dtype == CAB_F32)
    st = launch_pack_split("cab_flash_attn_fwd/pack_split", k, k_strides, v, v_strides, B, H_kv,
                           N_k, D, workspace, s);
  else
    st = launch_pack("cab_flash_attn_fwd/pack_v", v, v_strides, B, H_kv, N_k, D, workspace, s);
  if (st != CAB_OK) return st;
  const AttnGeom g{B, H, H_kv, N_q, N_k, D, N_k - N_q, LIST_DENSE};
  return launch_attn(fn, q, k, workspace, dtype, g, q_strides, k_strides, o_strides, nullptr,
                     nullptr, 1, scale, causal, out, lse, s);
}

extern "C" cab_status_t cab_attn_key_scores(
    const void* q, const void* k, const float* lse, cab_dtype_t dtype, int64_t B, int64_t H,
    int64_t H_kv, int64_t N_q, int64_t N_k, int64_t D, const int64_t q_strides[4],
    const int64_t k_strides[4], float scale, int causal, float* scores,
    const int64_t score_strides[3], int accumulate, void* stream) {
  const char* fn = "cab_attn_key_scores";
  clear_error();
  cab_status_t st = check_dense(fn, dtype, true, B, H, H_kv, N_q, N_k, D);
  if (st != CAB_OK) return st;
  CAB_REQUIRE(std::isfinite(scale) && scale > 0.f, CAB_EINVAL, "%s: scale must be finite and > 0",
              fn);
  CAB_REQUIRE(q_strides && k_strides && score_strides, CAB_EINVAL, "%s: null stride array", fn);
  const int64_t esize = dtype == CAB_F32 ? 4 : 2;
  if (B == 0 || H == 0 || N_k == 0) return CAB_OK;
  CAB_REQUIRE(scores != nullptr, CAB_EINVAL, "%s: null scores", fn);
  CAB_REQUIRE(score_strides[2] == 1 && score_strides[0] >= 0 && score_strides[1] >= 0,
              CAB_ESHAPE, "%s: scores must have a contiguous token dim", fn);
  if (N_q > 0) {
    if ((st = check_tensor(fn, "q", q, q_strides, esize)) != CAB_OK) return st;
    CAB_REQUIRE(lse != nullptr && reinterpret_cast<uintptr_t>(lse) % 4 == 0, CAB_EINVAL,
                "%s: lse must be the fp32 [B, H, N_q] rows cab_flash_attn_fwd wrote", fn);
    // 16 query rows are staged through one buffer descriptor (32-bit offsets).
    CAB_REQUIRE(q_strides[2] * esize < (int64_t{1} << 27), CAB_ESHAPE,
                "%s: q token stride of %lld elements exceeds the 2^27-byte limit", fn,
                (long long)q_strides[2]);
  }
  if ((st = check_tensor(fn, "k", k, k_strides, esize)) != CAB_OK) return st;
  KeyScoreArgs a;
  a.q = q;
  a.k = k;
  a.lse = lse;
  a.score = scores;
  for (int d = 0; d < 3; ++d) {
    a.qs[d] = q_strides[d];
    a.ks[d] = k_strides[d];
  }
  a.ss[0] = score_strides[0];
  a.ss[1] = score_strides[1];
  a.BH = static_cast<int32_t>(B * H);
  a.H = static_cast<int32_t>(H);
  a.group = static_cast<int32_t>(H / H_kv);
  a.Nq = static_cast<int32_t>(N_q);
  a.Nk = static_cast<int32_t>(N_k);
  a.Mk = static_cast<int32_t>(ceil_div(N_k, BS));
  a.Mkg = static_cast<int32_t>(ceil_div(a.Mk, KS_WAVES));
  a.qoff = static_cast<int32_t>(N_k - N_q);
  a.causal = causal ? 1 : 0;
  a.accumulate = accumulate ? 1 : 0;
  a.scale_log2 = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
  const dim3 grid(static_cast<unsigned>(B * H * a.Mkg));
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto launch = [&](auto hd_tag) {
    constexpr int HDT = decltype(hd_tag)::value;
    switch (dtype) {
      case CAB_BF16: key_score_kernel<CAB_BF16, KS_WAVES, HDT><<<grid, 64 * KS_WAVES, 0, s>>>(a); break;
      case CAB_F16: key_score_kernel<CAB_F16, KS_WAVES, HDT><<<grid, 64 * KS_WAVES, 0, s>>>(a); break;
      default: key_score_kernel<CAB_F32, KS_WAVES, HDT><<<grid, 64 * KS_WAVES, 0, s>>>(a); break;
    }
  };
  if (D == 64)
    launch(std::integral_constant<int, 64>{});
  else
    launch(std::integral_constant<int, 128>{});
  return launch_status(fn);
}
