// Coarse Forman-Ricci curvature (cab_block_frc).
//
// Pipeline per (b, h), Mp = M rounded up to 128:
//  1. STATS: A = qc kc^T * alpha on MFMA, min/max partials per tile or strip
//     (aff_strip_kernel for 16-bit inputs with D <= 128: strips of LDS-staged
//     128 x 128 tiles; affinity_stats_kernel otherwise: operands straight
//     from memory).
//  2. per-(b,h) min/max from the partials: inside aff_strip_kernel's EMIT
//     pass, minmax_finalize_kernel ahead of affinity_kernel.
//  3. EMIT (aff_strip_kernel / affinity_kernel): recomputes the A tile, normalises it, and writes
//     Ahat in row-major X and transposed XT planes (zero outside M), the fp32
//     Ahat diagnostic and, for the augmented formula, row-sum partials. The
//     planes hold either
//       - fp16 (minmax normalisation, additive or multiplicative formula):
//         Ahat lies in [0, 1], X = f16(Ahat), XT likewise, plus the low part
//         f16(Ahat - X) of X for the epilogue; for the additive formula
//         without the T diagnostic, XT = f16(I - lambda Ahat)^T instead, so
//         that the GEMM accumulates F = Ahat (I - lambda Ahat) itself; or
//       - a bf16 hi/lo pair (hi = bf16(Ahat), lo = bf16(Ahat - hi)) of X and
//         of XT, for unnormalised values of any range and for the augmented
//         formula, whose S_i + S_j cancels against 3 T.
//  4. rowsum_finalize_kernel (augmented only).
//  5. triangle_kernel: T = Ahat Ahat = X XT^T on MFMA with fp32 accumulate,
//     one fp16 product per site (relative error <= 2^-10 + 2^-22 per product
//     for Ahat in fp16's normal range) or hi*hi + hi*lo + lo*hi in bf16 (the
//     dropped lo*lo term is below 2^-16 relative); LDS double-buffered, with
//     the FRC combination fused into the epilogue.
// Algorithmic work: 2 M^2 D flops (affinity) + 2 M^3 flops (triangles).
#include <atomic>

#include "cab_internal.h"

namespace cab {
namespace {

constexpr int AT = 64;    // affinity quadrant (one wave; row-sum partials per AT columns)
constexpr int AW = 128;   // affinity tile per workgroup (2 x 2 quadrants)
constexpr int TT = 128;   // triangle tile
constexpr int TT_WIDE = 256;  // wide triangle tile (large M)
constexpr int TK = 32;    // triangle k-slice depth

struct FrcLayout {
  int64_t Mp, nta, ntw;  // padded M, AT column blocks and AW workgroup tiles per dim
  size_t plane;     // bytes of one [BH][Mp][Mp] bf16 plane
  size_t off_xhi, off_xlo, off_xthi, off_xtlo, off_mmpart, off_mm, off_rspart, off_rs, total;
};

FrcLayout frc_layout(int64_t BH, int64_t M) {
  FrcLayout L;
  L.Mp = round_up(M, TT);
  L.nta = L.Mp / AT;
  L.ntw = L.Mp / AW;
  L.plane = static_cast<size_t>(BH) * L.Mp * L.Mp * 2;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    size_t at = o;
    o += static_cast<size_t>(round_up(static_cast<int64_t>(bytes), 256));
    return at;
  };
  L.off_xhi = take(L.plane);
  L.off_xlo = take(L.plane);
  L.off_xthi = take(L.plane);
  L.off_xtlo = take(L.plane);
  L.off_mmpart = take(static_cast<size_t>(BH) * L.ntw * L.ntw * 2 * sizeof(float));
  L.off_mm = take(static_cast<size_t>(BH) * 2 * sizeof(float));
  L.off_rspart = take(static_cast<size_t>(BH) * L.nta * L.Mp * sizeof(float));
  L.off_rs = take(static_cast<size_t>(BH) * L.Mp * sizeof(float));
  L.total = o;
  return L;
}

struct AffArgs {
  const void* qc;
  const void* kc;
  int64_t M, Mp, nta, ntw;
  int32_t D;
  float alpha;
  int normalization;
  float* mmpart;       // [BH][nparts][2] min / max partials, nparts <= (Mp / 128)^2
  float* mm;           // [BH][2] min / max of alpha A
  int64_t nparts;      // min / max partials per (b, h)
  uint16_t* xhi;       // [BH][Mp][Mp]
  uint16_t* xlo;
  uint16_t* xthi;
  uint16_t* xtlo;
  float* affinity;     // [BH][M][M] or null
  float* rspart;       // [BH][nta][Mp] or null
  int f16_planes;      // X = f16, xlo = f16 low part of X, XT = f16 (xtlo unused)
  int fused;           // with f16_planes: XT = f16(I - lambda Ahat^T), xlo unused
  float lambda;
  int64_t strip;       // aff_strip_kernel: 128 x 128 tiles per workgroup
};

// One wave computes a 64 x 32 YT block of qc kc^T (fp32 accumulate) as
// 2 x YT MFMA tiles: acc[x][y] covers rows row0 + 32 x .., columns
// col0 + 32 y ..; lane l owns column l % 32 and rows 8 * (e / 4) +
// 4 * (l / 32) + e % 4 of each tile's element e.
template <typename T, int YT>
__device__ __forceinline__ void aff_block(const void* qcv, const void* kcv, int64_t row0,
                                          int64_t col0, int64_t M, int D, int lane,
                                          f32x16 (&acc)[2][YT]) {
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < YT; ++y) acc[x][y] = f32x16{};
  const int half = lane >> 5;
  int64_t r[2], c[YT];
  bool ra[2], cb[YT];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    r[x] = row0 + 32 * x + (lane & 31);
    ra[x] = r[x] < M;
  }
#pragma unroll
  for (int y = 0; y < YT; ++y) {
    c[y] = col0 + 32 * y + (lane & 31);
    cb[y] = c[y] < M;
  }
  if constexpr (sizeof(T) == 4) {
    // fp32: 32x32x2 MFMA; lane half h holds k = 8q + 4h + s in step s.
    const float* q = static_cast<const float*>(qcv);
    const float* k = static_cast<const float*>(kcv);
    for (int k0 = 0; k0 < D; k0 += 8) {
      f32x4 av[2], bv[YT];
#pragma unroll
      for (int x = 0; x < 2; ++x)
        av[x] = ra[x] ? *reinterpret_cast<const f32x4*>(q + r[x] * D + k0 + 4 * half) : f32x4{};
#pragma unroll
      for (int y = 0; y < YT; ++y)
        bv[y] = cb[y] ? *reinterpret_cast<const f32x4*>(k + c[y] * D + k0 + 4 * half) : f32x4{};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int y = 0; y < YT; ++y)
            acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[x][s], bv[y][s], acc[x][y], 0, 0, 0);
    }
  } else {
    const uint16_t* q = static_cast<const uint16_t*>(qcv);
    const uint16_t* k = static_cast<const uint16_t*>(kcv);
    for (int k0 = 0; k0 < D; k0 += 16) {
      const bool kin = k0 + 8 * half < D;  // D % 16 == 8: the upper half is past the row
      u32x4 av[2], bv[YT];
#pragma unroll
      for (int x = 0; x < 2; ++x)
        av[x] = ra[x] && kin ? *reinterpret_cast<const u32x4*>(q + r[x] * D + k0 + 8 * half) : u32x4{};
#pragma unroll
      for (int y = 0; y < YT; ++y)
        bv[y] = cb[y] && kin ? *reinterpret_cast<const u32x4*>(k + c[y] * D + k0 + 8 * half) : u32x4{};
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < YT; ++y) {
          if constexpr (std::is_same<T, bf16_t>::value)
            acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8, av[x]), __builtin_bit_cast(bf16x8, bv[y]), acc[x][y], 0, 0, 0);
          else
            acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                __builtin_bit_cast(f16x8, av[x]), __builtin_bit_cast(f16x8, bv[y]), acc[x][y], 0, 0, 0);
        }
    }
  }
}

__device__ __forceinline__ float normalize_minmax(float a, float mn, float mx) {
  return mx > mn ? (a - mn) / (mx - mn + 1e-8f) : a;
}

// STATS pass: per-tile min / max of A. A 256 x 256 tile per workgroup of 8
// waves; wave w computes rows 64 (w / 2) .., columns 128 (w % 2) .. as 2 x 4
// MFMA tiles (eight accumulators share each operand load).
constexpr int AS = 256;  // STATS tile per workgroup

template <typename T>
__global__ __launch_bounds__(512) void affinity_stats_kernel(AffArgs a) {
  const int64_t bh = blockIdx.y;
  const int64_t tile = blockIdx.x;
  const int64_t ns = (a.Mp + AS - 1) / AS;
  const int64_t ti = tile / ns, tj = tile - (tile / ns) * ns;
  const int w = threadIdx.x >> 6, lane = lane_id();
  const int64_t row0 = ti * AS + (w >> 1) * 64, col0 = tj * AS + (w & 1) * 128;
  const size_t esz = sizeof(T) == 4 ? 4 : 2;
  const char* qcb = static_cast<const char*>(a.qc) + static_cast<size_t>(bh) * a.M * a.D * esz;
  const char* kcb = static_cast<const char*>(a.kc) + static_cast<size_t>(bh) * a.M * a.D * esz;
  f32x16 acc[2][4];
  aff_block<T, 4>(qcb, kcb, row0, col0, a.M, a.D, lane, acc);
  const int half = lane >> 5;
  float mn = INFINITY, mx = -INFINITY;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t i = row0 + 32 * x + 8 * (e >> 2) + 4 * half + (e & 3);
        const int64_t j = col0 + 32 * y + (lane & 31);
        if (i < a.M && j < a.M) {
          const float v = acc[x][y][e] * a.alpha;
          mn = fminf(mn, v);
          mx = fmaxf(mx, v);
        }
      }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    mn = fminf(mn, shfl_xor_f32(mn, off));
    mx = fmaxf(mx, shfl_xor_f32(mx, off));
  }
  __shared__ float red[8][2];
  if (lane == 0) {
    red[w][0] = mn;
    red[w][1] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float m0 = red[0][0], m1 = red[0][1];
#pragma unroll
    for (int q = 1; q < 8; ++q) {
      m0 = fminf(m0, red[q][0]);
      m1 = fmaxf(m1, red[q][1]);
    }
    float* p = a.mmpart + (bh * ns * ns + tile) * 2;
    p[0] = m0;
    p[1] = m1;
  }
}

// EMIT pass: a 128 x 128 tile per workgroup; wave w computes quadrant
// (w / 2, w % 2), normalises it and writes the planes.
template <typename T>
__global__ __launch_bounds__(256) void affinity_kernel(AffArgs a) {
  const int64_t bh = blockIdx.y;
  const int64_t tile = blockIdx.x;
  const int64_t ti = tile / a.ntw, tj = tile - (tile / a.ntw) * a.ntw;
  const int w = threadIdx.x >> 6, lane = lane_id();
  const int wi = w >> 1, wj = w & 1;
  const int64_t row0 = ti * AW + wi * AT, col0 = tj * AW + wj * AT;
  const size_t esz = sizeof(T) == 4 ? 4 : 2;
  const char* qcb = static_cast<const char*>(a.qc) + static_cast<size_t>(bh) * a.M * a.D * esz;
  const char* kcb = static_cast<const char*>(a.kc) + static_cast<size_t>(bh) * a.M * a.D * esz;
  f32x16 acc[2][2];
  aff_block<T, 2>(qcb, kcb, row0, col0, a.M, a.D, lane, acc);

  const int half = lane >> 5;
  // Row and column of element e of MFMA tile (x, y), relative to the quadrant.
  auto qrow = [&](int x, int e) { return 32 * x + 8 * (e >> 2) + 4 * half + (e & 3); };
  auto qcol = [&](int y) { return 32 * y + (lane & 31); };
  float mn = 0.f, mx = 0.f;
  if (a.normalization == CAB_NORM_MINMAX) {
    mn = a.mm[bh * 2 + 0];
    mx = a.mm[bh * 2 + 1];
  }
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float v = 0.f;
        if (row0 + qrow(x, e) < a.M && col0 + qcol(y) < a.M) {
#pragma clang fp contract(off)
          v = acc[x][y][e] * a.alpha;  // rounded as in STATS (no fused multiply-add)
          if (a.normalization == CAB_NORM_MINMAX) v = normalize_minmax(v, mn, mx);
        }
        acc[x][y][e] = v;
      }
  if (a.rspart) {
    // Row sums over the quadrant's 64 columns (one AT column block).
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float sum = acc[x][0][e] + acc[x][1][e];
#pragma unroll
        for (int off = 1; off < 32; off <<= 1) sum += shfl_xor_f32(sum, off);
        if ((lane & 31) == 0)
          a.rspart[(static_cast<size_t>(bh) * a.nta + col0 / AT) * a.Mp + row0 + qrow(x, e)] = sum;
      }
  }
  // Each normalised 64 x 64 quadrant goes through LDS in turn, so that every
  // plane is written as whole 16-byte row chunks: X rows from the
  // quadrant's rows, XT rows from its columns (zero outside M: the planes
  // are Mp x Mp).
  __shared__ float stile[AT][AT + 1];
  const size_t pbase = static_cast<size_t>(bh) * a.Mp * a.Mp;
  for (int qd = 0; qd < 4; ++qd) {
    if (qd > 0) __syncthreads();  // the previous quadrant's reads are done
    if (w == qd) {
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
          for (int e = 0; e < 16; ++e) stile[qrow(x, e)][qcol(y)] = acc[x][y][e];
    }
    __syncthreads();
    const int64_t ti0 = ti * AW + AT * (qd >> 1), tj0 = tj * AW + AT * (qd & 1);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int cid = threadIdx.x + 256 * q;  // 64 rows x 8 chunks of 8 values
      const int r = cid >> 3, c8 = (cid & 7) * 8;
      const size_t xo = pbase + static_cast<size_t>(ti0 + r) * a.Mp + tj0 + c8;
      const size_t to = pbase + static_cast<size_t>(tj0 + r) * a.Mp + ti0 + c8;
      u32x4 h4, l4, th4, tl4;
      if (a.fused) {
        // XT row tj0 + r, column ti0 + c: delta - lambda Ahat[ti0 + c][tj0 + r]
        // (the delta only inside M; the planes are zero beyond it).
        const int64_t jrow = tj0 + r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x0 = stile[r][c8 + 2 * e], x1 = stile[r][c8 + 2 * e + 1];
          const int64_t k0 = ti0 + c8 + 2 * e;
          const float d0 = (k0 == jrow && k0 < a.M) ? 1.f : 0.f;
          const float d1 = (k0 + 1 == jrow && k0 + 1 < a.M) ? 1.f : 0.f;
          const float y0 = d0 - a.lambda * stile[c8 + 2 * e][r];
          const float y1 = d1 - a.lambda * stile[c8 + 2 * e + 1][r];
          h4[e] = static_cast<uint32_t>(f32_to_f16(x0)) | (static_cast<uint32_t>(f32_to_f16(x1)) << 16);
          th4[e] = static_cast<uint32_t>(f32_to_f16(y0)) | (static_cast<uint32_t>(f32_to_f16(y1)) << 16);
        }
        *reinterpret_cast<u32x4*>(a.xhi + xo) = h4;
        *reinterpret_cast<u32x4*>(a.xthi + to) = th4;
        continue;
      }
      if (a.f16_planes) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x0 = stile[r][c8 + 2 * e], x1 = stile[r][c8 + 2 * e + 1];
          const float y0 = stile[c8 + 2 * e][r], y1 = stile[c8 + 2 * e + 1][r];
          const uint16_t hx0 = f32_to_f16(x0), hx1 = f32_to_f16(x1);
          h4[e] = static_cast<uint32_t>(hx0) | (static_cast<uint32_t>(hx1) << 16);
          l4[e] = static_cast<uint32_t>(f32_to_f16(x0 - f16_to_f32(hx0))) |
                  (static_cast<uint32_t>(f32_to_f16(x1 - f16_to_f32(hx1))) << 16);
          th4[e] = static_cast<uint32_t>(f32_to_f16(y0)) | (static_cast<uint32_t>(f32_to_f16(y1)) << 16);
        }
        *reinterpret_cast<u32x4*>(a.xhi + xo) = h4;
        *reinterpret_cast<u32x4*>(a.xlo + xo) = l4;
        *reinterpret_cast<u32x4*>(a.xthi + to) = th4;
        continue;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = stile[r][c8 + 2 * e], x1 = stile[r][c8 + 2 * e + 1];    // X row ti0 + r
        const float y0 = stile[c8 + 2 * e][r], y1 = stile[c8 + 2 * e + 1][r];    // XT row tj0 + r
        const uint16_t hx0 = f32_to_bf16(x0), hx1 = f32_to_bf16(x1);
        const uint16_t hy0 = f32_to_bf16(y0), hy1 = f32_to_bf16(y1);
        h4[e] = static_cast<uint32_t>(hx0) | (static_cast<uint32_t>(hx1) << 16);
        l4[e] = static_cast<uint32_t>(f32_to_bf16(x0 - bf16_to_f32(hx0))) |
                (static_cast<uint32_t>(f32_to_bf16(x1 - bf16_to_f32(hx1))) << 16);
        th4[e] = static_cast<uint32_t>(hy0) | (static_cast<uint32_t>(hy1) << 16);
        tl4[e] = static_cast<uint32_t>(f32_to_bf16(y0 - bf16_to_f32(hy0))) |
                 (static_cast<uint32_t>(f32_to_bf16(y1 - bf16_to_f32(hy1))) << 16);
      }
      *reinterpret_cast<u32x4*>(a.xhi + xo) = h4;
      *reinterpret_cast<u32x4*>(a.xlo + xo) = l4;
      *reinterpret_cast<u32x4*>(a.xthi + to) = th4;
      *reinterpret_cast<u32x4*>(a.xtlo + to) = tl4;
    }
    if (a.affinity) {
      // fp32 diagnostic, rows of the quadrant inside M (coalesced along j)
      for (int e = threadIdx.x; e < AT * AT; e += 256) {
        const int r = e >> 6, c = e & 63;
        const int64_t i = ti0 + r, jj = tj0 + c;
        if (i < a.M && jj < a.M) a.affinity[(static_cast<size_t>(bh) * a.M + i) * a.M + jj] = stile[r][c];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// aff_strip_kernel: the STATS and EMIT passes for 16-bit inputs with D <= 128.
// A workgroup walks a strip of up to `strip` consecutive 128 x 128 tiles of A
// along j, all in one 128-row band i0 of one (b, h):
//  - the band's Qc panel (128 rows x 256 bytes; 16-byte chunk c of row R at
//    chunk position c ^ (R % 16), so that the 16 rows one operand read
//    touches fall into 16 distinct bank groups; rows at or past M and dims at
//    or past D read as zero) is staged into LDS once, and each compute wave
//    then keeps its MFMA operands of it in registers for the whole strip;
//  - the Kc panel of every tile is staged in turn, double-buffered (the Qc
//    panel's space is the second buffer once its operands are in registers),
//    so that the next tile's panel is in flight while a tile is computed;
//  - eight compute waves split a tile into blocks of 64 rows j x 32 columns
//    i (EMIT) or 32 x 64 (STATS) and compute C = Kc Qc^T (C[j][i] =
//    A[i][j] / alpha) with 32x32x16 MFMAs; lane l then holds column
//    i = l % 32 of each of its two 32 x 32 tiles and rows
//    j = 8 (e / 4) + 4 (l / 32) + e % 4 of element e: runs of four
//    consecutive j of one row i of A.
// STATS (8 waves, two workgroups per CU): min / max of A over i, j < M per
// strip.
// EMIT (8 compute + 4 store waves, one workgroup per CU): the compute waves
// normalise a tile into two LDS tiles, X [128 i][128 j] (8-byte writes of the
// runs, chunk c of row il at chunk position c ^ (il % 16)) and XT
// [128 j][128 i] (2-byte writes: a wave's 32 lanes of one row j are
// consecutive i); the store waves copy both to the planes as whole 16-byte row
// pieces while the compute waves go on with the next tile. Loads and stores
// are thus issued by different waves: vmcnt counts both, so a wave that
// stored would wait for its stores whenever it waits for a panel.
// Row-sum partials (augmented formula) per 64 columns j.
// Work per tile: 2 128^2 D flops; EMIT writes 32 KB per plane and tile.
// ---------------------------------------------------------------------------
constexpr int AGT = 128;                 // tile edge and panel rows
constexpr int AG_PANEL = AGT * 256;      // bytes of one staged panel
constexpr int AG_DMAX = 128;             // largest D a panel holds
constexpr int AG_CW = 8;                 // compute waves
constexpr int AG_SW = 4;                 // store waves (EMIT)

// Stages rows [0, 128) of a row-major [rows][D] 16-bit panel at `base` (the
// first `rows` of them exist) into LDS `dst` in the swizzled layout; issued
// by the eight compute waves, four 1 KB buffer loads each.
__device__ __forceinline__ void ag_stage(const char* base, int64_t rows, uint32_t rowb, int kch,
                                         int w, int lane, char* dst) {
  const brsrc_t rs = make_rsrc(base, static_cast<uint32_t>((rows < AGT ? rows : AGT) * rowb));
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int blk = 4 * w + n;
    const int R = 4 * blk + (lane >> 4);
    const int c = (lane & 15) ^ (R & 15);
    const uint32_t voff = c < kch ? static_cast<uint32_t>(R) * rowb + 16u * c : 0x80000000u;
    bdma16(rs, voff, 0, dst + blk * 1024);
  }
}

template <typename T, bool EMIT, int KS>
__global__ __launch_bounds__(EMIT ? 64 * (AG_CW + AG_SW) : 64 * AG_CW, EMIT ? 3 : 4) void aff_strip_kernel(
    AffArgs a) {
  constexpr bool BF = std::is_same<T, bf16_t>::value;
  // [panel buffer 0 (Qc, then Kc)][panel buffer 1]; EMIT: [X tile][XT tile]
  __shared__ __attribute__((aligned(16))) char lds[(EMIT ? 4 : 2) * AG_PANEL];
  __shared__ float red[EMIT ? 2 * AGT : 2 * AG_CW];  // EMIT: row-sum partials; STATS: min / max
  const int64_t ns = a.Mp / AGT;  // Mp is a multiple of 128
  const int64_t strip = a.strip;
  const int64_t nstrip = (ns + strip - 1) / strip;
  const int64_t logical = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x));
  const int64_t bh = logical / (ns * nstrip);
  const int64_t part = logical - bh * ns * nstrip;  // strip index within (b, h)
  const int64_t ti = part / nstrip;
  const int64_t tj0 = (part - ti * nstrip) * strip;
  const int cnt = static_cast<int>(ns - tj0 < strip ? ns - tj0 : strip);
  const int64_t i0 = ti * AGT;
  // The wave index is uniform within a wave: the role branches below are scalar.
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = lane_id(), tid = threadIdx.x;
  const bool compute = w < AG_CW;
  const int kch = a.D / 8;
  const uint32_t rowb = static_cast<uint32_t>(a.D) * 2;
  const char* const kbase = static_cast<const char*>(a.kc) + bh * a.M * rowb;
  // The Kc panel of tile t sits in buffer (t + 1) % 2.
  auto kbuf = [&](int t) { return lds + ((t + 1) & 1) * AG_PANEL; };
  auto stage_k = [&](int t) {
    const int64_t j0 = (tj0 + t) * AGT;
    ag_stage(kbase + j0 * rowb, a.M - j0, rowb, kch, w, lane, kbuf(t));
  };
  if (compute) {
    ag_stage(static_cast<const char*>(a.qc) + (bh * a.M + i0) * rowb, a.M - i0, rowb, kch, w, lane, lds);
    stage_k(0);
  }

  const int h = lane >> 5;
  // A wave's block is XW 32-row tiles (j) by YW 32-column tiles (i):
  // 64 x 32 for EMIT, whose staging code needs the registers, and 32 x 64
  // for STATS, which reads each Kc operand once for two MFMAs (half the LDS
  // reads of 64 x 32).
  constexpr int XW = EMIT ? 2 : 1, YW = EMIT ? 1 : 2, NI = 4 / YW;
  const int jr0 = 32 * XW * ((w / NI) & (4 / XW - 1)), ic0 = 32 * YW * (w % NI);
  // Tile-local coordinates: column i = li0 + 32 y of tile (x, y), rows
  // j = lj0 + 32 x + 8 g + r of run g (elements 4 g + r).
  const int li0 = ic0 + (lane & 31), lj0 = jr0 + 4 * h;
  auto extent = [](int64_t n) { return static_cast<int>(n < 0 ? 0 : (n < AGT ? n : AGT)); };
  const int mi = extent(a.M - i0);
  u32x4 qf[YW][KS];  // the wave's Qc operands: rows i of its column tiles
  auto load_q = [&]() {
#pragma unroll
    for (int y = 0; y < YW; ++y)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int R = li0 + 32 * y, c = 2 * ks + h;
        qf[y][ks] = *reinterpret_cast<const u32x4*>(lds + R * 256 + ((c ^ (R & 15)) << 4));
      }
  };
  f32x16 acc[XW * YW];  // tile (x, y) at x * YW + y
  auto product = [&](int t) {
    const char* kb = kbuf(t);
#pragma unroll
    for (int q = 0; q < XW * YW; ++q) acc[q] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c = 2 * ks + h;
#pragma unroll
      for (int x = 0; x < XW; ++x) {
        const int R = jr0 + 32 * x + (lane & 31);
        const u32x4 av = *reinterpret_cast<const u32x4*>(kb + R * 256 + ((c ^ (R & 15)) << 4));
#pragma unroll
        for (int y = 0; y < YW; ++y) {
          f32x16& d = acc[x * YW + y];
          if constexpr (BF)
            d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av),
                                                        __builtin_bit_cast(bf16x8, qf[y][ks]), d, 0, 0, 0);
          else
            d = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, av),
                                                       __builtin_bit_cast(f16x8, qf[y][ks]), d, 0, 0, 0);
        }
      }
    }
  };

  if constexpr (!EMIT) {
    // Extremes of the raw products: rounding alpha x is monotonic in x, so
    // the extremes of alpha A are alpha times these (swapped for alpha < 0),
    // rounded once, as the EMIT pass rounds every entry.
    float lo = INFINITY, hi = -INFINITY;
    for (int t = 0; t < cnt; ++t) {
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's panel loads have landed
      lds_barrier();                       // ... and every wave's; tile t - 1 is done
      if (t == 0) {
        load_q();
        lds_barrier();  // every wave holds its Qc operands: buffer 0 is free
      }
      if (t + 1 < cnt) stage_k(t + 1);  // into the buffer tile t - 1 used
      product(t);
      const int mj = extent(a.M - (tj0 + t) * AGT);
      if (mi == AGT && mj == AGT) {
#pragma unroll
        for (int q = 0; q < XW * YW; ++q)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            lo = fminf(lo, acc[q][e]);
            hi = fmaxf(hi, acc[q][e]);
          }
      } else {
        // Entries outside M enter as the identities: selects, not branches.
#pragma unroll
        for (int y = 0; y < YW; ++y) {
          // rows lj0 + o of column li0 + 32 y inside M: o < jlim
          const int jlim = li0 + 32 * y < mi ? mj - lj0 : 0;
#pragma unroll
          for (int x = 0; x < XW; ++x)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const bool in = 32 * x + 8 * (e >> 2) + (e & 3) < jlim;
              lo = fminf(lo, in ? acc[x * YW + y][e] : INFINITY);
              hi = fmaxf(hi, in ? acc[x * YW + y][e] : -INFINITY);
            }
        }
      }
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      lo = fminf(lo, shfl_xor_f32(lo, off));
      hi = fmaxf(hi, shfl_xor_f32(hi, off));
    }
    if (lane == 0) {
      red[2 * w] = lo;
      red[2 * w + 1] = hi;
    }
    lds_barrier();
    if (tid == 0) {
      float m0 = red[0], m1 = red[1];
#pragma unroll
      for (int q = 1; q < AG_CW; ++q) {
        m0 = fminf(m0, red[2 * q]);
        m1 = fmaxf(m1, red[2 * q + 1]);
      }
      const float e0 = m0 * a.alpha, e1 = m1 * a.alpha;
      float* p = a.mmpart + (bh * ns * nstrip + part) * 2;
      p[0] = a.alpha < 0.f ? e1 : e0;
      p[1] = a.alpha < 0.f ? e0 : e1;
    }
  } else {
    // min / max of alpha A over (b, h) from the STATS partials, reduced by
    // the store waves while the first panels load; the first strip of each
    // (b, h) also stores them for the triangle pass.
    __shared__ float mmred[AG_SW][2];
    const bool minmax = a.normalization == CAB_NORM_MINMAX;
    if (minmax && !compute) {
      float lo = INFINITY, hi = -INFINITY;
      for (int64_t q = tid - 64 * AG_CW; q < a.nparts; q += 64 * AG_SW) {
        lo = fminf(lo, a.mmpart[(bh * a.nparts + q) * 2 + 0]);
        hi = fmaxf(hi, a.mmpart[(bh * a.nparts + q) * 2 + 1]);
      }
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        lo = fminf(lo, shfl_xor_f32(lo, off));
        hi = fmaxf(hi, shfl_xor_f32(hi, off));
      }
      if (lane == 0) {
        mmred[w - AG_CW][0] = lo;
        mmred[w - AG_CW][1] = hi;
      }
    }
    float mn = 0.f, scale = 1.f;  // Ahat = (alpha A - mn) * scale
    auto take_minmax = [&]() {
      float m0 = mmred[0][0], m1 = mmred[0][1];
#pragma unroll
      for (int q = 1; q < AG_SW; ++q) {
        m0 = fminf(m0, mmred[q][0]);
        m1 = fmaxf(m1, mmred[q][1]);
      }
      if (part == 0 && tid == 64 * AG_CW) {
        a.mm[bh * 2 + 0] = m0;
        a.mm[bh * 2 + 1] = m1;
      }
      if (m1 > m0) {
        mn = m0;
        scale = 1.0f / (m1 - m0 + 1e-8f);
      }  // else constant A: left as is
    };
    const size_t pbase = static_cast<size_t>(bh) * a.Mp * a.Mp;
    const uint32_t Mp2 = static_cast<uint32_t>(a.Mp) * 2;  // bytes per plane row
    uint16_t* const sx = reinterpret_cast<uint16_t*>(lds + 2 * AG_PANEL);
    uint16_t* const st = reinterpret_cast<uint16_t*>(lds + 3 * AG_PANEL);
    // Pass 0 fills X = xhi and XT = xthi; the unfused forms add pass 1:
    // xlo (fp16) or xlo and xtlo (bf16).
    const int npass = a.fused ? 1 : 2;
    auto xplane = [&](int p) { return p == 0 ? a.xhi : a.xlo; };
    auto tplane = [&](int p) { return p == 0 ? a.xthi : (a.f16_planes ? nullptr : a.xtlo); };

    // Store waves: copy the staged tiles of pass p of tile t to the planes.
    auto flush = [&](int t, int p) {
      const int ts = tid - 64 * AG_CW;  // 0 .. 255
      const int rl0 = ts >> 4, c = ts & 15;
      const int64_t j0 = (tj0 + t) * AGT;
      const uint32_t voff = static_cast<uint32_t>(rl0) * Mp2 + 16u * c;
      const brsrc_t xr = make_rsrc(xplane(p) + pbase + i0 * a.Mp + j0, AGT * Mp2);
#pragma unroll
      for (int n = 0; n < AGT / 16; ++n) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(sx + (rl0 + 16 * n) * AGT + ((c ^ (rl0 & 15)) << 3));
        __builtin_amdgcn_raw_buffer_store_b128(v, xr, voff, static_cast<uint32_t>(16 * n) * Mp2, 0);
      }
      uint16_t* const tp = tplane(p);
      if (tp) {
        const brsrc_t tr = make_rsrc(tp + pbase + j0 * a.Mp + i0, AGT * Mp2);
#pragma unroll
        for (int n = 0; n < AGT / 16; ++n) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(st + (rl0 + 16 * n) * AGT + 8 * c);
          __builtin_amdgcn_raw_buffer_store_b128(v, tr, voff, static_cast<uint32_t>(16 * n) * Mp2, 0);
        }
      }
      if (a.rspart && p == npass - 1) {
        // Row sums over the 64 columns j of each half of the tile.
        const int q = ts >> 7, il = ts & 127;
        a.rspart[(static_cast<size_t>(bh) * a.nta + j0 / AT + q) * a.Mp + i0 + il] = red[q * AGT + il];
      }
    };

    // Compute waves: write pass p of the normalised tile t into the LDS tiles.
    auto f16v = [](float v) { return f32_to_f16(v); };
    auto f16lo = [](float v) { return f32_to_f16(v - f16_to_f32(f32_to_f16(v))); };
    auto bf16v = [](float v) { return f32_to_bf16(v); };
    auto bf16lo = [](float v) { return f32_to_bf16(v - bf16_to_f32(f32_to_bf16(v))); };
    // tval(v, k) gives the XT entry of element k = 16 x + e of the lane.
    auto stage_pass = [&](auto xval, bool with_t, auto tval) {
      const int il = li0;
#pragma unroll
      for (int x = 0; x < 2; ++x) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int jl = lj0 + 32 * x + 8 * g;  // a multiple of 4
          const uint32_t w0 = static_cast<uint32_t>(xval(acc[x][4 * g])) |
                              (static_cast<uint32_t>(xval(acc[x][4 * g + 1])) << 16);
          const uint32_t w1 = static_cast<uint32_t>(xval(acc[x][4 * g + 2])) |
                              (static_cast<uint32_t>(xval(acc[x][4 * g + 3])) << 16);
          *reinterpret_cast<u32x2*>(sx + il * AGT + ((((jl >> 3) ^ (il & 15)) << 3) | (jl & 4))) =
              u32x2{w0, w1};
          if (with_t) {
#pragma unroll
            for (int r = 0; r < 4; ++r) st[(jl + r) * AGT + il] = tval(acc[x][4 * g + r], 16 * x + 4 * g + r);
          }
        }
      }
    };
    // Element of the lane on the diagonal of a diagonal tile (j = i < M), or
    // -1: il - lj0 = 32 x + 8 g + r with r < 4.
    const int dd = li0 - lj0;
    const int ediag = li0 < mi && dd >= 0 && dd < 64 && (dd & 4) == 0
                          ? 16 * (dd >> 5) + 4 * ((dd >> 3) & 3) + (dd & 3)
                          : -1;
    auto stage = [&](int t, int p) {
      const int64_t j0 = (tj0 + t) * AGT;
      if (a.fused) {
        // X = f16(Ahat); XT[j][i] = delta_ij - lambda Ahat[i][j] (delta only inside M)
        const float lam = a.lambda;
        if (i0 == j0) {
          int ed = ediag;
          asm volatile("" : "+v"(ed));  // compared per tile, not held as 32 masks
          stage_pass(f16v, true, [&](float v, int k) {
            return f32_to_f16((k == ed ? 1.f : 0.f) - lam * v);
          });
        } else {
          stage_pass(f16v, true, [&](float v, int) { return f32_to_f16(-lam * v); });
        }
      } else if (a.f16_planes) {
        if (p == 0) stage_pass(f16v, true, [&](float v, int) { return f32_to_f16(v); });
        else stage_pass(f16lo, false, [&](float, int) { return uint16_t(0); });
      } else {
        if (p == 0) stage_pass(bf16v, true, [&](float v, int) { return f32_to_bf16(v); });
        else stage_pass(bf16lo, true, [&](float v, int) { return bf16lo(v); });
      }
    };

    if (minmax) {
      lds_barrier();  // the store waves' partial extremes are in (the panels still load)
      take_minmax();
    }
    for (int t = 0; t < cnt; ++t) {
      if (compute) __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's panel loads
      lds_barrier();  // tile t's panel is in; the tiles of t - 1 are staged
      if (compute) {
        if (t == 0) load_q();
        else if (t + 1 < cnt) stage_k(t + 1);  // into the buffer tile t - 1 used
        product(t);
      } else if (t > 0) {
        flush(t - 1, npass - 1);
      }
      lds_barrier();  // the panel buffer and the LDS tiles are free
      if (compute) {
        if (t == 0 && cnt > 1) stage_k(1);  // buffer 0: the Qc operands are in registers
        const int64_t j0 = (tj0 + t) * AGT;
        const int mj = extent(a.M - j0);
        // rows lj0 + o of the lane inside M: o < jlim (all of them inside the interior)
        const int jlim = li0 < mi ? mj - lj0 : 0;
        {
          // alpha A rounded on its own, as in the STATS pass (no fused
          // multiply-add with the subtraction): the minimum maps to exactly 0.
#pragma clang fp contract(off)
#pragma unroll
          for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const float v = (acc[x][e] * a.alpha - mn) * scale;
              acc[x][e] = 32 * x + 8 * (e >> 2) + (e & 3) < jlim ? v : 0.f;
            }
        }
        if (a.affinity && li0 < mi) {
          // fp32 diagnostic [M][M] (runs of four j of one row i)
          float* ar = a.affinity + (static_cast<size_t>(bh) * a.M + i0 + li0) * a.M + j0;
#pragma unroll
          for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int jl = lj0 + 32 * x + 8 * (e >> 2) + (e & 3);
              if (jl < mj) ar[jl] = acc[x][e];
            }
        }
        if (a.rspart) {
          // Row sums over the wave's 64 rows j (one AT column block), per column i.
          float sum = 0.f;
#pragma unroll
          for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int e = 0; e < 16; ++e) sum += acc[x][e];
          sum += shfl_xor_f32(sum, 32);
          if (h == 0) red[(jr0 / 64) * AGT + li0] = sum;
        }
        stage(t, 0);
      }
      for (int p = 1; p < npass; ++p) {
        lds_barrier();  // pass p - 1 is staged
        if (!compute) flush(t, p - 1);
        lds_barrier();  // ... and copied out
        if (compute) stage(t, p);
      }
    }
    lds_barrier();
    if (!compute) flush(cnt - 1, npass - 1);
  }
}

__global__ __launch_bounds__(256) void minmax_finalize_kernel(const float* part, int64_t nparts,
                                                              float* mm) {
  const int64_t bh = blockIdx.x;
  float mn = INFINITY, mx = -INFINITY;
  for (int64_t p = threadIdx.x; p < nparts; p += 256) {
    mn = fminf(mn, part[(bh * nparts + p) * 2 + 0]);
    mx = fmaxf(mx, part[(bh * nparts + p) * 2 + 1]);
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    mn = fminf(mn, shfl_xor_f32(mn, off));
    mx = fmaxf(mx, shfl_xor_f32(mx, off));
  }
  __shared__ float red[4][2];
  const int w = threadIdx.x >> 6;
  if (lane_id() == 0) {
    red[w][0] = mn;
    red[w][1] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    mm[bh * 2 + 0] = fminf(fminf(red[0][0], red[1][0]), fminf(red[2][0], red[3][0]));
    mm[bh * 2 + 1] = fmaxf(fmaxf(red[0][1], red[1][1]), fmaxf(red[2][1], red[3][1]));
  }
}

__global__ __launch_bounds__(256) void rowsum_finalize_kernel(const float* part, int64_t nta,
                                                              int64_t Mp, float* rs) {
  const int64_t bh = blockIdx.y;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= Mp) return;
  float s = 0.f;
  for (int64_t t = 0; t < nta; ++t) s += part[(bh * nta + t) * Mp + i];
  rs[bh * Mp + i] = s;
}

struct TriArgs {
  const uint16_t* xhi;
  const uint16_t* xlo;
  const uint16_t* xthi;
  const uint16_t* xtlo;
  const float* rowsum;  // [BH][Mp] (augmented only)
  const float* mm;      // [BH][2] minmax of A (fp16 planes only)
  float* frc;           // [BH][M][M]
  float* tri;           // [BH][M][M] or null
  int64_t M, Mp, nti, ntj, BH;  // nti x ntj tiles per (b, h)
  float lambda;
  int formula;
  int fused;            // fp16 planes with XT = I - lambda Ahat^T: the accumulator is F
};

// LDS operand tile in MFMA order: slot (kk, sub, lane) of 16 bytes holds the
// 8 consecutive k values lane needs for a 32x32x16 MFMA, so every operand
// read is one 1 KB wave access. Inside each 64-slot group the slot of lane L
// is stored at position L ^ swz(kk, L / 32), swz(kk, h) = 2 (2 kk + h): the
// eight chunks of one row (kc = 2 kk + h) then land in eight different
// 16-byte bank groups, and the two rows sixteen threads store fill all
// sixteen (bit 0 of the position is the row's); a wave's reads stay a
// permutation inside each 16-slot bank cycle.
template <int TILE, int KD>
constexpr int tri_slots() { return (KD / 16) * (TILE / 32) * 64; }

// A plane's TILE x KD slice is TILE rows of KD / 8 chunks of 16 bytes; KD / 8
// consecutive threads read one row (KD = 64: a whole 128-byte cache line).
// Thread t moves chunks t, t + THREADS, ...
template <int TILE, int THREADS, int KD>
constexpr int tri_chunks() { return TILE * (KD / 8) / THREADS; }

template <int TILE, int THREADS, int KD>
__device__ __forceinline__ void tri_load(const uint16_t* plane, int64_t row0, int64_t k0, int64_t Mp,
                                         u32x4 (&reg)[tri_chunks<TILE, THREADS, KD>()]) {
  constexpr int CPR = KD / 8;  // chunks per row
#pragma unroll
  for (int q = 0; q < tri_chunks<TILE, THREADS, KD>(); ++q) {
    const int cid = threadIdx.x + THREADS * q;
    const int row = cid / CPR, kc = cid % CPR;
    reg[q] = *reinterpret_cast<const u32x4*>(plane + (row0 + row) * Mp + k0 + 8 * kc);
  }
}

template <int TILE, int THREADS, int KD>
__device__ __forceinline__ void tri_store(u32x4* lds, const u32x4 (&reg)[tri_chunks<TILE, THREADS, KD>()]) {
  constexpr int CPR = KD / 8;
#pragma unroll
  for (int q = 0; q < tri_chunks<TILE, THREADS, KD>(); ++q) {
    const int cid = threadIdx.x + THREADS * q;
    const int row = cid / CPR, kc = cid % CPR;
    const int kk = kc >> 1, hf = kc & 1, sub = row >> 5;
    lds[(kk * (TILE / 32) + sub) * 64 + (((row & 31) + 32 * hf) ^ (2 * (2 * kk + hf)))] = reg[q];
  }
}

__device__ __forceinline__ float frc_combine(int formula, float ahat, float t, float lambda, float si,
                                             float sj) {
  float f;
  if (formula == CAB_FRC_ADDITIVE) {
    f = ahat - lambda * t;
    if (!isfinite(f)) f = 0.f;
  } else if (formula == CAB_FRC_MULTIPLICATIVE) {
    f = ahat * (1.0f / (1.0f + lambda * (t / (ahat + 1e-8f))));
    if (!isfinite(f)) f = 0.f;
  } else {
    f = ahat > 0.f ? 4.0f * ahat - si - sj + 3.0f * t : 1000.0f;
  }
  return f;
}

// T tile of TI x TJ per workgroup of WI x WJ waves; wave (wi, wj) owns rows
// wi TI / WI .. and columns wj TJ / WJ .. as XS x YS MFMA tiles. NBUF
// register buffers carry operand slices global -> registers -> LDS (two LDS
// stages): with NBUF = 2 a slice's loads have two slices of MFMA work to
// land, with NBUF = 1 one slice (for the wide bf16 tile, whose accumulators
// leave room for one buffer of four planes only); NBUF = 0 is the ping-pong
// schedule of two wave groups (fp16 256 x 256 tile). F16 selects the fp16 planes
// (A = X, B = XT, one product per site); otherwise the bf16 hi / lo planes of
// both operands (three products).
template <int TI, int TJ, int WI, int WJ, int NBUF, bool F16, int KD>
__global__ __launch_bounds__(WI * WJ * 64, 1) void triangle_kernel(TriArgs a) {
  constexpr int THREADS = WI * WJ * 64;
  constexpr int XS = TI / WI / 32, YS = TJ / WJ / 32;
  constexpr int SA = tri_slots<TI, KD>(), SB = tri_slots<TJ, KD>();
  constexpr int CA = tri_chunks<TI, THREADS, KD>(), CB = tri_chunks<TJ, THREADS, KD>();
  static_assert(CA * THREADS == TI * (KD / 8) && CB * THREADS == TJ * (KD / 8),
                "whole chunks per thread");
  constexpr int NH = F16 ? 1 : 2;           // planes per operand: hi (and lo)
  constexpr int STAGE = NH * (SA + SB);     // slots per LDS stage: A planes, then B planes
  __shared__ u32x4 lds[2 * STAGE];
  const int64_t per = a.nti * a.ntj;
  const int64_t total = a.BH * per;
  const int64_t logical = xcd_remap(blockIdx.x, total);
  const int64_t bh = logical / per;
  const int64_t rem = logical - bh * per;
  const int64_t ti = rem / a.ntj, tj = rem - (rem / a.ntj) * a.ntj;
  const size_t pbase = static_cast<size_t>(bh) * a.Mp * a.Mp;
  const uint16_t* pa[NH];
  const uint16_t* pb[NH];
  pa[0] = a.xhi + pbase;
  pb[0] = a.xthi + pbase;
  if constexpr (!F16) {
    pa[NH - 1] = a.xlo + pbase;
    pb[NH - 1] = a.xtlo + pbase;
  }
  const int64_t ra = ti * TI, rb = tj * TJ;
  // fp16 planes: a constant A (min == max) is left unnormalised and may lie
  // outside fp16's range; its T = M c^2 is formed directly in the epilogue.
  bool constant = false;
  float cval = 0.f;
  if constexpr (F16) {
    cval = a.mm[bh * 2 + 0];
    constant = !(a.mm[bh * 2 + 1] > cval);
  }

  const int w = threadIdx.x >> 6, lane = lane_id();
  const int wi = w / WJ, wj = w - (w / WJ) * WJ;
  f32x16 acc[XS][YS];
#pragma unroll
  for (int x = 0; x < XS; ++x)
#pragma unroll
    for (int y = 0; y < YS; ++y) acc[x][y] = f32x16{};

  const int nk = static_cast<int>(a.Mp / KD);
  auto compute = [&](auto st_tag) {
    constexpr int st = decltype(st_tag)::value;
    const u32x4* la = lds + st * STAGE;
    const u32x4* lb = la + NH * SA;
#pragma unroll
    for (int kk = 0; kk < KD / 16; ++kk) {
      const int lsw = lane ^ (2 * (2 * kk + (lane >> 5)));
      if constexpr (F16) {
        f16x8 b8[YS];
#pragma unroll
        for (int y = 0; y < YS; ++y)
          b8[y] = __builtin_bit_cast(f16x8, lb[(kk * (TJ / 32) + YS * wj + y) * 64 + lsw]);
#pragma unroll
        for (int x = 0; x < XS; ++x) {
          const f16x8 a8 = __builtin_bit_cast(f16x8, la[(kk * (TI / 32) + XS * wi + x) * 64 + lsw]);
#pragma unroll
          for (int y = 0; y < YS; ++y)
            acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a8, b8[y], acc[x][y], 0, 0, 0);
        }
      } else {
        bf16x8 bh8[YS], bl[YS];
#pragma unroll
        for (int y = 0; y < YS; ++y) {
          const int sb = (kk * (TJ / 32) + YS * wj + y) * 64 + lsw;
          bh8[y] = __builtin_bit_cast(bf16x8, lb[sb]);
          bl[y] = __builtin_bit_cast(bf16x8, lb[SB + sb]);
        }
        // A operands one 32-row strip at a time (fewer live registers).
#pragma unroll
        for (int x = 0; x < XS; ++x) {
          const int sa = (kk * (TI / 32) + XS * wi + x) * 64 + lsw;
          const bf16x8 ah = __builtin_bit_cast(bf16x8, la[sa]);
          const bf16x8 al = __builtin_bit_cast(bf16x8, la[SA + sa]);
#pragma unroll
          for (int y = 0; y < YS; ++y) {
            acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh8[y], acc[x][y], 0, 0, 0);
            acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl[y], acc[x][y], 0, 0, 0);
            acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh8[y], acc[x][y], 0, 0, 0);
          }
        }
      }
    }
  };
  constexpr int NB = NBUF > 0 ? NBUF : 1;  // register buffers (ping-pong: its own, below)
  u32x4 rga[NB][NH][CA], rgb[NB][NH][CB];
  auto load = [&](int buf, int kt) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      tri_load<TI, THREADS, KD>(pa[h], ra, static_cast<int64_t>(kt) * KD, a.Mp, rga[buf][h]);
      tri_load<TJ, THREADS, KD>(pb[h], rb, static_cast<int64_t>(kt) * KD, a.Mp, rgb[buf][h]);
    }
  };
  auto store = [&](int buf, int st) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      tri_store<TI, THREADS, KD>(lds + st * STAGE + h * SA, rga[buf][h]);
      tri_store<TJ, THREADS, KD>(lds + st * STAGE + NH * SA + h * SB, rgb[buf][h]);
    }
  };

  // The loop's barriers are uniform: `constant` depends on bh alone.
  if (!constant) {
    if constexpr (NBUF == 0) {
      // Ping-pong: wave group gp = wi (waves 4 gp .. 4 gp + 3, one per SIMD)
      // stages its own 128 A rows and half of the B rows of each slice. In
      // each slice, group 0 multiplies while group 1 stores slice kt + 1 and
      // loads slice kt + 2, then the roles swap, so every SIMD has one wave on
      // the MFMAs and one on memory. Slice kt + 1 is complete in LDS after
      // the slice's second barrier, and its stage was last read (slice kt - 1)
      // before the first.
      static_assert(WI == 2 && THREADS == 512 && F16, "ping-pong: two groups of four waves");
      constexpr int CPR = KD / 8;                        // 16-byte chunks per row
      constexpr int HA = TI / 2, HB = TJ / 2;            // rows per group and operand
      constexpr int CAH = HA * CPR / 256, CBH = HB * CPR / 256;
      static_assert(CAH * 256 == HA * CPR && CBH * 256 == HB * CPR, "whole chunks per thread");
      const int gp = wi, tg = threadIdx.x & 255;
      u32x4 pra[CAH], prb[CBH];
      // Loads through buffer descriptors over the tile's rows (Mp is a
      // multiple of the tile edge, so every row exists; TI Mp 2 bytes fit 32
      // bits): a lane's offsets are the same for every slice and the slice's
      // k offset is the scalar offset, so the loads cost no vector address
      // arithmetic.
      // (The bases go through readfirstlane: they are uniform, which the
      // compiler does not see, and a descriptor it takes for divergent is
      // wrapped in a loop over the lanes' values.)
      const uint32_t rowb = static_cast<uint32_t>(a.Mp) * 2u;
      auto uniform = [](const uint16_t* p) {
        const uint64_t u = reinterpret_cast<uint64_t>(p);
        const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u)));
        const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u >> 32)));
        return reinterpret_cast<const uint16_t*>((static_cast<uint64_t>(hi) << 32) | lo);
      };
      const brsrc_t ars = make_rsrc(uniform(pa[0] + ra * a.Mp), static_cast<uint32_t>(TI) * rowb);
      const brsrc_t brs = make_rsrc(uniform(pb[0] + rb * a.Mp), static_cast<uint32_t>(TJ) * rowb);
      uint32_t aoff[CAH], boff[CBH];
#pragma unroll
      for (int q = 0; q < CAH; ++q) {
        const int cid = tg + 256 * q, row = gp * HA + cid / CPR, kc = cid % CPR;
        aoff[q] = static_cast<uint32_t>(row) * rowb + 16u * kc;
      }
#pragma unroll
      for (int q = 0; q < CBH; ++q) {
        const int cid = tg + 256 * q, row = gp * HB + cid / CPR, kc = cid % CPR;
        boff[q] = static_cast<uint32_t>(row) * rowb + 16u * kc;
      }
      auto pload = [&](int kt) {
        const uint32_t k0b = static_cast<uint32_t>(kt) * (2u * KD);
#pragma unroll
        for (int q = 0; q < CAH; ++q) pra[q] = __builtin_amdgcn_raw_buffer_load_b128(ars, aoff[q], k0b, 0);
#pragma unroll
        for (int q = 0; q < CBH; ++q) prb[q] = __builtin_amdgcn_raw_buffer_load_b128(brs, boff[q], k0b, 0);
      };
      auto pstore = [&](int st) {
        u32x4* la = lds + st * STAGE;
        u32x4* lb = la + SA;
#pragma unroll
        for (int q = 0; q < CAH; ++q) {
          const int cid = tg + 256 * q, row = gp * HA + cid / CPR, kc = cid % CPR;
          const int kk = kc >> 1, hf = kc & 1, sub = row >> 5;
          la[(kk * (TI / 32) + sub) * 64 + (((row & 31) + 32 * hf) ^ (2 * (2 * kk + hf)))] = pra[q];
        }
#pragma unroll
        for (int q = 0; q < CBH; ++q) {
          const int cid = tg + 256 * q, row = gp * HB + cid / CPR, kc = cid % CPR;
          const int kk = kc >> 1, hf = kc & 1, sub = row >> 5;
          lb[(kk * (TJ / 32) + sub) * 64 + (((row & 31) + 32 * hf) ^ (2 * (2 * kk + hf)))] = prb[q];
        }
      };
      pload(0);
      pstore(0);
      if (nk > 1) pload(1);
      lds_barrier();
      auto slice = [&](int kt, auto st_tag) {
        constexpr int st = decltype(st_tag)::value;  // LDS stage of slice kt
        auto mem = [&]() {
          if (kt + 1 < nk) pstore(st ^ 1);
          if (kt + 2 < nk) pload(kt + 2);
        };
        // The multiplying group runs at raised wave priority.
        if (gp == 0) {
          __builtin_amdgcn_s_setprio(1);
          compute(st_tag);
          __builtin_amdgcn_s_setprio(0);
        } else {
          mem();
        }
        lds_barrier();
        if (gp == 0) {
          mem();
        } else {
          __builtin_amdgcn_s_setprio(1);
          compute(st_tag);
          __builtin_amdgcn_s_setprio(0);
        }
        lds_barrier();
      };
      for (int kt = 0; kt < nk; kt += 2) {
        slice(kt, std::integral_constant<int, 0>{});
        if (kt + 1 < nk) slice(kt + 1, std::integral_constant<int, 1>{});
      }
    } else if constexpr (NBUF == 2) {
      // The registers of slice kt + 2 are loaded while slice kt is multiplied.
      load(0, 0);
      if (nk > 1) load(1, 1);
      auto slice = [&](int kt, auto buf_tag) {
        constexpr int st = decltype(buf_tag)::value;  // register buffer and LDS stage kt % 2
        store(st, st);
        lds_barrier();
        if (kt + 2 < nk) load(st, kt + 2);
        compute(buf_tag);
      };
      for (int kt = 0; kt < nk; kt += 2) {
        slice(kt, std::integral_constant<int, 0>{});
        if (kt + 1 < nk) slice(kt + 1, std::integral_constant<int, 1>{});
      }
    } else {
      // One register buffer: slice kt + 1 is stored to the other LDS stage
      // after slice kt is multiplied, then slice kt + 2 is loaded.
      load(0, 0);
      store(0, 0);
      if (nk > 1) load(0, 1);
      lds_barrier();
      auto slice = [&](int kt, auto st_tag) {
        constexpr int st = decltype(st_tag)::value;  // LDS stage of slice kt
        compute(st_tag);
        if (kt + 1 < nk) store(0, st ^ 1);
        if (kt + 2 < nk) load(0, kt + 2);
        lds_barrier();
      };
      for (int kt = 0; kt < nk; kt += 2) {
        slice(kt, std::integral_constant<int, 0>{});
        if (kt + 1 < nk) slice(kt + 1, std::integral_constant<int, 1>{});
      }
    }
  }

  // Epilogue: F = combine(Ahat, T) for the wave's block, one code path per
  // formula (the switch is uniform). The Ahat values of each 32 x 32
  // accumulator are loaded together before its stores, so their latencies
  // overlap (the stores could alias the planes for all the compiler knows).
  // With fp16 planes the additive formula reads X alone: F = Ahat - lambda T
  // then errs by at most 2^-12 |Ahat|, far inside the bound on F.
  const int half = lane >> 5;
  const int64_t ib = ti * TI + wi * (TI / WI) + 4 * half;
  const int64_t jb = tj * TJ + wj * (TJ / WJ) + (lane & 31);
  const size_t obase = static_cast<size_t>(bh) * a.M * a.M;
  // Fused additive form: the accumulator is F. F is written once and read
  // once, by the block selection, so its stores carry the non-temporal
  // hint (FRC stage 4 % faster at config 3). Stores go through a buffer
  // descriptor over this (b, h)'s F with 32-bit byte offsets (M <= 32767, so
  // M^2 4 < 2^32; M = 32768 takes the general epilogue), so an element
  // outside the M x M matrix (the padded rows and columns of edge tiles) takes
  // an offset past the range, which the hardware drops: no branch per element.
  auto epilogue_fused = [&]() {
    const uint64_t fbytes = static_cast<uint64_t>(a.M) * static_cast<uint64_t>(a.M) * 4u;
    // The base and size through readfirstlane: computed through 64-bit
    // divisions, they would otherwise be taken for divergent, and every store
    // wrapped in a loop over the lanes' descriptors.
    auto uni = [](uint32_t x) {
      return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x)));
    };
    const uint64_t fb = reinterpret_cast<uint64_t>(a.frc + obase);
    float* const fbase = reinterpret_cast<float*>((static_cast<uint64_t>(uni(static_cast<uint32_t>(fb >> 32))) << 32) |
                                                  uni(static_cast<uint32_t>(fb)));
    const brsrc_t frs = make_rsrc(fbase, uni(static_cast<uint32_t>(fbytes)));
    constexpr uint32_t DROP = 0xffffffffu;
    const uint32_t m = static_cast<uint32_t>(a.M), rstep = 4u * m;
    if (constant) {  // uniform: a constant A's F = c - lambda M c^2 everywhere
      const float fconst = cval - a.lambda * (static_cast<float>(a.M) * cval * cval);
#pragma unroll
      for (int x = 0; x < XS; ++x)
#pragma unroll
        for (int y = 0; y < YS; ++y)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[x][y][e] = fconst;
    }
    // Whole tiles (every edge tile's padded rows and columns aside) store
    // without a range test; edge tiles send the padding past the range.
    auto store_all = [&](auto full_tag) {
      constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
      for (int y = 0; y < YS; ++y) {
        const uint32_t j = static_cast<uint32_t>(jb + y * 32);
#pragma unroll
        for (int x = 0; x < XS; ++x) {
          const uint32_t i0 = static_cast<uint32_t>(ib + x * 32);
          const uint32_t base = 4u * (i0 * m + j);  // wraps only for rows or columns past M
          const uint32_t rows_left = j < m && i0 < m ? m - i0 : 0u;  // rows r < rows_left are in M
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const uint32_t r = 8 * (e >> 2) + (e & 3);
            const float f = __builtin_isfinite(acc[x][y][e]) ? acc[x][y][e] : 0.f;
            uint32_t off = base + r * rstep;
            if constexpr (!FULL) off = r < rows_left ? off : DROP;
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, f), frs, off, 0u, CPOL_NT);
          }
        }
      }
    };
    if ((ti + 1) * TI <= a.M && (tj + 1) * TJ <= a.M)
      store_all(std::true_type{});
    else
      store_all(std::false_type{});
  };
  auto epilogue = [&](auto form_tag) {
    constexpr int FORM = decltype(form_tag)::value;
    constexpr bool FUSED = FORM < 0;  // F = X (I - lambda X) accumulated directly
    constexpr bool LO = !(F16 && (FORM == CAB_FRC_ADDITIVE || FUSED));
#pragma unroll
    for (int y = 0; y < YS; ++y) {
      const int64_t j = jb + y * 32;
      if (j >= a.M) continue;
      const float sj = FORM == CAB_FRC_AUGMENTED ? a.rowsum[bh * a.Mp + j] : 0.f;
#pragma unroll
      for (int x = 0; x < XS; ++x) {
        const int64_t i0 = ib + x * 32;
        // Rows past M (< Mp) lie inside the zero-padded planes.
        const uint16_t* xh = a.xhi + pbase + i0 * a.Mp + j;
        const uint16_t* xl = a.xlo + pbase + i0 * a.Mp + j;
        const int mp = static_cast<int>(a.Mp);
        uint16_t hi[16], lo[16];
        if constexpr (!FUSED) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int r = 8 * (e >> 2) + (e & 3);
            hi[e] = xh[r * mp];
            if constexpr (LO) lo[e] = xl[r * mp];
          }
        }
        float* fo = a.frc + obase + i0 * a.M + j;
        float* to = a.tri ? a.tri + obase + i0 * a.M + j : nullptr;
        const int m = static_cast<int>(a.M);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = 8 * (e >> 2) + (e & 3);
          if (i0 + r >= a.M) continue;
          float t = acc[x][y][e], ahat;
          if constexpr (FUSED) {
            float f = constant ? cval - a.lambda * (static_cast<float>(a.M) * cval * cval) : t;
            fo[r * m] = isfinite(f) ? f : 0.f;
            continue;
          } else if constexpr (F16) {
            ahat = f16_to_f32(hi[e]);
            if constexpr (LO) ahat += f16_to_f32(lo[e]);
            if (constant) {
              ahat = cval;
              t = static_cast<float>(a.M) * cval * cval;
            }
          } else {
            ahat = bf16_to_f32(hi[e]) + bf16_to_f32(lo[e]);
          }
          const float si = FORM == CAB_FRC_AUGMENTED ? a.rowsum[bh * a.Mp + i0 + r] : 0.f;
          fo[r * m] = frc_combine(FORM, ahat, t, a.lambda, si, sj);
          if (to) to[r * m] = t;
        }
      }
    }
  };
  if (a.fused && a.M <= 32767)  // M^2 4 bytes within the 32-bit offsets
    epilogue_fused();
  else if (a.fused)
    epilogue(std::integral_constant<int, -1>{});
  else if (a.formula == CAB_FRC_ADDITIVE)
    epilogue(std::integral_constant<int, CAB_FRC_ADDITIVE>{});
  else if (a.formula == CAB_FRC_MULTIPLICATIVE)
    epilogue(std::integral_constant<int, CAB_FRC_MULTIPLICATIVE>{});
  else
    epilogue(std::integral_constant<int, CAB_FRC_AUGMENTED>{});
}

// Compute units of the current device (queried once per device).
int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Launches the STATS (emit = false) or EMIT pass; returns the number of
// min / max partials per (b, h) the STATS pass writes.
// Inputs the strip kernel takes (the others use the direct-load kernels).
bool strip_path(int dtype, int64_t D) { return dtype != CAB_F32 && D <= AG_DMAX; }

template <typename T>
int64_t launch_affinity(const AffArgs& a, int64_t BH, bool emit, hipStream_t s) {
  if constexpr (sizeof(T) == 2) {  // bf16_t, f16_t
    if (a.D <= AG_DMAX) {  // strip_path()
      // Strips as long as keeps every CU busy: two STATS or one EMIT workgroup
      // per CU (their LDS footprints), each walking `strip` tiles.
      const int64_t ns = a.Mp / AGT;  // Mp is a multiple of 128
      const int64_t slots = (emit ? 1 : 2) * static_cast<int64_t>(device_cus());
      int64_t strip = ceil_div(BH * ns * ns, slots);
      strip = strip < 1 ? 1 : (strip > ns ? ns : strip);
      const int64_t nstrip = ceil_div(ns, strip);
      AffArgs b = a;
      b.strip = strip;
      const unsigned grid = static_cast<unsigned>(BH * ns * nstrip);
      const unsigned threads = 64 * (emit ? AG_CW + AG_SW : AG_CW);
      if (a.D <= 64) {
        if (emit) aff_strip_kernel<T, true, 4><<<grid, threads, 0, s>>>(b);
        else aff_strip_kernel<T, false, 4><<<grid, threads, 0, s>>>(b);
      } else {
        if (emit) aff_strip_kernel<T, true, 8><<<grid, threads, 0, s>>>(b);
        else aff_strip_kernel<T, false, 8><<<grid, threads, 0, s>>>(b);
      }
      return ns * nstrip;
    }
  }
  const int64_t ns = ceil_div(a.Mp, AS);
  if (emit) {
    affinity_kernel<T><<<dim3(static_cast<unsigned>(a.ntw * a.ntw), static_cast<unsigned>(BH)), 256, 0,
                         s>>>(a);
  } else {
    affinity_stats_kernel<T><<<dim3(static_cast<unsigned>(ns * ns), static_cast<unsigned>(BH)), 512, 0,
                               s>>>(a);
  }
  return ns * ns;
}

}  // namespace
}  // namespace cab

using namespace cab;

extern "C" size_t cab_block_frc_workspace_bytes(int64_t B, int64_t H, int64_t M, int64_t D,
                                                int normalization, int formula) {
  (void)D;
  (void)normalization;
  (void)formula;
  if (B <= 0 || H <= 0 || M <= 0) return 0;
  return frc_layout(B * H, M).total;
}

extern "C" cab_status_t cab_block_frc(const void* qc, const void* kc, cab_dtype_t dtype,
                                      int64_t B, int64_t H, int64_t M, int64_t D, float scale,
                                      float temperature, float lambda_redundancy,
                                      int normalization, int formula, float* frc,
                                      float* affinity, float* triangles, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  clear_error();
  CAB_REQUIRE(valid_dtype(dtype), CAB_EDTYPE, "cab_block_frc: unknown dtype %d", (int)dtype);
  CAB_REQUIRE(B >= 0 && H >= 0 && M >= 0, CAB_ESHAPE, "cab_block_frc: negative size");
  CAB_REQUIRE(D >= 8 && D <= 512 && D % 8 == 0, CAB_ESHAPE,
              "cab_block_frc: head dim D=%lld must be a multiple of 8 in [8, 512]", (long long)D);
  CAB_REQUIRE(normalization == CAB_NORM_NONE || normalization == CAB_NORM_MINMAX, CAB_EINVAL,
              "cab_block_frc: unsupported normalization %d", normalization);
  CAB_REQUIRE(formula == CAB_FRC_ADDITIVE || formula == CAB_FRC_MULTIPLICATIVE ||
                  formula == CAB_FRC_AUGMENTED,
              CAB_EINVAL, "cab_block_frc: unsupported formula %d", formula);
  CAB_REQUIRE(temperature != 0.f && std::isfinite(temperature) && std::isfinite(scale) &&
                  std::isfinite(lambda_redundancy),
              CAB_EINVAL, "cab_block_frc: scale, temperature and lambda must be finite, temperature != 0");
  if (B == 0 || H == 0 || M == 0) return CAB_OK;
  CAB_REQUIRE(qc && kc && frc, CAB_EINVAL, "cab_block_frc: null tensor pointer");
  CAB_REQUIRE(reinterpret_cast<uintptr_t>(qc) % 16 == 0 && reinterpret_cast<uintptr_t>(kc) % 16 == 0,
              CAB_ESHAPE, "cab_block_frc: qc/kc not 16-byte aligned");
  CAB_REQUIRE(M <= 32768, CAB_ESHAPE, "cab_block_frc: M=%lld exceeds 32768", (long long)M);
  const int64_t BH = B * H;
  CAB_REQUIRE(BH <= 65535, CAB_ESHAPE, "cab_block_frc: B*H=%lld exceeds 65535", (long long)BH);
  const FrcLayout L = frc_layout(BH, M);
  CAB_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, CAB_EWORKSPACE,
              "cab_block_frc: workspace of %zu bytes given, %zu needed", workspace_bytes, L.total);
  CAB_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, CAB_EWORKSPACE,
              "cab_block_frc: workspace not 256-byte aligned");

  char* ws = static_cast<char*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  AffArgs a;
  a.qc = qc;
  a.kc = kc;
  a.M = M;
  a.Mp = L.Mp;
  a.nta = L.nta;
  a.ntw = L.ntw;
  a.D = static_cast<int32_t>(D);
  a.alpha = static_cast<float>(static_cast<double>(scale) / static_cast<double>(temperature));
  a.normalization = normalization;
  a.mmpart = reinterpret_cast<float*>(ws + L.off_mmpart);
  a.mm = reinterpret_cast<float*>(ws + L.off_mm);
  a.xhi = reinterpret_cast<uint16_t*>(ws + L.off_xhi);
  a.xlo = reinterpret_cast<uint16_t*>(ws + L.off_xlo);
  a.xthi = reinterpret_cast<uint16_t*>(ws + L.off_xthi);
  a.xtlo = reinterpret_cast<uint16_t*>(ws + L.off_xtlo);
  a.affinity = affinity;
  a.rspart = formula == CAB_FRC_AUGMENTED ? reinterpret_cast<float*>(ws + L.off_rspart) : nullptr;
  // fp16 planes where Ahat is known to lie in [0, 1] and the formula does not
  // cancel T against row sums.
  const bool f16 = normalization == CAB_NORM_MINMAX && formula != CAB_FRC_AUGMENTED;
  a.f16_planes = f16 ? 1 : 0;
  // Additive formula without the T diagnostic: F = Ahat (I - lambda Ahat) in
  // one GEMM (|lambda| bounded so that I - lambda Ahat fits fp16).
  const bool fused = f16 && formula == CAB_FRC_ADDITIVE && triangles == nullptr &&
                     std::fabs(lambda_redundancy) <= 1024.f;
  a.fused = fused ? 1 : 0;
  a.lambda = lambda_redundancy;
  a.strip = 1;

  a.nparts = 0;
  if (normalization == CAB_NORM_MINMAX) {
    switch (dtype) {
      case CAB_BF16: a.nparts = launch_affinity<bf16_t>(a, BH, false, s); break;
      case CAB_F16: a.nparts = launch_affinity<f16_t>(a, BH, false, s); break;
      default: a.nparts = launch_affinity<float>(a, BH, false, s); break;
    }
    cab_status_t st = launch_status("cab_block_frc/affinity_stats");
    if (st != CAB_OK) return st;
    // aff_strip_kernel's EMIT pass reduces the partials itself.
    if (!strip_path(dtype, D)) {
      minmax_finalize_kernel<<<static_cast<unsigned>(BH), 256, 0, s>>>(a.mmpart, a.nparts, a.mm);
      st = launch_status("cab_block_frc/minmax_finalize");
      if (st != CAB_OK) return st;
    }
  }
  switch (dtype) {
    case CAB_BF16: launch_affinity<bf16_t>(a, BH, true, s); break;
    case CAB_F16: launch_affinity<f16_t>(a, BH, true, s); break;
    default: launch_affinity<float>(a, BH, true, s); break;
  }
  cab_status_t st = launch_status("cab_block_frc/affinity_emit");
  if (st != CAB_OK) return st;
  if (formula == CAB_FRC_AUGMENTED) {
    dim3 g(static_cast<unsigned>(ceil_div(L.Mp, 256)), static_cast<unsigned>(BH));
    rowsum_finalize_kernel<<<g, 256, 0, s>>>(a.rspart, L.nta, L.Mp,
                                             reinterpret_cast<float*>(ws + L.off_rs));
    st = launch_status("cab_block_frc/rowsum_finalize");
    if (st != CAB_OK) return st;
  }
  TriArgs t;
  t.xhi = a.xhi;
  t.xlo = a.xlo;
  t.xthi = a.xthi;
  t.xtlo = a.xtlo;
  t.rowsum = reinterpret_cast<const float*>(ws + L.off_rs);
  t.mm = reinterpret_cast<const float*>(ws + L.off_mm);
  t.frc = frc;
  t.tri = triangles;
  t.M = M;
  t.Mp = L.Mp;
  t.BH = BH;
  t.lambda = lambda_redundancy;
  t.formula = formula;
  t.fused = fused ? 1 : 0;
  // The 256-wide tile (8 waves) stages half the bytes per flop of the
  // 128-wide one (4 waves); it is used when Mp allows it and its tiles still
  // give every CU work.
  const bool wide = L.Mp % TT_WIDE == 0 && BH * (L.Mp / TT_WIDE) * (L.Mp / TT_WIDE) >= 256;
  t.nti = t.ntj = L.Mp / (wide ? TT_WIDE : TT);
  const int64_t blocks = BH * t.nti * t.ntj;
  CAB_REQUIRE(blocks <= INT32_MAX, CAB_ESHAPE, "cab_block_frc: problem too large");
  const unsigned nb = static_cast<unsigned>(blocks);
  if (wide && f16)
    triangle_kernel<TT_WIDE, TT_WIDE, 2, 4, 0, true, 2 * TK><<<nb, 512, 0, s>>>(t);
  else if (wide)
    triangle_kernel<TT_WIDE, TT_WIDE, 2, 4, 1, false, TK><<<nb, 512, 0, s>>>(t);
  else if (f16)
    triangle_kernel<TT, TT, 2, 2, 2, true, TK><<<nb, 256, 0, s>>>(t);
  else
    triangle_kernel<TT, TT, 2, 2, 2, false, TK><<<nb, 256, 0, s>>>(t);
  return launch_status("cab_block_frc/triangles");
}
