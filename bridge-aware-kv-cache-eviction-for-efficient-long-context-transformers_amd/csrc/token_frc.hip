// Token-level Forman-Ricci curvature (cab_token_frc, cab_token_frc_from_keys)
// and the aggregated key-key attention matrix (cab_attention_symmetrize).
//
// For a weighted directed graph A [n, n]:
//   S_i = sum_j A_ij                              (node strength)
//   T_i = sum_j sum_k A_ij A_jk = sum_j A_ij S_j  (2-hop weight)
//   F_i = 4 S_i - 2 S_i + 3 T_i                   (node weight taken = S)
// T is A times the vector S, so the curvature is two HBM-bound passes over
// A (token_row_kernel<PASS 0>: row sums; <PASS 1>: row dots with S).
//
// From cached keys [B, H, N, D]:
//   x_n = mean_{b,h} keys[b,h,n,:],  kn_n = x_n / max(|x_n|, 1e-12),
//   r_i = sum_j relu(kn_i . kn_j),   A_ij = relu(kn_i . kn_j) / (r_i + 1e-8).
// A is never stored: S_i = r_i / (r_i + 1e-8) and
// T_i = (sum_j relu(kn_i . kn_j) S_j) / (r_i + 1e-8). keys_prep_kernel
// writes kn as bf16 hi/lo planes in MFMA operand order; gram_kernel<PASS>
// computes 32x32 tiles of kn kn^T on MFMA (hi*hi + hi*lo + lo*hi, fp32
// accumulate; column operands staged once per workgroup through LDS) and
// folds each tile into per-row sums of relu(g) * w_j (w = 1, then w = S).
// The Gram matrix is symmetric, so only the tiles at or right of each
// 256-row block's diagonal block are formed: those right of it also fold
// their columns, relu(g) * w_i summed over the block's rows, into the sums of
// the rows j they stand for. gram_finalize_kernel adds the row partials of
// the column splits and the column partials of the earlier row blocks, in a
// fixed order. Algorithmic work: N^2 D flops per Gram pass (the upper
// triangle), plus the 256 x 256 diagonal blocks in full.
#include "cab_internal.h"

namespace cab {
namespace {

// ---------------------------------------------------------------------------
// Matrix form
// ---------------------------------------------------------------------------

template <typename T>
__device__ __forceinline__ float ld_elem(const T* p);
template <>
__device__ __forceinline__ float ld_elem<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float ld_elem<bf16_t>(const bf16_t* p) { return bf16_to_f32(p->bits); }
template <>
__device__ __forceinline__ float ld_elem<f16_t>(const f16_t* p) { return f16_to_f32(p->bits); }

// 16 bytes of elements as floats (4 fp32 or 8 16-bit values), read with the
// non-temporal hint: each pass streams the matrix once (passes 10 % faster).
template <typename T>
__device__ __forceinline__ void ld_vec(const T* p, float* x) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  if constexpr (std::is_same<T, float>::value) {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = __uint_as_float(v[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t lo = static_cast<uint16_t>(v[e] & 0xffffu), hi = static_cast<uint16_t>(v[e] >> 16);
      if constexpr (std::is_same<T, bf16_t>::value) {
        x[2 * e] = bf16_to_f32(lo);
        x[2 * e + 1] = bf16_to_f32(hi);
      } else {
        x[2 * e] = f16_to_f32(lo);
        x[2 * e + 1] = f16_to_f32(hi);
      }
    }
  }
}

struct RowArgs {
  const void* a;
  int64_t n, lda;  // elements
  float* s;        // strengths: written by pass 0, read by pass 1
  float* t;        // triangles (pass 1) or null
  float* f;        // curvature (pass 1)
};

// One wave per row; each lane sums a fixed, strided subset of the row and a
// butterfly adds the lanes, so the result does not depend on timing.
template <typename T, int PASS, bool VEC>
__global__ __launch_bounds__(256) void token_row_kernel(RowArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (i >= a.n) return;  // whole wave
  const int lane = lane_id();
  const T* row = static_cast<const T*>(a.a) + i * a.lda;
  float acc = 0.f;
  int64_t j_tail = 0;
  if constexpr (VEC) {
    constexpr int V = 16 / sizeof(T);
    const int64_t nv = a.n / V * V;
#pragma unroll 8  // eight 16-byte loads in flight per lane (4: 5 % slower, 16: 1 % slower)
    for (int64_t j = static_cast<int64_t>(lane) * V; j < nv; j += 64 * V) {
      float x[V];
      ld_vec<T>(row + j, x);
      float part = 0.f;
      if constexpr (PASS == 0) {
#pragma unroll
        for (int e = 0; e < V; ++e) part += x[e];
      } else {
        float w[V];
#pragma unroll
        for (int q = 0; q < V / 4; ++q) {
          const f32x4 sv = *reinterpret_cast<const f32x4*>(a.s + j + 4 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) w[4 * q + e] = sv[e];
        }
#pragma unroll
        for (int e = 0; e < V; ++e) part = fmaf(x[e], w[e], part);
      }
      acc += part;
    }
    j_tail = nv;
  }
  for (int64_t j = j_tail + lane; j < a.n; j += 64) {
    const float x = ld_elem<T>(row + j);
    acc += PASS == 0 ? x : x * a.s[j];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += shfl_xor_f32(acc, off);
  if (lane == 0) {
    if constexpr (PASS == 0) {
      a.s[i] = acc;
    } else {
      const float s = a.s[i];
      if (a.t) a.t[i] = acc;
      a.f[i] = 4.f * s - 2.f * s + 3.f * acc;
    }
  }
}

struct SymArgs {
  const void* a;
  int64_t bh, H, nq, nk, n;
  int64_t st[4];
  float* out;
  int64_t ldo;
  int64_t tiles;  // tiles per dim (32 x 32)
};

// out[x][y] = (agg[y][x] + agg[x][y]) / 2, agg = mean over (b, h), with a
// size-1 query or key dim broadcast. A workgroup owns the tile pair
// (I, J), (J, I) for I <= J: every input element is read once.
template <typename T>
__global__ __launch_bounds__(256) void symmetrize_kernel(SymArgs a) {
  const int64_t I = blockIdx.y, J = blockIdx.x;
  if (I > J) return;
  __shared__ float t1[32][33], t2[32][33];
  const int r = threadIdx.x >> 3, c0 = (threadIdx.x & 7) * 4;
  float s1[4] = {0.f, 0.f, 0.f, 0.f}, s2[4] = {0.f, 0.f, 0.f, 0.f};
  const T* base = static_cast<const T*>(a.a);
  const int64_t x1 = I * 32 + r, x2 = J * 32 + r;
  for (int64_t bh = 0; bh < a.bh; ++bh) {
    const int64_t b = bh / a.H, h = bh - (bh / a.H) * a.H;
    const T* m = base + b * a.st[0] + h * a.st[1];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t y1 = J * 32 + c0 + q, y2 = I * 32 + c0 + q;
      if (x1 < a.n && y1 < a.n)
        s1[q] += ld_elem<T>(m + (a.nq == 1 ? 0 : x1) * a.st[2] + (a.nk == 1 ? 0 : y1) * a.st[3]);
      if (x2 < a.n && y2 < a.n)
        s2[q] += ld_elem<T>(m + (a.nq == 1 ? 0 : x2) * a.st[2] + (a.nk == 1 ? 0 : y2) * a.st[3]);
    }
  }
  const float cnt = static_cast<float>(a.bh);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    t1[r][c0 + q] = s1[q] / cnt;  // agg[I*32 + r][J*32 + c]
    t2[r][c0 + q] = s2[q] / cnt;  // agg[J*32 + r][I*32 + c]
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = c0 + q;
    const int64_t y1 = J * 32 + c, y2 = I * 32 + c;
    if (x1 < a.n && y1 < a.n) a.out[x1 * a.ldo + y1] = (t2[c][r] + t1[r][c]) / 2.f;
    if (I != J && x2 < a.n && y2 < a.n) a.out[x2 * a.ldo + y2] = (t1[c][r] + t2[r][c]) / 2.f;
  }
}

// ---------------------------------------------------------------------------
// Key form
// ---------------------------------------------------------------------------

constexpr int GRAM_WAVES = 8;                // waves (32-row tiles) per Gram workgroup
constexpr int GRAM_ROWS = 32 * GRAM_WAVES;   // rows per workgroup

// Operand planes: for row tile t (32 rows) and k-step s (16 dims), lane
// L = (row % 32) + 32 * h holds dims 16 s + 8 h .. + 7 as one 16-byte value
// at index (t * dk + s) * 64 + L. This is the operand order of
// mfma_f32_32x32x16_bf16 for A (rows) and B (columns) alike.
struct KeyLayout {
  int64_t Np, dk, rb, tiles;  // padded rows, k-steps, 256-row blocks, 32-column tiles
  int64_t col_tiles, cs, wgs;  // tiles per workgroup, most splits of a row block, workgroups
  size_t off_hi, off_lo, off_r, off_s, off_part, off_cpart, total;
};

// Column splits of row block x: its tiles run from 8 x (the diagonal block)
// to the last one.
__host__ __device__ __forceinline__ int64_t gram_splits(int64_t x, int64_t tiles, int64_t col_tiles) {
  return (tiles - 8 * x + col_tiles - 1) / col_tiles;
}

KeyLayout key_layout(int64_t N, int64_t D) {
  KeyLayout L;
  L.Np = round_up(N > 0 ? N : 1, GRAM_ROWS);
  L.dk = D <= 64 ? 4 : D <= 128 ? 8 : 16;
  L.rb = L.Np / GRAM_ROWS;
  L.tiles = L.Np / 32;
  // About 512 workgroups (two rounds over the CUs) over the upper-triangle
  // tiles, at least 8 tiles each; splits up to 10 % longer are taken when
  // they keep the count at 512 (each row block's last split is shorter).
  const int64_t work = L.rb * L.tiles - 4 * L.rb * (L.rb - 1);
  L.col_tiles = ceil_div(work, 512);
  if (L.col_tiles < 8) L.col_tiles = 8;
  const int64_t longest = L.col_tiles + L.col_tiles / 10;
  for (;;) {
    L.wgs = 0;
    for (int64_t x = 0; x < L.rb; ++x) L.wgs += gram_splits(x, L.tiles, L.col_tiles);
    if (L.wgs <= 512 || L.col_tiles >= longest || L.col_tiles >= L.tiles) break;
    ++L.col_tiles;
  }
  L.cs = gram_splits(0, L.tiles, L.col_tiles);
  const size_t plane = static_cast<size_t>(L.Np) * L.dk * 16 * 2;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += static_cast<size_t>(round_up(static_cast<int64_t>(bytes), 256));
    return at;
  };
  L.off_hi = take(plane);
  L.off_lo = take(plane);
  L.off_r = take(static_cast<size_t>(L.Np) * 4);
  L.off_s = take(static_cast<size_t>(L.Np) * 4);
  L.off_part = take(static_cast<size_t>(L.cs) * L.Np * 4);
  L.off_cpart = take(static_cast<size_t>(L.rb) * L.Np * 4);
  L.total = o;
  return L;
}

struct PrepArgs {
  const void* k;
  int64_t H, bh, N, D, Np, dk;
  int64_t st[4];
  u32x4* hi;
  u32x4* lo;
};

// One wave per position: lane l (l < 32) owns dims 8 (l % 32) .. + 7, and
// the two lane halves sum the even and odd (b, h) slices. VEC: unit dim
// stride and 16-byte aligned rows, so a lane's dims are one or two 16-byte
// loads per slice.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void keys_prep_kernel(PrepArgs a) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (n >= a.Np) return;
  const int lane = lane_id(), g = lane & 31, par = lane >> 5;
  float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (n < a.N) {
    const T* base = static_cast<const T*>(a.k);
    for (int64_t bh = par; bh < a.bh; bh += 2) {
      const int64_t b = bh / a.H, h = bh - (bh / a.H) * a.H;
      const T* p = base + b * a.st[0] + h * a.st[1] + n * a.st[2];
      if constexpr (VEC) {
        if (8 * g < a.D) {  // D % 8 == 0 on this path
          float v[8];
          if constexpr (sizeof(T) == 4) {
            ld_vec<T>(p + 8 * g, v);
            ld_vec<T>(p + 8 * g + 4, v + 4);
          } else {
            ld_vec<T>(p + 8 * g, v);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] += v[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t d = 8 * g + e;
          if (d < a.D) x[e] += ld_elem<T>(p + d * a.st[3]);
        }
      }
    }
  }
  const float cnt = static_cast<float>(a.bh);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x[e] += __shfl_xor(x[e], 32, 64);
    x[e] = x[e] / cnt;
    ss = fmaf(x[e], x[e], ss);
  }
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) ss += shfl_xor_f32(ss, off);
  const float den = fmaxf(sqrtf(ss), 1e-12f);
  if (par == 0 && g < 2 * a.dk) {
    u32x4 h4, l4;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float v0 = x[2 * q] / den, v1 = x[2 * q + 1] / den;
      const uint16_t h0 = f32_to_bf16(v0), h1 = f32_to_bf16(v1);
      const uint16_t l0 = f32_to_bf16(v0 - bf16_to_f32(h0)), l1 = f32_to_bf16(v1 - bf16_to_f32(h1));
      h4[q] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
      l4[q] = static_cast<uint32_t>(l0) | (static_cast<uint32_t>(l1) << 16);
    }
    const int64_t s = g >> 1, hh = g & 1;
    const int64_t idx = ((n >> 5) * a.dk + s) * 64 + (n & 31) + 32 * hh;
    a.hi[idx] = h4;
    a.lo[idx] = l4;
  }
}

struct GramArgs {
  const u32x4* hi;
  const u32x4* lo;
  const float* w;  // pass 1: S (zero past N)
  float* part;     // [cs][Np] row partials per column split
  float* cpart;    // [Np][rb] column partials per row block (columns right of its diagonal block)
  int64_t Np, tiles, col_tiles, rb;
};


constexpr int GRAM_STAGES = 3;

// Workgroup b stands for split y of row block x (the splits of the blocks in
// order). Wave w owns row tile GRAM_WAVES x + w (its A operands in
// registers) and the waves walk the same column tiles 8 x + [y col_tiles,
// (y + 1) col_tiles). Each column tile's B operands (hi and lo, 1 KB per
// k-step and plane) and, in pass 1, its 32 weights are staged once per
// workgroup into a ring of three LDS stages by buffer loads to LDS, two tiles
// ahead (the waves split the 2 DK 1 KB loads evenly). Each 32x32 tile of
// kn kn^T is folded into 16 per-lane row partials (lane l: column l % 32, rows
// 8 (e / 4) + 4 (l / 32) + e % 4), added over the lanes at the end. A tile
// right of the diagonal block also yields its 32 column sums over the wave's
// rows; the waves' sums meet in LDS and wave 0 adds them in order after the
// next barrier.
template <int DK, int PASS>
__global__ __launch_bounds__(64 * GRAM_WAVES) void gram_kernel(GramArgs a) {
  constexpr int PLANE_BYTES = DK * 1024;           // one plane's k-steps of a column tile
  constexpr int STAGE_BYTES = 2 * PLANE_BYTES + 256 * GRAM_WAVES;  // hi, lo, weight copies
  constexpr int PER_WAVE = 2 * DK / GRAM_WAVES;    // 1 KB operand loads per wave and tile
  static_assert(PER_WAVE * GRAM_WAVES == 2 * DK, "operand loads split evenly over the waves");
  constexpr int NDMA = PER_WAVE + (PASS == 1 ? 1 : 0);
  static_assert(NDMA < 16, "vmcnt immediate");
  __shared__ __attribute__((aligned(16))) char ring[GRAM_STAGES * STAGE_BYTES];
  __shared__ float cbuf[GRAM_STAGES][GRAM_WAVES][32];
  const int lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  int64_t x = 0, y = blockIdx.x;
  for (;;) {
    if (x >= a.rb) return;  // past the last split (uniform per workgroup)
    const int64_t n = gram_splits(x, a.tiles, a.col_tiles);
    if (y < n) break;
    y -= n;
    ++x;
  }
  const int64_t rt = x * GRAM_WAVES + w;
  const int64_t diag_end = (x + 1) * GRAM_WAVES;  // first column tile right of the diagonal block
  u32x4 ah[DK], al[DK];
#pragma unroll
  for (int s = 0; s < DK; ++s) {
    ah[s] = a.hi[(rt * DK + s) * 64 + lane];
    al[s] = a.lo[(rt * DK + s) * 64 + lane];
  }
  const int half = lane >> 5;
  // Row weights of this lane's 16 rows (for the column sums).
  float wr[16];
#pragma unroll
  for (int e = 0; e < 16; ++e)
    wr[e] = PASS == 0 ? 1.f : a.w[rt * 32 + 8 * (e >> 2) + 4 * half + (e & 3)];
  float p[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) p[e] = 0.f;
  const int64_t c0 = x * GRAM_WAVES + y * a.col_tiles;
  const int64_t c1 = c0 + a.col_tiles < a.tiles ? c0 + a.col_tiles : a.tiles;
  const int nt = static_cast<int>(c1 - c0);

  const int plane = (w * PER_WAVE) / DK, s0 = (w * PER_WAVE) % DK;
  const u32x4* src_plane = plane == 0 ? a.hi : a.lo;
  // The loads go through a buffer descriptor per column tile (its DK KB of
  // one plane; pass 1: its 32 weights), so a lane's offsets are the same for
  // every tile and the staging costs no vector address arithmetic. The bases
  // are uniform; readfirstlane lets the compiler see it (a descriptor it
  // takes for divergent is wrapped in a loop over the lanes' values).
  auto uniform = [](const void* p) {
    const uint64_t u = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u >> 32)));
    return reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo);
  };
  auto issue = [&](int it) {
    const int64_t ct = c0 + it;
    char* st = ring + (it % GRAM_STAGES) * STAGE_BYTES;
    const brsrc_t prs = make_rsrc(uniform(src_plane + ct * DK * 64), static_cast<uint32_t>(DK * 1024));
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q)
      bdma16(prs, static_cast<uint32_t>(((s0 + q) * 64 + lane) * 16), 0u,
             st + plane * PLANE_BYTES + (s0 + q) * 1024);
    if constexpr (PASS == 1) {
      const brsrc_t wrs = make_rsrc(uniform(a.w + ct * 32), 128u);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void*)(st + 2 * PLANE_BYTES + 256 * w), 4,
                                               4u * static_cast<uint32_t>(lane & 31), 0, 0, 0);
    }
  };
  // Wave 0 adds the waves' column sums of tile it (staged in cbuf[S]).
  auto flush_cols = [&](int it, int S) {
    const int64_t ct = c0 + it;
    if (w == 0 && ct >= diag_end && lane < 32) {
      float v = 0.f;
#pragma unroll
      for (int q = 0; q < GRAM_WAVES; ++q) v += cbuf[S][q][lane];
      a.cpart[(ct * 32 + lane) * a.rb + x] = v;
    }
  };
  for (int it = 0; it < GRAM_STAGES - 1 && it < nt; ++it) issue(it);
  // Tile it lives in stage it % 3, a compile-time constant below, so the
  // compiler sees the staging of tile it + 2 cannot alias this tile's reads.
  auto step = [&](int it, auto stage_tag) {
    constexpr int S = decltype(stage_tag)::value;
    // vmcnt(NDMA) (tile it + 1 may be in flight) or vmcnt(0), and lgkmcnt(0):
    // the column sums this wave wrote to cbuf are in LDS before the barrier.
    if (it + 1 < nt)
      __builtin_amdgcn_s_waitcnt(0x0070 | NDMA);
    else
      __builtin_amdgcn_s_waitcnt(0x0070);
    __builtin_amdgcn_s_barrier();  // every wave's part of tile it landed; stage (S + 2) % 3 is free
    if (it + GRAM_STAGES - 1 < nt) issue(it + GRAM_STAGES - 1);
    if (it > 0) flush_cols(it - 1, (S + GRAM_STAGES - 1) % GRAM_STAGES);
    const char* st = ring + S * STAGE_BYTES;
    const float wc = PASS == 0 ? 1.f : reinterpret_cast<const float*>(st + 2 * PLANE_BYTES + 256 * w)[lane & 31];
    f32x16 acc = {};
#pragma unroll
    for (int s = 0; s < DK; ++s) {
      const u32x4 bh = reinterpret_cast<const u32x4*>(st + s * 1024)[lane];
      const u32x4 bl = reinterpret_cast<const u32x4*>(st + PLANE_BYTES + s * 1024)[lane];
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, al[s]),
                                                    __builtin_bit_cast(bf16x8, bh), acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ah[s]),
                                                    __builtin_bit_cast(bf16x8, bl), acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ah[s]),
                                                    __builtin_bit_cast(bf16x8, bh), acc, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) p[e] = fmaf(fmaxf(acc[e], 0.f), wc, p[e]);
    if (c0 + it >= diag_end) {
      float cs = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) cs = fmaf(fmaxf(acc[e], 0.f), wr[e], cs);
      cs += shfl_xor_f32(cs, 32);
      if (lane < 32) cbuf[S][w][lane] = cs;
    }
  };
  for (int it = 0; it < nt; it += GRAM_STAGES) {
    step(it, std::integral_constant<int, 0>{});
    if (it + 1 < nt) step(it + 1, std::integral_constant<int, 1>{});
    if (it + 2 < nt) step(it + 2, std::integral_constant<int, 2>{});
  }
  __syncthreads();
  flush_cols(nt - 1, (nt - 1) % GRAM_STAGES);
#pragma unroll
  for (int e = 0; e < 16; ++e) {
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) p[e] += shfl_xor_f32(p[e], off);
  }
  if ((lane & 31) == 0) {
    float* out = a.part + y * a.Np + rt * 32;
#pragma unroll
    for (int e = 0; e < 16; ++e) out[8 * (e >> 2) + 4 * half + (e & 3)] = p[e];
  }
}

struct FinArgs {
  const float* part;   // [cs][Np] row partials per column split
  const float* cpart;  // [Np][rb] column partials per row block
  int64_t tiles, col_tiles, rb, Np, N;
  float* r;           // workspace row sums
  float* s;           // workspace strengths (zero past N)
  float* out_s;       // optional outputs
  float* out_t;
  float* out_r;
  float* out_f;
};

template <int PASS>
__global__ __launch_bounds__(256) void gram_finalize_kernel(FinArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= a.Np) return;
  // Row i of block xi: its splits' row partials, then the column partials
  // of the blocks above it, in order.
  const int64_t xi = i / GRAM_ROWS;
  const int64_t ns = gram_splits(xi, a.tiles, a.col_tiles);
  float sum = 0.f;
  for (int64_t c = 0; c < ns; ++c) sum += a.part[c * a.Np + i];
  const float* cp = a.cpart + i * a.rb;
  for (int64_t xb = 0; xb < xi; ++xb) sum += cp[xb];
  if constexpr (PASS == 0) {
    const float s = i < a.N ? sum / (sum + 1e-8f) : 0.f;
    a.r[i] = sum;
    a.s[i] = s;
    if (i < a.N) {
      if (a.out_r) a.out_r[i] = sum;
      if (a.out_s) a.out_s[i] = s;
    }
  } else {
    if (i >= a.N) return;
    const float t = sum / (a.r[i] + 1e-8f);
    const float s = a.s[i];
    if (a.out_t) a.out_t[i] = t;
    a.out_f[i] = 4.f * s - 2.f * s + 3.f * t;
  }
}

template <typename T>
cab_status_t launch_rows(const void* A, int64_t n, int64_t lda, float* s, float* t, float* f,
                         hipStream_t st, const char* fn) {
  RowArgs a{A, n, lda, s, t, f};
  const bool vec = reinterpret_cast<uintptr_t>(A) % 16 == 0 &&
                   (lda * static_cast<int64_t>(sizeof(T))) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(s) % 16 == 0;
  const unsigned grid = static_cast<unsigned>(ceil_div(n, 4));
  if (vec) {
    token_row_kernel<T, 0, true><<<grid, 256, 0, st>>>(a);
  } else {
    token_row_kernel<T, 0, false><<<grid, 256, 0, st>>>(a);
  }
  cab_status_t r = launch_status(fn);
  if (r != CAB_OK) return r;
  if (vec) {
    token_row_kernel<T, 1, true><<<grid, 256, 0, st>>>(a);
  } else {
    token_row_kernel<T, 1, false><<<grid, 256, 0, st>>>(a);
  }
  return launch_status(fn);
}

template <int DK, int PASS>
void launch_gram(const GramArgs& g, const KeyLayout& L, hipStream_t st) {
  gram_kernel<DK, PASS><<<static_cast<unsigned>(L.wgs), 64 * GRAM_WAVES, 0, st>>>(g);
}

}  // namespace
}  // namespace cab

using namespace cab;

extern "C" cab_status_t cab_token_frc(const void* attention, cab_dtype_t dtype, int64_t n,
                                      int64_t row_stride, float* strengths, float* triangles,
                                      float* frc, void* stream) {
  const char* fn = "cab_token_frc";
  clear_error();
  CAB_REQUIRE(valid_dtype(dtype), CAB_EDTYPE, "%s: unknown dtype %d", fn, static_cast<int>(dtype));
  CAB_REQUIRE(n >= 0 && ceil_div(n, 4) <= INT32_MAX, CAB_ESHAPE, "%s: bad n %lld", fn,
              static_cast<long long>(n));
  if (n == 0) return CAB_OK;
  CAB_REQUIRE(attention && strengths && frc, CAB_EINVAL, "%s: null attention / strengths / frc", fn);
  CAB_REQUIRE(row_stride >= n, CAB_ESHAPE, "%s: row_stride %lld below n %lld", fn,
              static_cast<long long>(row_stride), static_cast<long long>(n));
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case CAB_F32: return launch_rows<float>(attention, n, row_stride, strengths, triangles, frc, st, fn);
    case CAB_BF16: return launch_rows<bf16_t>(attention, n, row_stride, strengths, triangles, frc, st, fn);
    default: return launch_rows<f16_t>(attention, n, row_stride, strengths, triangles, frc, st, fn);
  }
}

extern "C" cab_status_t cab_attention_symmetrize(const void* attention, cab_dtype_t dtype, int64_t B,
                                                 int64_t H, int64_t N_q, int64_t N_k,
                                                 const int64_t strides[4], float* out,
                                                 int64_t out_stride, void* stream) {
  const char* fn = "cab_attention_symmetrize";
  clear_error();
  CAB_REQUIRE(valid_dtype(dtype), CAB_EDTYPE, "%s: unknown dtype %d", fn, static_cast<int>(dtype));
  CAB_REQUIRE(B >= 1 && H >= 1 && N_q >= 1 && N_k >= 1, CAB_ESHAPE, "%s: empty input", fn);
  CAB_REQUIRE(N_q == N_k || N_q == 1 || N_k == 1, CAB_ESHAPE,
              "%s: (agg^T + agg) needs N_q == N_k or a size-1 dim (got %lld, %lld)", fn,
              static_cast<long long>(N_q), static_cast<long long>(N_k));
  const int64_t n = N_q > N_k ? N_q : N_k;
  CAB_REQUIRE(attention && out && strides, CAB_EINVAL, "%s: null argument", fn);
  CAB_REQUIRE(out_stride >= n, CAB_ESHAPE, "%s: out_stride below n", fn);
  for (int d = 0; d < 4; ++d) CAB_REQUIRE(strides[d] >= 0, CAB_ESHAPE, "%s: negative stride", fn);
  const int64_t tiles = ceil_div(n, 32);
  CAB_REQUIRE(tiles <= 65535, CAB_ESHAPE, "%s: n %lld too large", fn, static_cast<long long>(n));
  SymArgs a{attention, B * H, H, N_q, N_k, n, {strides[0], strides[1], strides[2], strides[3]},
            out, out_stride, tiles};
  const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(tiles));
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case CAB_F32: symmetrize_kernel<float><<<grid, 256, 0, st>>>(a); break;
    case CAB_BF16: symmetrize_kernel<bf16_t><<<grid, 256, 0, st>>>(a); break;
    default: symmetrize_kernel<f16_t><<<grid, 256, 0, st>>>(a); break;
  }
  return launch_status(fn);
}

extern "C" size_t cab_token_frc_keys_workspace_bytes(int64_t N, int64_t D) {
  if (N < 0 || D < 1 || D > 256) return 0;
  return key_layout(N, D).total;
}

extern "C" cab_status_t cab_token_frc_from_keys(const void* keys, cab_dtype_t dtype, int64_t B,
                                                int64_t H, int64_t N, int64_t D,
                                                const int64_t strides[4], float* strengths,
                                                float* triangles, float* row_sums, float* frc,
                                                void* workspace, size_t workspace_bytes,
                                                void* stream) {
  const char* fn = "cab_token_frc_from_keys";
  clear_error();
  CAB_REQUIRE(valid_dtype(dtype), CAB_EDTYPE, "%s: unknown dtype %d", fn, static_cast<int>(dtype));
  CAB_REQUIRE(B >= 1 && H >= 1 && N >= 0 && D >= 1, CAB_ESHAPE, "%s: bad shape", fn);
  CAB_REQUIRE(D <= 256, CAB_ESHAPE, "%s: D %lld above 256", fn, static_cast<long long>(D));
  if (N == 0) return CAB_OK;
  CAB_REQUIRE(keys && frc && strides && workspace, CAB_EINVAL, "%s: null argument", fn);
  for (int d = 0; d < 4; ++d) CAB_REQUIRE(strides[d] >= 0, CAB_ESHAPE, "%s: negative stride", fn);
  const KeyLayout L = key_layout(N, D);
  CAB_REQUIRE(workspace_bytes >= L.total, CAB_EWORKSPACE, "%s: workspace %zu < %zu bytes", fn,
              workspace_bytes, L.total);
  CAB_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, CAB_EWORKSPACE,
              "%s: workspace not 256-byte aligned", fn);
  CAB_REQUIRE(L.Np / 4 <= INT32_MAX && L.wgs <= INT32_MAX, CAB_ESHAPE, "%s: N too large", fn);
  char* ws = static_cast<char*>(workspace);
  u32x4* hi = reinterpret_cast<u32x4*>(ws + L.off_hi);
  u32x4* lo = reinterpret_cast<u32x4*>(ws + L.off_lo);
  float* r = reinterpret_cast<float*>(ws + L.off_r);
  float* s = reinterpret_cast<float*>(ws + L.off_s);
  float* part = reinterpret_cast<float*>(ws + L.off_part);
  float* cpart = reinterpret_cast<float*>(ws + L.off_cpart);
  hipStream_t st = static_cast<hipStream_t>(stream);

  PrepArgs pa{keys, H, B * H, N, D, L.Np, L.dk, {strides[0], strides[1], strides[2], strides[3]},
              hi, lo};
  const unsigned pgrid = static_cast<unsigned>(L.Np / 4);
  // 16-byte loads when each position's D values are contiguous and every
  // row start (all b, h, n strides) keeps 16-byte alignment.
  const int64_t esz = dtype == CAB_F32 ? 4 : 2;
  const bool vec = strides[3] == 1 && D % 8 == 0 && reinterpret_cast<uintptr_t>(keys) % 16 == 0 &&
                   (strides[0] * esz) % 16 == 0 && (strides[1] * esz) % 16 == 0 &&
                   (strides[2] * esz) % 16 == 0;
  switch (dtype) {
    case CAB_F32:
      vec ? keys_prep_kernel<float, true><<<pgrid, 256, 0, st>>>(pa)
          : keys_prep_kernel<float, false><<<pgrid, 256, 0, st>>>(pa);
      break;
    case CAB_BF16:
      vec ? keys_prep_kernel<bf16_t, true><<<pgrid, 256, 0, st>>>(pa)
          : keys_prep_kernel<bf16_t, false><<<pgrid, 256, 0, st>>>(pa);
      break;
    default:
      vec ? keys_prep_kernel<f16_t, true><<<pgrid, 256, 0, st>>>(pa)
          : keys_prep_kernel<f16_t, false><<<pgrid, 256, 0, st>>>(pa);
      break;
  }
  cab_status_t rc = launch_status(fn);
  if (rc != CAB_OK) return rc;

  GramArgs g{hi, lo, s, part, cpart, L.Np, L.tiles, L.col_tiles, L.rb};
  FinArgs f{part, cpart, L.tiles, L.col_tiles, L.rb, L.Np, N, r, s, strengths, triangles, row_sums, frc};
  const unsigned fgrid = static_cast<unsigned>(ceil_div(L.Np, 256));
  for (int pass = 0; pass < 2; ++pass) {
    if (L.dk == 4) {
      pass == 0 ? launch_gram<4, 0>(g, L, st) : launch_gram<4, 1>(g, L, st);
    } else if (L.dk == 8) {
      pass == 0 ? launch_gram<8, 0>(g, L, st) : launch_gram<8, 1>(g, L, st);
    } else {
      pass == 0 ? launch_gram<16, 0>(g, L, st) : launch_gram<16, 1>(g, L, st);
    }
    rc = launch_status(fn);
    if (rc != CAB_OK) return rc;
    if (pass == 0) {
      gram_finalize_kernel<0><<<fgrid, 256, 0, st>>>(f);
    } else {
      gram_finalize_kernel<1><<<fgrid, 256, 0, st>>>(f);
    }
    rc = launch_status(fn);
    if (rc != CAB_OK) return rc;
  }
  return CAB_OK;
}
