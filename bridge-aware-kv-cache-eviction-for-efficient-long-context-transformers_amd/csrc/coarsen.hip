// Max-L2 coarsening (cab_coarsen_maxl2).
//
// One wave64 per (tensor in {q, k}, b, h, block m). L lanes cooperate on a
// token row: lane c of the group reads the 8 consecutive elements
// [8c, 8c+8) with one 16-byte (32-byte for fp32) load and sums their squares
// left to right in float64; the L partial sums are combined by an xor
// butterfly, which adds adjacent pairs first, so the norm is bit-identical to
// the documented canonical order. 64/L rows are in flight per step and U steps
// are loaded before any is reduced, so each lane keeps U loads outstanding;
// the rows are read once, with the non-temporal hint.
// The best (norm, token) per group is kept in registers, the groups are
// combined with the same comparator (NaN largest, ties to the lower token),
// and the chosen row is copied with 16-byte stores.
//
// HBM traffic per block: block_size * D * elem bytes read, D * elem + 4 bytes
// written; the kernel is bound by HBM bandwidth.
#include "cab_internal.h"

namespace cab {
namespace {

struct CoarsenArgs {
  const void* src[2];
  void* dst[2];
  int32_t* idx[2];
  int64_t stride[2][3];  // b, h, token strides in elements
  int64_t B, H, N, M;
  int32_t D, bs;
};

template <typename T> struct Chunk;

// 8 bf16 values in one 16-byte register quad.
template <> struct Chunk<bf16_t> {
  using elem = uint16_t;
  u32x4 v;
  __device__ __forceinline__ void load(const elem* p) { v = *reinterpret_cast<const u32x4*>(p); }
  __device__ __forceinline__ void load_nt(const elem* p) {
    v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  }
  __device__ __forceinline__ void zero() { v = u32x4{0u, 0u, 0u, 0u}; }
  __device__ __forceinline__ double sumsq() const {
    double s = 0.0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const double lo = static_cast<double>(__uint_as_float(v[w] << 16));
      const double hi = static_cast<double>(__uint_as_float(v[w] & 0xffff0000u));
      s = s + lo * lo;
      s = s + hi * hi;
    }
    return s;
  }
  __device__ __forceinline__ void store(elem* p) const { *reinterpret_cast<u32x4*>(p) = v; }
};

template <> struct Chunk<f16_t> {
  using elem = uint16_t;
  u32x4 v;
  __device__ __forceinline__ void load(const elem* p) { v = *reinterpret_cast<const u32x4*>(p); }
  __device__ __forceinline__ void load_nt(const elem* p) {
    v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  }
  __device__ __forceinline__ void zero() { v = u32x4{0u, 0u, 0u, 0u}; }
  __device__ __forceinline__ double sumsq() const {
    double s = 0.0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const double lo = static_cast<double>(f16_to_f32(static_cast<uint16_t>(v[w] & 0xffffu)));
      const double hi = static_cast<double>(f16_to_f32(static_cast<uint16_t>(v[w] >> 16)));
      s = s + lo * lo;
      s = s + hi * hi;
    }
    return s;
  }
  __device__ __forceinline__ void store(elem* p) const { *reinterpret_cast<u32x4*>(p) = v; }
};

// 8 fp32 values in two 16-byte quads.
template <> struct Chunk<float> {
  using elem = float;
  u32x4 a, b;
  __device__ __forceinline__ void load(const elem* p) {
    a = reinterpret_cast<const u32x4*>(p)[0];
    b = reinterpret_cast<const u32x4*>(p)[1];
  }
  __device__ __forceinline__ void load_nt(const elem* p) {
    a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + 1);
  }
  __device__ __forceinline__ void zero() {
    a = u32x4{0u, 0u, 0u, 0u};
    b = a;
  }
  __device__ __forceinline__ double sumsq() const {
    double s = 0.0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const double x = static_cast<double>(__uint_as_float(a[w]));
      s = s + x * x;
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const double x = static_cast<double>(__uint_as_float(b[w]));
      s = s + x * x;
    }
    return s;
  }
  __device__ __forceinline__ void store(elem* p) const {
    reinterpret_cast<u32x4*>(p)[0] = a;
    reinterpret_cast<u32x4*>(p)[1] = b;
  }
};

// Total order of candidates: NaN first, then larger norm, then lower token.
__device__ __forceinline__ bool better(double v, int64_t t, double bv, int64_t bt) {
  const bool vn = isnan(v), bn = isnan(bv);
  if (vn != bn) return vn;
  if (!vn && v != bv) return v > bv;
  return t < bt;
}

template <typename T, int L>
__global__ __launch_bounds__(256) void coarsen_kernel(CoarsenArgs a) {
  using elem = typename Chunk<T>::elem;
  constexpr int R = 64 / L;  // rows per step
  constexpr int U = 4;       // steps loaded before reduction (more waves beat deeper batches)
  const int lane = lane_id();
  const int64_t units = a.B * a.H * a.M;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (wave >= 2 * units) return;  // uniform per wave
  const int which = wave >= units ? 1 : 0;
  const int64_t u = wave - which * units;
  const int64_t bh = u / a.M;
  const int64_t m = u - bh * a.M;
  const int64_t b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const elem* base = static_cast<const elem*>(a.src[which]) + b * a.stride[which][0] +
                     h * a.stride[which][1];
  const int64_t ts = a.stride[which][2];
  const int64_t t0 = m * a.bs;
  const int64_t tend = min(t0 + static_cast<int64_t>(a.bs), a.N);
  const int c = lane % L, r = lane / L;
  const bool cact = c < (a.D >> 3);

  double best_v = -1.0;
  int64_t best_t = INT64_MAX;
  for (int64_t tb = t0; tb < tend; tb += R * U) {
    Chunk<T> ch[U];
#pragma unroll
    for (int s = 0; s < U; ++s) {
      const int64_t t = tb + s * R + r;
      if (cact && t < tend)
        ch[s].load_nt(base + t * ts + 8 * c);  // streamed once: non-temporal (4-6 % faster)
      else
        ch[s].zero();
    }
#pragma unroll
    for (int s = 0; s < U; ++s) {
      double v = ch[s].sumsq();
#pragma unroll
      for (int off = 1; off < L; off <<= 1) v = v + shfl_xor_f64(v, off);
      const int64_t t = tb + s * R + r;
      if (t < tend && better(v, t, best_v, best_t)) {
        best_v = v;
        best_t = t;
      }
    }
  }
#pragma unroll
  for (int off = L; off < 64; off <<= 1) {
    const double ov = shfl_xor_f64(best_v, off);
    const int64_t ot = __shfl_xor(best_t, off, 64);
    if (better(ov, ot, best_v, best_t)) {
      best_v = ov;
      best_t = ot;
    }
  }
  if (lane == 0 && a.idx[which] != nullptr) a.idx[which][u] = static_cast<int32_t>(best_t);
  if (r == 0 && cact) {
    Chunk<T> row;
    row.load(base + best_t * ts + 8 * c);
    row.store(static_cast<elem*>(a.dst[which]) + u * a.D + 8 * c);
  }
}

template <typename T>
void launch_coarsen(const CoarsenArgs& a, int lanes, dim3 grid, hipStream_t s) {
  switch (lanes) {
    case 1: coarsen_kernel<T, 1><<<grid, 256, 0, s>>>(a); break;
    case 2: coarsen_kernel<T, 2><<<grid, 256, 0, s>>>(a); break;
    case 4: coarsen_kernel<T, 4><<<grid, 256, 0, s>>>(a); break;
    case 8: coarsen_kernel<T, 8><<<grid, 256, 0, s>>>(a); break;
    case 16: coarsen_kernel<T, 16><<<grid, 256, 0, s>>>(a); break;
    case 32: coarsen_kernel<T, 32><<<grid, 256, 0, s>>>(a); break;
    default: coarsen_kernel<T, 64><<<grid, 256, 0, s>>>(a); break;
  }
}

}  // namespace
}  // namespace cab

using namespace cab;

extern "C" cab_status_t cab_coarsen_maxl2(const void* q, const void* k, cab_dtype_t dtype,
                                          int64_t B, int64_t H, int64_t N, int64_t D,
                                          const int64_t q_strides[4], const int64_t k_strides[4],
                                          int32_t block_size, void* qc, void* kc,
                                          int32_t* q_idx, int32_t* k_idx, void* stream) {
  clear_error();
  CAB_REQUIRE(valid_dtype(dtype), CAB_EDTYPE, "cab_coarsen_maxl2: unknown dtype %d", (int)dtype);
  CAB_REQUIRE(B >= 0 && H >= 0 && N >= 0, CAB_ESHAPE,
              "cab_coarsen_maxl2: negative size B=%lld H=%lld N=%lld", (long long)B,
              (long long)H, (long long)N);
  CAB_REQUIRE(D >= 8 && D <= 512 && D % 8 == 0, CAB_ESHAPE,
              "cab_coarsen_maxl2: head dim D=%lld must be a multiple of 8 in [8, 512]",
              (long long)D);
  CAB_REQUIRE(block_size >= 1, CAB_EINVAL, "cab_coarsen_maxl2: block_size=%d must be >= 1",
              (int)block_size);
  CAB_REQUIRE(q_strides != nullptr && k_strides != nullptr, CAB_EINVAL,
              "cab_coarsen_maxl2: null stride array");
  const int64_t M = ceil_div(N, block_size);
  if (B == 0 || H == 0 || M == 0) return CAB_OK;
  CAB_REQUIRE(q && k && qc && kc, CAB_EINVAL, "cab_coarsen_maxl2: null tensor pointer");
  const size_t es = dtype_size(dtype);
  const void* srcs[2] = {q, k};
  const int64_t* strides[2] = {q_strides, k_strides};
  for (int w = 0; w < 2; ++w) {
    CAB_REQUIRE(strides[w][3] == 1, CAB_ESHAPE,
                "cab_coarsen_maxl2: %s last-dim stride %lld must be 1", w ? "k" : "q",
                (long long)strides[w][3]);
    CAB_REQUIRE(reinterpret_cast<uintptr_t>(srcs[w]) % 16 == 0, CAB_ESHAPE,
                "cab_coarsen_maxl2: %s base pointer not 16-byte aligned", w ? "k" : "q");
    for (int d = 0; d < 3; ++d)
      CAB_REQUIRE(strides[w][d] >= 0 && (strides[w][d] * (int64_t)es) % 16 == 0, CAB_ESHAPE,
                  "cab_coarsen_maxl2: %s stride[%d]=%lld must keep rows 16-byte aligned",
                  w ? "k" : "q", d, (long long)strides[w][d]);
  }
  CAB_REQUIRE(reinterpret_cast<uintptr_t>(qc) % 16 == 0 && reinterpret_cast<uintptr_t>(kc) % 16 == 0,
              CAB_ESHAPE, "cab_coarsen_maxl2: output pointers not 16-byte aligned");
  CAB_REQUIRE(N <= INT32_MAX, CAB_ESHAPE, "cab_coarsen_maxl2: N=%lld exceeds int32 token index",
              (long long)N);

  CoarsenArgs a;
  a.src[0] = q;
  a.src[1] = k;
  a.dst[0] = qc;
  a.dst[1] = kc;
  a.idx[0] = q_idx;
  a.idx[1] = k_idx;
  for (int d = 0; d < 3; ++d) {
    a.stride[0][d] = q_strides[d];
    a.stride[1][d] = k_strides[d];
  }
  a.B = B;
  a.H = H;
  a.N = N;
  a.M = M;
  a.D = static_cast<int32_t>(D);
  a.bs = block_size;
  int lanes = 1;
  while (lanes < D / 8) lanes <<= 1;
  const int64_t waves = 2 * B * H * M;
  const int64_t blocks = ceil_div(waves, 4);
  CAB_REQUIRE(blocks <= INT32_MAX, CAB_ESHAPE, "cab_coarsen_maxl2: problem too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(blocks));
  switch (dtype) {
    case CAB_BF16: launch_coarsen<bf16_t>(a, lanes, grid, s); break;
    case CAB_F16: launch_coarsen<f16_t>(a, lanes, grid, s); break;
    default: launch_coarsen<float>(a, lanes, grid, s); break;
  }
  return launch_status("cab_coarsen_maxl2");
}
