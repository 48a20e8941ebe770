// Shared helpers of libcab_hip.so: status/error plumbing, element types,
// MFMA vector types and wave-level primitives for gfx950 (wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>

#include "../../include/cab_hip.h"

namespace cab {

// ----------------------------------------------------------------------------
// Host-side status handling
// ----------------------------------------------------------------------------

void set_error(const char* fmt, ...);
void clear_error();

#define CAB_REQUIRE(cond, code, ...)      \
  do {                                    \
    if (!(cond)) {                        \
      ::cab::set_error(__VA_ARGS__);      \
      return (code);                      \
    }                                     \
  } while (0)

// Checks the launch that was just enqueued.
cab_status_t launch_status(const char* what);

inline size_t dtype_size(cab_dtype_t dt) {
  return dt == CAB_F32 ? 4 : 2;
}

inline bool valid_dtype(int dt) {
  return dt == CAB_F32 || dt == CAB_F16 || dt == CAB_BF16;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// Workgroups are dispatched round-robin over the chip's 8 XCDs. This maps the
// hardware workgroup id to a logical id such that consecutive logical ids run
// on one XCD and share its L2. It is a bijection on [0, total).
__device__ __forceinline__ int64_t xcd_remap(int64_t hw, int64_t total) {
  const int64_t per = total / 8, rem = total % 8;
  const int64_t xcd = hw % 8, pos = hw / 8;
  return xcd < rem ? xcd * (per + 1) + pos : rem * (per + 1) + (xcd - rem) * per + pos;
}

// ----------------------------------------------------------------------------
// Element types (16-bit values are carried as raw uint16_t bits)
// ----------------------------------------------------------------------------

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bf16 bits (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t b) {
  _Float16 h = __builtin_bit_cast(_Float16, b);
  return static_cast<float>(h);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  static __device__ __forceinline__ double to_f64(float x) { return static_cast<double>(x); }
};
template <> struct Elem<bf16_t> {
  static __device__ __forceinline__ double to_f64(uint16_t x) { return static_cast<double>(bf16_to_f32(x)); }
};
template <> struct Elem<f16_t> {
  static __device__ __forceinline__ double to_f64(uint16_t x) { return static_cast<double>(f16_to_f32(x)); }
};

// ----------------------------------------------------------------------------
// Wave primitives
// ----------------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ double shfl_xor_f64(double v, int mask) {
  return __shfl_xor(v, mask, 64);
}

__device__ __forceinline__ float shfl_xor_f32(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

__device__ __forceinline__ int shfl_xor_i32(int v, int mask) {
  return __shfl_xor(v, mask, 64);
}

__device__ __forceinline__ uint64_t ballot64(bool p) {
  return __ballot(p);
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// Workgroup barrier that orders LDS accesses only: the fences are limited to
// the local address space, so global loads still in flight (a prefetch of a
// later stage) are not waited for, unlike __syncthreads().
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ----------------------------------------------------------------------------
// Buffer loads to LDS
// ----------------------------------------------------------------------------

typedef __attribute__((address_space(3))) void lds_void;

// 16-byte buffer load to LDS per lane: bytes [voff + soff, +16) of the buffer
// r land at LDS l + 16 * lane. Offsets at or past the buffer's size read as
// zero. The per-lane offset is a 32-bit register and the base a scalar
// descriptor, so no per-lane 64-bit address arithmetic is spent on a load.
typedef __amdgpu_buffer_rsrc_t brsrc_t;
__device__ __forceinline__ brsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // word 3 0x00020000: raw (untyped) dword access, the gfx9 buffer default
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ void bdma16(brsrc_t r, uint32_t voff, uint32_t soff, char* l) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)l, 16, voff, soff, 0, 0);
}

}  // namespace cab
