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

// Number of set bits of the wave mask m below this lane (v_mbcnt).
__device__ __forceinline__ uint32_t rank_below64(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
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
// Cache-policy operand of the buffer load / store builtins on gfx950: the
// non-temporal hint, for data written once and not read back soon.
constexpr int CPOL_NT = 2;
__device__ __forceinline__ void bdma16(brsrc_t r, uint32_t voff, uint32_t soff, char* l) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)l, 16, voff, soff, 0, 0);
}

// The same load issued as inline asm on a descriptor held in four scalar
// registers (base, size; raw dword access). The compiler does not see this
// load write LDS, so it adds no wait for it before later LDS reads: for a
// builtin LDS load it makes every later LDS read wait for all outstanding
// loads, whatever address they read. Callers wait (vmcnt(0)) and pass a
// workgroup barrier before any wave reads the bytes such a load writes, and
// never read a region while a load into it may be in flight.
typedef uint32_t sgpr_rsrc_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ sgpr_rsrc_t make_sgpr_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  auto uni = [](uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x)));
  };
  return sgpr_rsrc_t{uni(static_cast<uint32_t>(p)), uni(static_cast<uint32_t>(p >> 32) & 0xffffu),
                     uni(bytes), 0x00020000u};
}
__device__ __forceinline__ void bdma16_untracked(const sgpr_rsrc_t& r, uint32_t voff, uint32_t soff,
                                                 const void* l) {
  const uint32_t lds = static_cast<uint32_t>(
      __builtin_amdgcn_readfirstlane(static_cast<int>(reinterpret_cast<uintptr_t>(l))));
  // M0 (the LDS base of the load) is an input the compiler sets; the s_nop
  // is the wait state an LDS load needs after an M0 write.
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(r), "s"(soff), "{m0}"(lds)
               : "memory");
}

}  // namespace cab
