// Shared device/host helpers for the gfx950 paged-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tmopt_attn.h"

namespace tmopt {

// ---- vector types (clang ext_vector_type, as the MFMA builtins expect) ----
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---- bf16 bit helpers ----------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) {
  return __builtin_bit_cast(float, b16 << 16);
}

// fp32 -> bf16 round-to-nearest-even (NaN kept quiet), as bits.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)f);
}

// pack two bf16 bit patterns (lo, hi) into one dword
__device__ __forceinline__ uint32_t pack_bf16x2(uint32_t lo, uint32_t hi) {
  return (lo & 0xffffu) | (hi << 16);
}

// Two fp32 -> one dword of two bf16 (lo, hi), round-to-nearest-even, in one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2_rn(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(
      uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// Interleave the low (sel=0) or high (sel=1) bf16 halves of two dwords:
// result = { a.half[sel], b.half[sel] }.
__device__ __forceinline__ uint32_t interleave_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t interleave_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}
__device__ __forceinline__ float fast_log2(float x) {
  return __builtin_amdgcn_logf(x);
}

// Reductions over lane pairs (l, l ^ 16) and (l, l ^ 32) by the gfx950
// row-swap instructions (VALU, a few cycles) instead of LDS-routed shuffles.
// permlane16_swap(x, x) returns the rows (r0, r0, r2, r2) and (r1, r1, r3,
// r3) (permlane32_swap likewise for the wave halves), so for every lane the
// two results are its own value and its partner's, in some order: the
// sum / max of the two is the pair's.
__device__ __forceinline__ float lane_pair(float x, int dist, bool want_max) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = dist == 16
                     ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                     : __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const float a = __builtin_bit_cast(float, (uint32_t)r[0]);
  const float b = __builtin_bit_cast(float, (uint32_t)r[1]);
  return want_max ? fmaxf(a, b) : a + b;
}

// View of read-only global memory through the constant address space: a
// wave-uniform load through it becomes a scalar (s_load) fetch that waits on
// lgkmcnt, so it never drains the wave's in-flight vector loads. Only for
// buffers that no kernel of the launch writes.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(4))) T*
as_const(const T* p) {
  return (const __attribute__((address_space(4))) T*)p;
}

// Order LDS accesses of one wave: every lane's prior LDS writes are visible
// to every lane's later LDS reads, and the compiler may not move LDS traffic
// across this point.
// ---- LDS access by 32-bit LDS byte address -------------------------------
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

__device__ __forceinline__ bf16x8 lds_ld128(uint32_t addr) {
  return __builtin_bit_cast(bf16x8, *(const lds_u32x4*)(uintptr_t)addr);
}

__device__ __forceinline__ void lds_st128(uint32_t addr, u32x4 v) {
  *(lds_u32x4*)(uintptr_t)addr = v;
}

typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
__device__ __forceinline__ void lds_st64(uint32_t addr, u32x2 v) {
  *(lds_u32x2*)(uintptr_t)addr = v;
}
__device__ __forceinline__ u32x2 lds_ld64(uint32_t addr) {
  return *(const lds_u32x2*)(uintptr_t)addr;
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// i % 4 of the 8-byte chunks addressed by lanes 4j + i / 4 (j = 0..3), i.e.
// a 4 x 16 block of 16-bit values comes back transposed
__device__ __forceinline__ bf16x4 lds_tr16(uint32_t addr) {
  return __builtin_bit_cast(
      bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)addr));
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- error reporting (host) ----------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();
int check_launch(const char* what);
// compute units of the current device (cached per device; 256 if unknown)
int device_cus();

}  // namespace tmopt

#define TMOPT_REQUIRE(cond, code, ...)      \
  do {                                      \
    if (!(cond)) {                          \
      ::tmopt::set_error(__VA_ARGS__);      \
      return (code);                        \
    }                                       \
  } while (0)
