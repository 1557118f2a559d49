// Shared device helpers for the gfx950 attention kernels: bf16 vector types, the CDNA4
// MFMA wrappers, 128-bit global/LDS moves and the 64-lane cross-half exchange.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dadgpt {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// D(32x32 fp32) += A(32x16 bf16) * B(16x32 bf16). Lane l supplies A[l%32][8*(l/32)+e] and
// B[8*(l/32)+e][l%32] for e = 0..7; it receives C[8*(r/4) + 4*(l/32) + r%4][l%32] in
// element r of the result.
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row index (within a 32-row MFMA block) held by element r of lane half `hi`.
__device__ __forceinline__ constexpr int c32_row(int r, int hi) {
  return 8 * (r >> 2) + 4 * hi + (r & 3);
}

// The A-operand row permutation used for score tiles: loading A row m from source row
// sigma(m) (bits 2 and 3 of m swapped) makes output elements 8j..8j+7 of lane half hi hold
// source rows 16j + 8hi + 0..7 — exactly the 8-element K-slice lane half hi supplies as an
// MFMA operand in the next product, so scores feed the next MFMA without any lane exchange.
__device__ __forceinline__ constexpr int sigma32(int m) {
  return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1);
}

__device__ __forceinline__ bf16x8 ld_g128(const bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}
__device__ __forceinline__ u32x4 ld_g128u(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st_g64(bf16* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ u32x4 as_u32x4(bf16x8 v) { return __builtin_bit_cast(u32x4, v); }

// Two fp32 -> packed bf16 pair (round to nearest even; v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 p = {static_cast<bf16>(lo), static_cast<bf16>(hi)};
  return __builtin_bit_cast(uint32_t, p);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Reductions over lanes l and l ^ 32 with v_permlane32_swap (no LDS round trip). With both
// operands x, the swap returns {x[l % 32], x[32 + l % 32]} in every lane, so both lanes of a
// pair compute the same value in the same order.
__device__ __forceinline__ float max_halves(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ bool or_halves(bool x) {
  const uint32_t u = x ? 1u : 0u;
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return (r[0] | r[1]) != 0;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Flips the sign of the 8 bf16 values (exact).
__device__ __forceinline__ bf16x8 neg_bf16x8(bf16x8 x) {
  return as_bf16x8(as_u32x4(x) ^ 0x80008000u);
}

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

}  // namespace dadgpt
