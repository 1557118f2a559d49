// Cross-lane reductions on VALU data paths for gfx950: DPP row permutations and
// v_permlane16/32_swap instead of __shfl_xor, which compiles to ds_bpermute_b32 (a round trip
// through the LDS crossbar per step). Used where a reduction sits on a latency-bound path
// (decode attention, the decode-step LayerNorm).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dadgpt {
namespace lanes {

// DPP controls (CDNA encoding): quad_perm selects within each group of 4 lanes; row_mirror and
// row_half_mirror reverse each row of 16 lanes / each half row of 8; row_ror:8 rotates each row
// by 8, which is lane l ^ 8.
constexpr int kQuadXor1 = 0xB1;    // quad_perm [1, 0, 3, 2]
constexpr int kQuadXor2 = 0x4E;    // quad_perm [2, 3, 0, 1]
constexpr int kHalfMirror = 0x141;
constexpr int kMirror = 0x140;
constexpr int kRor8 = 0x128;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}

// The value of lane l ^ 16 and of lane l ^ 32 (v_permlane16_swap / v_permlane32_swap with the
// same register on both sides: each lane keeps its own value in one result and receives its
// partner's in the other).
__device__ __forceinline__ float sum_xor16(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor32(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over each aligned group of N lanes (N a power of two, 2..64); every lane of the group
// ends with the same value. Each step adds the partial sums of two disjoint halves of a
// group twice the size, so its partner need not be lane l ^ k: after the two quad steps every
// lane holds its quad's sum, the half-row mirror pairs quads, the row mirror pairs half rows.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N >= 2 && N <= 64 && (N & (N - 1)) == 0, "power-of-two group");
  x += dpp<kQuadXor1>(x);
  if constexpr (N >= 4) x += dpp<kQuadXor2>(x);
  if constexpr (N >= 8) x += dpp<kHalfMirror>(x);
  if constexpr (N >= 16) x += dpp<kMirror>(x);
  if constexpr (N >= 32) x = sum_xor16(x);
  if constexpr (N >= 64) x = sum_xor32(x);
  return x;
}

// Maximum over each aligned group of N lanes, as group_sum.
template <int N>
__device__ __forceinline__ float group_max(float x) {
  static_assert(N >= 2 && N <= 64 && (N & (N - 1)) == 0, "power-of-two group");
  x = fmaxf(x, dpp<kQuadXor1>(x));
  if constexpr (N >= 4) x = fmaxf(x, dpp<kQuadXor2>(x));
  if constexpr (N >= 8) x = fmaxf(x, dpp<kHalfMirror>(x));
  if constexpr (N >= 16) x = fmaxf(x, dpp<kMirror>(x));
  if constexpr (N >= 32) x = max_xor16(x);
  if constexpr (N >= 64) x = max_xor32(x);
  return x;
}

// Maximum over all 64 lanes of a value that is already uniform within aligned groups of G
// lanes (G = 4, 8, 16 or 32).
template <int G>
__device__ __forceinline__ float wave_max_of_groups(float x) {
  if constexpr (G <= 4) x = fmaxf(x, dpp<kHalfMirror>(x));
  if constexpr (G <= 8) x = fmaxf(x, dpp<kMirror>(x));
  if constexpr (G <= 16) x = max_xor16(x);
  return max_xor32(x);
}

// Sum of x over the lanes l ^ k for k = K0, 2 K0, ..., 32 (K0 = 8, 16 or 32): lanes that agree
// in their low bits below K0 are summed exactly with their partners (the values need not be
// uniform within groups).
template <int K0>
__device__ __forceinline__ float sum_across(float x) {
  static_assert(K0 == 8 || K0 == 16 || K0 == 32, "partners l ^ 8, l ^ 16, l ^ 32");
  if constexpr (K0 <= 8) x += dpp<kRor8>(x);
  if constexpr (K0 <= 16) x = sum_xor16(x);
  return sum_xor32(x);
}

}  // namespace lanes
}  // namespace dadgpt
