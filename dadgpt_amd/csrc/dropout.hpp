// Attention-probability dropout inside the flash kernels: the keep bit of probability
// (row = bh*S + query, key j) is regenerated wherever it is needed (forward, dQ, dK/dV) from a
// counter-based generator, so no mask is stored.
//
// Generator: Philox4x32-10 as published (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC'11). One block gives 8 keys: the keep bit of (row, j) is
// 16-bit half j%2 (low half first) of word (j%8)/2 of the block at counter
// {row lo, row hi, j/8, 0} under key {seed lo, seed hi}, kept iff that 16-bit uniform is
// >= thr = ceil(p * 2^16). Kept probabilities are scaled by 1/(1-p) in fp32, as the
// reference's dropout (cuda/gpu_ops.cu:712-749); its cuRAND stream is not reproduced, so
// masks match this definition, not the reference's.
#pragma once

#include <math.h>

#include "common.hpp"
#include "kernels.hpp"
#include "lanes.hpp"

namespace dadgpt {

// Kernel argument: the key (seed), the keep threshold and the scale of kept values.
struct DropParams {
  uint32_t k0, k1;  // seed lo, hi
  uint32_t thr;     // keep iff the 16-bit uniform >= thr
  float scale;      // 1 / (1 - p)
};

// Kernel arguments of a call (zeros without dropout).
inline DropParams drop_params(const Dropout* d) {
  DropParams r{0u, 0u, 0u, 1.0f};
  if (d != nullptr) {
    r.k0 = (uint32_t)d->seed;
    r.k1 = (uint32_t)(d->seed >> 32);
    r.thr = (uint32_t)ceil((double)d->p * 65536.0);
    r.scale = 1.0f / (1.0f - d->p);
  }
  return r;
}

__device__ __forceinline__ u32x4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2,
                                               uint32_t c3, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {  // key schedule (wave-uniform: scalar registers)
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    // three-input XORs as one v_bitop3_b32 each (truth table 0x96: odd parity), the key from
    // a scalar register; the compiler otherwise issues two v_xor_b32
    c0 = __builtin_amdgcn_bitop3_b32(hi1, c1, k0, 0x96);
    c1 = lo1;
    c2 = __builtin_amdgcn_bitop3_b32(hi0, c3, k1, 0x96);
    c3 = lo0;
  }
  return u32x4{c0, c1, c2, c3};
}

// Keep bits of keys 8*j8 .. 8*j8+7 of `row` (bit e: key 8*j8 + e).
__device__ __forceinline__ uint32_t keep8(const DropParams& dr, uint64_t row, uint32_t j8) {
  const u32x4 w = philox4x32_10((uint32_t)row, (uint32_t)(row >> 32), j8, 0u, dr.k0, dr.k1);
  uint32_t bits = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    bits |= (uint32_t)((w[e] & 0xFFFFu) >= dr.thr) << (2 * e);
    bits |= (uint32_t)((w[e] >> 16) >= dr.thr) << (2 * e + 1);
  }
  return bits;
}

// Keep tests for the score layout with a fixed row per lane and keys along the registers:
// register 8j + e of lane half hi holds key key0 + 16j + 8hi + e (j < 2, e < 8; key0 a
// multiple of 8), i.e. two groups of 8 consecutive keys, one Philox block each. The blocks'
// words are kept as they are: register 8j + e tests 16-bit half e%2 of word e/2 of block j.
// Testing a half where it is used (extract, compare, select: three VALU per register) replaces
// packing it into a bit (about four) and unpacking that again (three).
struct KeepWords16 {
  u32x4 w[2];
};
__device__ __forceinline__ KeepWords16 keep_words16(const DropParams& dr, uint64_t row, int key0,
                                                    int hi) {
  KeepWords16 k;
#pragma unroll
  for (int j = 0; j < 2; ++j)
    k.w[j] = philox4x32_10((uint32_t)row, (uint32_t)(row >> 32),
                           (uint32_t)(key0 + 16 * j + 8 * hi) >> 3, 0u, dr.k0, dr.k1);
  return k;
}

// Bit-matrix transpose across the 8 lanes of a group, for each byte of x (bits 8j .. 8j+7)
// independently: on entry lane t holds row t of an 8x8 bit matrix in each byte (bit k =
// column k), on exit column t (bit e = row e). Butterflies of distance 4, 2, 1: at each, the
// lanes of the lower half keep their low-half columns and take the partner's low-half
// columns into their high half, and the upper lanes the reverse (three lane shuffles).
template <int S>
__device__ __forceinline__ uint32_t transpose8_step(uint32_t x, int t) {
  constexpr uint32_t hi_cols = S == 4 ? 0xF0F0u : S == 2 ? 0xCCCCu : 0xAAAAu;  // column bit S set
  constexpr uint32_t lo_cols = hi_cols ^ 0xFFFFu;
  // partner l ^ S: quad_perm gives it exactly for S = 1, 2 (a VALU op); S = 4 crosses quads
  uint32_t y;
  if constexpr (S == 1)
    y = lanes::dpp_u32<lanes::kQuadXor1>(x);
  else if constexpr (S == 2)
    y = lanes::dpp_u32<lanes::kQuadXor2>(x);
  else
    y = (uint32_t)__shfl_xor((int)x, S, 64);
  return (t & S) ? (x & hi_cols) | ((y & hi_cols) >> S) : (x & lo_cols) | ((y & lo_cols) << S);
}
__device__ __forceinline__ uint32_t transpose8_bits(uint32_t x, int t) {
  return transpose8_step<1>(transpose8_step<2>(transpose8_step<4>(x, t), t), t);
}

// Keep bits for the transposed layout (a fixed key per lane, rows along the registers):
// lane (l32, hi) holds key key0 + l32 (key0 a multiple of 8) and register 8j + e holds row
// row0 + 16j + 8hi + e. The 8 lanes of a group hold 8 consecutive keys, which one Philox
// block per row gives: lane t of the group computes the blocks of rows e = t (j = 0 and 1),
// and a bit transpose across the group hands every lane its own key's bit of all 16 rows.
// Bit 8j + e of the result = register 8j + e.
__device__ __forceinline__ uint32_t keep_col16(const DropParams& dr, uint64_t row0, int key0,
                                               int lane) {
  const int l32 = lane & 31, hi = lane >> 5, t = l32 & 7;
  const uint32_t j8 = (uint32_t)(key0 + (l32 & ~7)) >> 3;
  const uint64_t r = row0 + 8 * hi + t;
  // byte j, bit k: key k of the group in row row0 + 16j + 8hi + t
  const uint32_t m = keep8(dr, r, j8) | (keep8(dr, r + 16, j8) << 8);
  return transpose8_bits(m, t);
}

// The factor of a probability: scale if kept, 0 if dropped.
__device__ __forceinline__ float keep_factor(uint32_t bits, int i, float scale) {
  return (bits >> i) & 1u ? scale : 0.0f;
}
__device__ __forceinline__ float keep_factor(const KeepWords16& k, int r, const DropParams& dr) {
  const uint32_t w = k.w[r >> 3][(r & 7) >> 1];
  return ((r & 1) ? w >> 16 : w & 0xFFFFu) >= dr.thr ? dr.scale : 0.0f;
}

}  // namespace dadgpt
