// Attention-probability dropout inside the flash kernels: the keep bit of probability
// (row = bh*S + query, key j) is regenerated wherever it is needed (forward, dQ, dK/dV) from a
// counter-based generator, so no mask is stored.
//
// Generator: Philox4x32-10 as published (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC'11). Keep bit of (row, j) = word j%4 of the block at
// counter {row lo, row hi, j/4, 0} under key {seed lo, seed hi}, kept iff (word >> 8) >= thr
// with thr = ceil(p * 2^24) (a 24-bit uniform u >= p). Kept probabilities are scaled by
// 1/(1-p) in fp32, as the reference's dropout (cuda/gpu_ops.cu:712-749); its cuRAND stream is
// not reproduced, so masks match this definition, not the reference's.
#pragma once

#include <math.h>

#include "common.hpp"
#include "kernels.hpp"

namespace dadgpt {

// Kernel argument: the key (seed), the keep threshold and the scale of kept values.
struct DropParams {
  uint32_t k0, k1;  // seed lo, hi
  uint32_t thr;     // keep iff (word >> 8) >= thr
  float scale;      // 1 / (1 - p)
};

// Kernel arguments of a call (zeros without dropout).
inline DropParams drop_params(const Dropout* d) {
  DropParams r{0u, 0u, 0u, 1.0f};
  if (d != nullptr) {
    r.k0 = (uint32_t)d->seed;
    r.k1 = (uint32_t)(d->seed >> 32);
    r.thr = (uint32_t)ceil((double)d->p * 16777216.0);
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
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
  }
  return u32x4{c0, c1, c2, c3};
}

// Keep bits of keys 4*j4 .. 4*j4+3 of `row` (bit e: key 4*j4 + e).
__device__ __forceinline__ uint32_t keep4(const DropParams& dr, uint64_t row, uint32_t j4) {
  const u32x4 w = philox4x32_10((uint32_t)row, (uint32_t)(row >> 32), j4, 0u, dr.k0, dr.k1);
  uint32_t bits = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) bits |= (uint32_t)((w[e] >> 8) >= dr.thr) << e;
  return bits;
}

// Keep bits for the score layout with a fixed row per lane and keys along the registers:
// register 8j + e of lane half hi holds key key0 + 16j + 8hi + e (j < 2, e < 8), i.e. four
// groups of 4 consecutive keys. Bit 8j + e of the result = register 8j + e.
__device__ __forceinline__ uint32_t keep_row16(const DropParams& dr, uint64_t row, int key0,
                                               int hi) {
  uint32_t bits = 0;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int j = g >> 1, u = g & 1;
    const int kb = key0 + 16 * j + 8 * hi + 4 * u;  // a multiple of 4
    bits |= keep4(dr, row, (uint32_t)kb >> 2) << (8 * j + 4 * u);
  }
  return bits;
}

// Keep bits for the transposed layout (a fixed key per lane, rows along the registers):
// lane (l32, hi) holds key key0 + l32 (key0 a multiple of 4) and register 8j + e holds row
// row0 + 16j + 8hi + e. Each group of 4 rows needs the 4 consecutive keys of a lane quad, which
// one Philox block gives: lane t of the quad computes the block of row (group + t), and a
// 4x4 exchange across the quad hands every lane its own key's word of all 4 rows. Bit 8j + e
// of the result = register 8j + e.
__device__ __forceinline__ uint32_t keep_col16(const DropParams& dr, uint64_t row0, int key0,
                                               int lane) {
  const int l32 = lane & 31, hi = lane >> 5, t = l32 & 3;
  const uint32_t j4 = (uint32_t)(key0 + (l32 & ~3)) >> 2;
  uint32_t bits = 0;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int j = g >> 1, u = g & 1;
    const uint64_t row = row0 + 16 * j + 8 * hi + 4 * u + t;
    const u32x4 w = philox4x32_10((uint32_t)row, (uint32_t)(row >> 32), j4, 0u, dr.k0, dr.k1);
    // round d: send word (t ^ d), receive the word of this lane's key (t) of row t ^ d
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int c = t ^ d;
      const uint32_t send = c == 0 ? w[0] : c == 1 ? w[1] : c == 2 ? w[2] : w[3];
      const uint32_t got = d == 0 ? send : (uint32_t)__shfl_xor((int)send, d, 64);
      bits |= (uint32_t)((got >> 8) >= dr.thr) << (8 * j + 4 * u + (t ^ d));
    }
  }
  return bits;
}

// The factor of a probability: scale if kept, 0 if dropped.
__device__ __forceinline__ float keep_factor(uint32_t bits, int i, float scale) {
  return (bits >> i) & 1u ? scale : 0.0f;
}

}  // namespace dadgpt
