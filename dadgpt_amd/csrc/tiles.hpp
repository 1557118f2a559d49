// Global -> register -> LDS staging of 64-row tiles of a [S, D] bf16 matrix, in two LDS
// layouts:
//   row-major  [64][D]   read as MFMA operands along D (16-byte chunks, XOR-swizzled by row)
//   transposed [D][64]   read as MFMA operands along the 64 rows (keys or queries)
// The transposed layout is built in registers: a thread holds the same 8-column chunk of two
// adjacent rows and interleaves them into 2-row dwords, so each LDS write is 4 bytes and each
// operand read is one 16-byte ds_read.
#pragma once

#include "common.hpp"

namespace dadgpt {

constexpr int kTileRows = 64;

// Element offset of 16-byte chunk `chunk` (8 bf16) of row `row` in a row-major [64][D] tile.
template <int D>
__device__ __forceinline__ int rm_off(int row, int chunk) {
  constexpr int C = D / 8;
  return row * D + ((chunk ^ (row & (C - 1))) << 3);
}

// Element offset of chunk `chunk` (tile rows 8*chunk .. 8*chunk+7) of column `col` in a
// transposed [D][64] tile. The swizzle keeps both the operand reads (32 consecutive columns,
// one chunk) and the staging writes (8 columns x 8 chunks) spread over the LDS banks.
__device__ __forceinline__ int tr_off(int col, int chunk) {
  return col * kTileRows + ((chunk ^ ((col ^ (col >> 3)) & 7)) << 3);
}

__device__ __forceinline__ bf16x8 lds_op(const bf16* lds, int off) {
  return *reinterpret_cast<const bf16x8*>(lds + off);
}

// Tile staged as 16-byte chunks: unit u -> row u / (D/8), chunk u % (D/8). Consecutive
// threads read consecutive 16-byte pieces of a row (fully used 64-byte segments).
template <int D, int NT>
struct RowTile {
  static constexpr int C = D / 8;
  static constexpr int UNITS = kTileRows * C;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  u32x4 a[PER];

  __device__ __forceinline__ void load(const bf16* g, int row0, int S, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      const int row = u / C, ch = u % C;
      a[i] = u32x4{0, 0, 0, 0};
      if (u < UNITS && row0 + row < S) a[i] = ld_g128u(g + (size_t)(row0 + row) * D + ch * 8);
    }
  }
  __device__ __forceinline__ void store_rm(bf16* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      if (u < UNITS) *reinterpret_cast<u32x4*>(lds + rm_off<D>(u / C, u % C)) = a[i];
    }
  }
};

// Tile staged as row pairs: unit u -> rows 2*(u / (D/8)) and +1, chunk u % (D/8). Can be
// stored row-major, transposed, or both from the same registers.
template <int D, int NT>
struct PairTile {
  static constexpr int C = D / 8;
  static constexpr int UNITS = (kTileRows / 2) * C;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  u32x4 a[PER], b[PER];

  __device__ __forceinline__ void load(const bf16* g, int row0, int S, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      const int r = row0 + 2 * (u / C), ch = u % C;
      a[i] = u32x4{0, 0, 0, 0};
      b[i] = u32x4{0, 0, 0, 0};
      if (u < UNITS) {
        if (r < S) a[i] = ld_g128u(g + (size_t)r * D + ch * 8);
        if (r + 1 < S) b[i] = ld_g128u(g + (size_t)(r + 1) * D + ch * 8);
      }
    }
  }
  __device__ __forceinline__ void store_rm(bf16* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      if (u < UNITS) {
        const int p = u / C, ch = u % C;
        *reinterpret_cast<u32x4*>(lds + rm_off<D>(2 * p, ch)) = a[i];
        *reinterpret_cast<u32x4*>(lds + rm_off<D>(2 * p + 1, ch)) = b[i];
      }
    }
  }
  __device__ __forceinline__ void store_tr(bf16* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + i * NT;
      if (u < UNITS) {
        const int p = u / C, ch = u % C;
        const int col0 = ch * 8, chunk = p >> 2, within = 2 * (p & 3);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t x = a[i][w], y = b[i][w];
          const uint32_t even = (x & 0xffffu) | (y << 16);          // column col0 + 2w
          const uint32_t odd = (x >> 16) | (y & 0xffff0000u);       // column col0 + 2w + 1
          *reinterpret_cast<uint32_t*>(lds + tr_off(col0 + 2 * w, chunk) + within) = even;
          *reinterpret_cast<uint32_t*>(lds + tr_off(col0 + 2 * w + 1, chunk) + within) = odd;
        }
      }
    }
  }
};

}  // namespace dadgpt
