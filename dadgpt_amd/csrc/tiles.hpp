// Direct global -> LDS staging of 64-row tiles of an [S, D] bf16 matrix (rows at any pitch),
// and the two ways the MFMA kernels read them back:
//   row operands        one ds_read_b128: 8 consecutive columns of one row (along D)
//   transposed operands two ds_read_b64_tr_b16: 8 consecutive rows of one column (along the
//                       64 tile rows), so the tile never has to be stored transposed
// Tiles are row-major [64][D] in LDS with the 16-byte chunks of each row XOR-swizzled by a
// function of the row. The swizzle was chosen by enumerating the XOR maps of the row bits
// against the exact lane patterns of the three accesses (sigma32-permuted row reads,
// transposed reads, staging writes): with it none of them has a bank conflict, for either a
// 32- or a 64-bank LDS.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace dadgpt {

constexpr int kTileRows = 64;

// Where tensor t's rows of slice bh lie. STRIDED = false is the contiguous [BH, S, D] layout
// with every offset a compile-time multiple of D; STRIDED = true reads the layout (kernels.hpp).
template <int D, bool STRIDED>
struct Slice {
  const AttnLayout& L;
  int bh, S, b, h;
  __device__ __forceinline__ Slice(const AttnLayout& layout, int bh_, int S_)
      : L(layout), bh(bh_), S(S_), b(STRIDED ? bh_ / layout.n_heads : bh_),
        h(STRIDED ? bh_ - b * layout.n_heads : 0) {}
  // row pitch (elements) of tensor t
  __device__ __forceinline__ int pitch(int t) const { return STRIDED ? L.t[t].row : D; }
  // first element of tensor t's slice
  template <typename T>
  __device__ __forceinline__ T* base(T* p, int t) const {
    if constexpr (STRIDED)
      return p + (b * L.t[t].batch + h * L.t[t].head);
    else
      return p + (size_t)bh * S * D;
  }
  // element `row` of tensor t's slice
  template <typename T>
  __device__ __forceinline__ T* row(T* p, int t, int r) const {
    return base(p, t) + (size_t)r * pitch(t);
  }
};

__device__ __forceinline__ constexpr int parity(int x) { return __builtin_popcount(x) & 1; }

// Chunk swizzle of row `row` (D=64: 8 chunks per row, D=32: 4).
template <int D>
__device__ __forceinline__ constexpr int swz(int row) {
  if constexpr (D == 64)
    return parity(row & 2) | (parity(row & 5) << 1) | (parity(row & 10) << 2);
  else
    return parity(row & 6) | (parity(row & 10) << 1);
}

// Element offset of 16-byte chunk `chunk` (8 bf16) of row `row` in a [64][D] tile.
template <int D>
__device__ __forceinline__ int rm_off(int row, int chunk) {
  return row * D + ((chunk ^ swz<D>(row)) << 3);
}

__device__ __forceinline__ bf16x8 lds_op(const bf16* lds, int off) {
  return *reinterpret_cast<const bf16x8*>(lds + off);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) bf16 lds_bf16;

// MFMA operand (A or B of v_mfma_f32_32x32x16_bf16) read across rows of a row-major tile T:
// lane l receives T[row0 + 8*(l/32) + e][col0 + l%32] for e = 0..7, i.e. the operand
// X[idx = l%32][k = 8*(l/32) + e] of X = T^T.
//
// ds_read_b64_tr_b16 works on 16-lane groups: if lane j of a group supplies the address of 4
// consecutive bf16 M_j[0..3], lane i of the group receives M_{4e + i/4}[i % 4] for e = 0..3.
// So lane j points at row row0 + 8*(g/2) + 4*half + (j%16)/4, columns
// col0 + 16*(g%2) + 4*(j%4) .. +3 (g = j/16), once for rows +0..3 (half 0) and once for +4..7.
template <int D>
__device__ __forceinline__ bf16x8 lds_tr_op(const bf16* tile, int row0, int col0, int lane) {
  const int g = lane >> 4;
  const int col = col0 + 16 * (g & 1) + 4 * (lane & 3);
  const lds_bf16* t = (const lds_bf16*)(tile);  // generic -> LDS address space
  s16x4 v[2];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int row = row0 + 8 * (g >> 1) + 4 * half + ((lane >> 2) & 3);
    const int off = row * D + (((col >> 3) ^ swz<D>(row)) << 3) + (col & 7);
    v[half] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + off));
  }
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7));
}

// Per-lane LDS byte offsets, within a [64][D] (or [32][D]) tile, of the two read patterns of
// a 32-row score block, from which every read of a block is one XOR and an immediate offset
// away:
//   row reads (row r0 + sigma32(l32), chunk 2ds + hi)   ro ^ 32ds: the swizzle XORs the chunk
//       index, and 2ds + hi = 2ds ^ hi
//   transposed reads (lds_tr_op at rows r0 + 16j ..., columns 32db ...), half h
//                                                       tr[h] ^ 64db: the column block flips
//       chunk bit 2
// where r0 and 16j, whole groups of 16 rows, leave the swizzle alone and add constants. A
// kernel short of registers keeps these three and issues the XORs once per phase (volatile
// asm: row_addr_xor, tr_addr_xor), where the compiler otherwise hoists every derived address
// out of its tile loop.
struct LaneLds {
  uint32_t ro, tr[2];
};
template <int D>
__device__ __forceinline__ LaneLds lane_lds(int lane) {
  LaneLds o;
  const int l32 = lane & 31, hi = lane >> 5, g = lane >> 4;
  o.ro = 2u * (uint32_t)rm_off<D>(sigma32(l32), hi);
  const int cl = 16 * (g & 1) + 4 * (lane & 3);  // the lane's column within a 32-column block
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rl = 8 * (g >> 1) + 4 * h + ((lane >> 2) & 3);  // its row within 16 rows
    o.tr[h] = 2u * (uint32_t)(rl * D + (((cl >> 3) ^ swz<D>(rl)) << 3) + (cl & 7));
  }
  return o;
}
// Row-read offsets of chunks ds = 0 .. D/16-1.
template <int D>
__device__ __forceinline__ void row_addr_xor(uint32_t (&a)[D / 16], uint32_t ro) {
  a[0] = ro;
  if constexpr (D == 64)
    asm volatile("v_xor_b32 %0, 32, %3\n\tv_xor_b32 %1, 64, %3\n\tv_xor_b32 %2, 0x60, %3"
                 : "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3])
                 : "v"(ro));
  else
    asm volatile("v_xor_b32 %0, 32, %1" : "=&v"(a[1]) : "v"(ro));
}
// Transposed-read offsets [half][db].
template <int D>
__device__ __forceinline__ void tr_addr_xor(uint32_t (&a)[2][D / 32], const uint32_t (&tr)[2]) {
  a[0][0] = tr[0];
  a[1][0] = tr[1];
  if constexpr (D == 64)
    asm volatile("v_xor_b32 %0, 64, %2\n\tv_xor_b32 %1, 64, %3"
                 : "=&v"(a[0][1]), "=&v"(a[1][1])
                 : "v"(tr[0]), "v"(tr[1]));
}
__device__ __forceinline__ bf16x8 lds_row_at(const bf16* base, uint32_t byte_off) {
  return *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(base) + byte_off);
}
// lds_tr_op's read, at byte offsets (within `base`) of its two halves
__device__ __forceinline__ bf16x8 lds_tr_at(const bf16* base, uint32_t off0, uint32_t off1) {
  const lds_bf16* t = (const lds_bf16*)base;
  const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + off0 / 2));
  const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + off1 / 2));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Direct global -> LDS staging (global_load_lds_dwordx4): lane i of a wave-instruction writes
// its 16 bytes to LDS at (M0 + 16*i), so the swizzle is applied on the global side: the lane
// that fills LDS slot (row, physical chunk c) reads logical chunk c ^ swz(row). No registers
// hold the tile and the loads complete asynchronously into LDS, which lets a kernel keep
// tiles in flight across barriers. Rows past S read row S-1 instead (in bounds; the kernels
// mask every key or query past S).
//
// The instruction is issued from inline assembly, so the compiler does not see these loads:
// with the builtin it inserts a wait for every pending direct load before each transposed
// read (ds_read_b64_tr_b16 carries no alias information), which would serialise the
// pipeline. Completion is therefore the caller's job: wait_vm_lds<N>() before the barrier
// that publishes a tile. The compiler's own vector-memory waits stay correct because loads
// complete in order, so unseen younger loads can only lengthen them. M0 is written here and
// used by nothing else in these kernels.
// LDS byte offset of a generic pointer into LDS: the low 32 bits of a flat address in the
// shared aperture are the LDS address (an address-space cast would add a null check).
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)p;
}

// A wave-uniform pointer as the compiler's SGPR value (a no-op for a value already known to
// be uniform; otherwise it reads lane 0).
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// One 16-byte (or 4-byte) piece per lane: a wave-uniform 64-bit base in SGPRs plus a 32-bit
// per-lane byte offset (the instruction's saddr form), so a tile loop moves only the scalar
// base.
__device__ __forceinline__ void dma_lds16_sbase(const void* gbase, uint32_t voff,
                                                const void* lds_dst) {
  const uint32_t lds = lds_offset(lds_dst);
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(base), "v"(voff), "s"(uniform_ptr(gbase))
               : "memory");
}
__device__ __forceinline__ void dma_lds4_sbase(const void* gbase, uint32_t voff,
                                               const void* lds_dst) {
  const uint32_t lds = lds_offset(lds_dst);
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
               :
               : "s"(base), "v"(voff), "s"(uniform_ptr(gbase))
               : "memory");
}

// 64 consecutive fp32 values g[row0 .. row0+63] into LDS, one per lane; rows past S read
// row S-1.
__device__ __forceinline__ void dma_row64(float* lds, const float* g, int row0, int S,
                                          int lane) {
  const int rows_left = S - row0;  // wave-uniform
  const uint32_t off = (uint32_t)(rows_left < 64 ? min(lane, rows_left - 1) : lane) * 4u;
  dma_lds4_sbase(g + row0, off, lds);
}

template <int D, int WAVES>
struct DmaTile {
  static constexpr int C = D / 8;                       // 16-byte chunks per row
  static constexpr int SLOTS = kTileRows * C;           // 16-byte slots per tile
  // wave-instructions per tile and wave; with more waves than instructions the surplus waves
  // stage nothing (and their waits for these loads return at once)
  static constexpr int PER_WAVE = SLOTS >= 64 * WAVES ? SLOTS / (64 * WAVES) : 1;
  static constexpr int ACTIVE = SLOTS / (64 * PER_WAVE);  // waves that stage
  static_assert(SLOTS % (64 * WAVES) == 0 || (64 * WAVES) % SLOTS == 0,
                "whole wave-instructions per tile");

  // Byte offset, from the tile's first row, of the global piece that fills this lane's slot
  // of wave-instruction n (fixed for the whole kernel). Rows are `pitch` elements apart in
  // global memory (D for a contiguous [S, D] matrix; the caller keeps 64 * pitch * 2 bytes
  // within 32 bits).
  __device__ __forceinline__ static void offsets(uint32_t (&off)[PER_WAVE], int wave, int lane,
                                                 int pitch) {
#pragma unroll
    for (int n = 0; n < PER_WAVE; ++n) {
      const int slot = (wave * PER_WAVE + n) * 64 + lane;
      const int row = slot / C;
      off[n] = (uint32_t)(row * pitch + ((slot % C) ^ swz<D>(row)) * 8) * 2u;
    }
  }

  // Tile rows row0 .. row0+63 of g (rows `pitch` elements apart, offsets from offsets() with
  // the same pitch). A tile that crosses S moves the offsets of rows past S back to row S-1
  // (the slot's chunk swizzle is kept; it is the destination's). FRESH_LANE: that correction
  // is computed here from a fresh copy of the lane index, for callers short of registers,
  // where the compiler would otherwise hoist its per-lane products out of the tile loop and
  // spill them (the fresh copy costs the kernels with registers to spare time).
  template <bool FRESH_LANE = false>
  __device__ __forceinline__ static void load_any(bf16* lds_tile, const bf16* g, int row0, int S,
                                                  const uint32_t (&off)[PER_WAVE], int wave,
                                                  int lane, int pitch) {
    if (wave >= ACTIVE) return;
    const int rows_left = S - row0;  // wave-uniform
    const bf16* base = g + (size_t)row0 * pitch;
    int ln = lane;
    if constexpr (FRESH_LANE) asm volatile("" : "+v"(ln));
#pragma unroll
    for (int n = 0; n < PER_WAVE; ++n) {
      uint32_t o = off[n];
      if (rows_left < kTileRows) {
        const int r = (wave * PER_WAVE + n) * (64 / C) + ln / C;
        if (r >= rows_left) o -= (uint32_t)((r - rows_left + 1) * pitch * 2);
      }
      dma_lds16_sbase(base, o, lds_tile + (wave * PER_WAVE + n) * 64 * 8);
    }
  }
};

// Stores a wave's 32 x D result, held in MFMA accumulator layout (lane row l32; element 4g+e
// of acc[db] is column 32db + 8g + 4hi + e), times the lane's `mul`, as bf16 rows dst[r *
// pitch ..] for r < rows_valid. The rows pass through the wave's own `stage` (32 * D bf16 of
// LDS no other wave touches, 16-byte chunks XOR-swizzled by row): written in accumulator
// layout, read back row-contiguous, so every global store instruction writes whole rows
// (64 lanes x 16 bytes) instead of 16-byte pieces of 32 rows.
template <int D>
__device__ __forceinline__ void store_rows_staged(bf16* dst, int pitch, int rows_valid,
                                                  const f32x16 (&acc)[D / 32], float mul,
                                                  bf16* stage, int lane) {
  constexpr int C = D / 8;  // 16-byte chunks per row
  const int l32 = lane & 31, hi = lane >> 5;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int chunk = (32 * db + 8 * g) / 8;
      u32x2 w;
      w[0] = pack_bf16x2(acc[db][4 * g] * mul, acc[db][4 * g + 1] * mul);
      w[1] = pack_bf16x2(acc[db][4 * g + 2] * mul, acc[db][4 * g + 3] * mul);
      *reinterpret_cast<u32x2*>(stage + l32 * D + ((chunk ^ (l32 % C)) << 3) + 4 * hi) = w;
    }
  // the wave's own LDS writes complete before its reads (in order); no barrier needed
#pragma unroll
  for (int it = 0; it < 32 * C / 64; ++it) {
    const int idx = it * 64 + lane, r = idx / C, c = idx % C;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + r * D + ((c ^ (r % C)) << 3));
    // non-temporal: the output is not read again by this kernel, and keeping it out of the
    // L2 leaves room for the streamed tiles other workgroups re-read (forward 2% faster)
    if (r < rows_valid)
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst + (size_t)r * pitch + c * 8));
  }
}

// s_waitcnt: vector-memory count <= N and every LDS operation done (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4 left at its maximum, lgkmcnt 11:8 = 0).
template <int N>
__device__ __forceinline__ void wait_vm_lds() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

}  // namespace dadgpt
