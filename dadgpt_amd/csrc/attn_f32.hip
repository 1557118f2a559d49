// fp32 causal flash attention at fp32 accuracy on gfx950. This is the reference's precision
// (cuda/attention.cu:1): forward with online softmax and a saved natural-log logsumexp, backward
// recomputing the probabilities from it. Every fp32 product runs on the bf16 matrix cores,
// each float split into three bf16 values and each product formed from the six cross terms
// that matter (see X3 below: as accurate as the fp32 MFMA, in 37% of its matrix time, and
// beside the VALU, which the fp32 MFMA of gfx950 does not run beside). The softmax
// exponentials are exp_acc (below: 1.24 ulp in six VALU operations, the library expf 0.85 in
// thirteen) and the logsumexp's logarithm is logf; results match float64 to ~1e-6 (O, lse)
// and the fp32 CPU path within its own rounding. The forward moves its running maximum lazily
// (as the bf16 forward does) and masking runs only where a chunk needs it.
//
// Work decomposition (every product a 32 x 32 MFMA tile, one wave per 32 rows):
//  forward  a wave owns 32 queries (lane l holds query l % 32): S^T = K Q^T over each 32-key
//           chunk with Q in registers (split once), the online softmax per lane, O^T += V^T P^T
//           with P split from the score registers (the K rows are read through sigma32, so
//           score registers 8j..8j+7 of lane half h are the MFMA k-slice of that half: no lane
//           exchange). K and V tiles are split once per workgroup as they are staged, into
//           three bf16 planes each in the bf16 kernels' swizzled layout, read with
//           ds_read_b128 (K rows) and ds_read_b64_tr_b16 (V^T);
//  dK/dV    a wave owns 32 keys (lane l holds key l % 32) and walks every later query chunk:
//           S = Q K^T and dP = dO V^T with K and V in registers (floats, split at each use),
//           Q and dO as bf16 planes, P and dS in registers, dV^T += dO^T P and
//           dK^T += Q^T dS; nothing is shared between waves (no atomics);
//  dQ       a wave owns 32 queries again: S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T, with
//           Q split once, dO split at each use and K, V as bf16 planes;
//  delta    rowsum(dO * O), a separate pass that dK/dV and dQ both read.
// The next tile is loaded into registers while the current one is on the matrix cores and
// split into planes as it is stored: 64 rows in the forward, 32 in dK/dV and dQ, where the
// prefetch registers are needed for the operands.
//
// The DROP instantiations apply attention-probability dropout with the keep bits of
// dropout.hpp: the forward and dQ hold keys along registers (keep_words16), dK/dV holds queries
// along registers (keep_col16).
#include "common.hpp"
#include "dropout.hpp"
#include "kernels.hpp"
#include "lanes.hpp"
#include "tiles.hpp"

namespace dadgpt {
namespace {

constexpr int kWaves = 4;             // waves per workgroup
// Two workgroups per CU, i.e. at most 256 registers a lane (one wave per SIMD runs the backward
// ~15% slower). At D = 64 the forward, dQ and dK/dV fit (dK/dV with its plane addresses from
// LaneLds); the dropout dK/dV spills 19 registers, loop-invariant values reloaded per chunk.
constexpr int kMinBlocks = 2;
constexpr int kRows = 32 * kWaves;    // rows (queries or keys) a workgroup owns
constexpr int kTile = 64;             // rows per staged tile (two 32-row chunks)

// Row (within a 32-row chunk) that score register u of lane half h stands for, when the A
// operand rows were read through sigma32: 16 * (u / 8) + 8 * h + u % 8.
__device__ __forceinline__ constexpr int reg_row(int u, int h) {
  return 16 * (u >> 3) + 8 * h + (u & 7);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// e^x to ~1.3 ulp (measured over [-87, 44] against double exp: 1.24 ulp, the library expf
// 0.85) in six VALU operations instead of the library's thirteen: x log2(e) as a rounded
// product e plus its exact remainder r (an FMA, with log2(e) split into two floats), then
// 2^e on the hardware exp2 and the first-order correction 2^(e+r) = 2^e (1 + r ln 2). Results
// below 2^-126 flush to zero and above 2^128 are +inf (no range reduction): the softmax
// weights these kernels exponentiate are either negligible there or take the rescaling path.
// An infinite x gives NaN (its remainder is inf - inf): callers keep -inf out.
__device__ __forceinline__ float exp_acc(float x) {
  constexpr float kL1 = 1.44269502162933349609375f;  // log2(e) rounded to float
  constexpr float kL2 = 1.925963033500011079e-08f;   // log2(e) - kL1
  const float e = x * kL1;
  const float r = fmaf(x, kL2, fmaf(x, kL1, -e));
  const float p = __builtin_amdgcn_exp2f(e);
  return fmaf(p, r * kLn2, p);
}

// A chunk whose weights reach this in some row moves that row's running maximum: with
// weights below 2^64, the running sums stay far inside fp32 range over any sequence length.
constexpr float kMaxW = 0x1p64f;

// A TR-row fp32 tile (64 rows in the forward, 32 in the backward kernels, whose registers are
// scarcer) and its register prefetch: 256 threads, TR*D/1024 16-byte pieces each; rows at or
// past S read as zeros. Epilogues stage rows at pitch D + 4 floats.
template <int D, int TR = kTile>
struct Tile {
  static constexpr int kPitch = D + 4;
  static constexpr int kPieces = TR * D / 4 / 256;
  f32x4 r[kPieces];

  __device__ __forceinline__ void load(const float* src, int row0, int S) {
#pragma unroll
    for (int i = 0; i < kPieces; ++i) {
      const int u = threadIdx.x + 256 * i, row = u / (D / 4), c = u % (D / 4);
      r[i] = row0 + row < S ? *reinterpret_cast<const f32x4*>(src + (size_t)(row0 + row) * D +
                                                              4 * c)
                            : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  __device__ __forceinline__ void store(float* lds) const {
#pragma unroll
    for (int i = 0; i < kPieces; ++i) {
      const int u = threadIdx.x + 256 * i, row = u / (D / 4), c = u % (D / 4);
      *reinterpret_cast<f32x4*>(lds + row * kPitch + 4 * c) = r[i];
    }
  }
};

// fp32 products on the bf16 matrix cores. A float x is split into three bf16 values
// x = x1 + x2 + x3 (each the round-to-nearest of what the previous ones leave, so the three
// carry 24 significant bits and the rest is below 2^-27 |x|); a product x y is then the six
// cross terms whose weight is at least 2^-18 (x1y1, x1y2, x2y1, x1y3, x3y1, x2y2), each exact
// in fp32 and summed by the MFMA in fp32. Six v_mfma_f32_32x32x16_bf16 (32 cycles each) do
// the work of eight v_mfma_f32_32x32x2_f32 (64 cycles each), and, unlike the fp32 MFMA, they
// run beside the VALU. Measured over random 32x32x64 products: largest error 2.5e-7 of
// sum |x_k y_k|, against 3.5e-7 for the fp32 MFMA.
struct X3 {
  bf16x8 v[3];
};

__device__ __forceinline__ X3 split3(const float (&x)[8]) {
  u32x4 w[3];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a0 = x[2 * i], a1 = x[2 * i + 1];
    const uint32_t p = pack_bf16x2(a0, a1);
    const float b0 = a0 - bf16_lo(p), b1 = a1 - bf16_hi(p);  // exact
    const uint32_t q = pack_bf16x2(b0, b1);
    const float c0 = b0 - bf16_lo(q), c1 = b1 - bf16_hi(q);  // exact
    w[0][i] = p;
    w[1][i] = q;
    w[2][i] = pack_bf16x2(c0, c1);
  }
  return X3{{as_bf16x8(w[0]), as_bf16x8(w[1]), as_bf16x8(w[2])}};
}

// acc += A B over a 16-deep slice, A and B as X3 (smallest terms first).
__device__ __forceinline__ f32x16 mfma_x6(const X3& a, const X3& b, f32x16 acc) {
  acc = mfma32(a.v[1], b.v[1], acc);
  acc = mfma32(a.v[2], b.v[0], acc);
  acc = mfma32(a.v[0], b.v[2], acc);
  acc = mfma32(a.v[1], b.v[0], acc);
  acc = mfma32(a.v[0], b.v[1], acc);
  return mfma32(a.v[0], b.v[0], acc);
}

// A 64-row tile split into three bf16 planes in LDS, each in the row-major swizzled layout of
// the bf16 kernels (tiles.hpp), so the score operands are ds_read_b128 and the transposed
// ones ds_read_b64_tr_b16 reads. Each float is split once per workgroup, when the tile is
// staged, instead of once per wave that reads it.
template <int D, int TR = kTile>
__device__ __forceinline__ void store_x3(const Tile<D, TR>& t, bf16* planes) {
#pragma unroll
  for (int i = 0; i < Tile<D, TR>::kPieces; ++i) {
    const int u = threadIdx.x + 256 * i, row = u / (D / 4), c = u % (D / 4);
    const int off = rm_off<D>(row, c >> 1) + 4 * (c & 1);  // 4 floats: half a 16-byte chunk
    uint32_t w[3][2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float a0 = t.r[i][2 * k], a1 = t.r[i][2 * k + 1];
      const uint32_t p = pack_bf16x2(a0, a1);
      const float b0 = a0 - bf16_lo(p), b1 = a1 - bf16_hi(p);
      const uint32_t q = pack_bf16x2(b0, b1);
      w[0][k] = p;
      w[1][k] = q;
      w[2][k] = pack_bf16x2(b0 - bf16_lo(q), b1 - bf16_hi(q));
    }
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
      *reinterpret_cast<u32x2*>(planes + pl * TR * D + off) = u32x2{w[pl][0], w[pl][1]};
  }
}

// The B operand of a score product from a global row: lane half h supplies columns
// 16 ds + 8 h + 0..7 of `row`, split into three bf16 planes.
template <int D>
__device__ __forceinline__ void load_split_row(X3 (&x)[D / 16], const float* row, int h) {
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds) {
    float a[8];
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(row + 16 * ds + 8 * h);
    const f32x4 v1 = *reinterpret_cast<const f32x4*>(row + 16 * ds + 8 * h + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = v0[e], a[4 + e] = v1[e];
    x[ds] = split3(a);
  }
}

template <int D, int TR = kTile>
__device__ __forceinline__ f32x16 score_tile_p(const bf16* planes, int chunk_row0,
                                               const X3 (&qb)[D / 16], int lane) {
  const int krow = chunk_row0 + sigma32(lane & 31), hi = lane >> 5;
  f32x16 acc = zero16();
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds) {
    X3 a;
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
      a.v[pl] = lds_op(planes + pl * TR * D, rm_off<D>(krow, 2 * ds + hi));
    acc = mfma_x6(a, qb[ds], acc);
  }
  return acc;
}

// A global row in the B-operand layout of the score products, as floats: element 8 ds + e is
// column 16 ds + 8 h + e.
template <int D>
__device__ __forceinline__ void load_row_b(float (&x)[D / 2], const float* row, int h) {
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds) {
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(row + 16 * ds + 8 * h);
    const f32x4 v1 = *reinterpret_cast<const f32x4*>(row + 16 * ds + 8 * h + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[8 * ds + e] = v0[e], x[8 * ds + 4 + e] = v1[e];
  }
}

// score_tile_p with the B operand held as floats (the load_split_row layout) and split at
// each use: for kernels whose registers cannot hold two split rows.
template <int D, int TR = kTile>
__device__ __forceinline__ f32x16 score_tile_pf(const bf16* planes, int chunk_row0,
                                                const float (&bf)[D / 2], int lane) {
  const int krow = chunk_row0 + sigma32(lane & 31), hi = lane >> 5;
  f32x16 acc = zero16();
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds) {
    X3 a;
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
      a.v[pl] = lds_op(planes + pl * TR * D, rm_off<D>(krow, 2 * ds + hi));
    float b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      b[e] = bf[8 * ds + e];
      // split here, at each use: hoisted out of the tile loop, the splits of a whole row would
      // hold 1.5x its registers for the kernel's life
      asm volatile("" : "+v"(b[e]));
    }
    acc = mfma_x6(a, split3(b), acc);
  }
  return acc;
}

template <int D, int TR = kTile>
__device__ __forceinline__ void accumulate_t_p(f32x16 (&acc)[D / 32], const bf16* planes,
                                               int chunk_row0, const f32x16& p, int lane) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = p[8 * j + e];
    const X3 pb = split3(x);
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      X3 a;
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        a.v[pl] = lds_tr_op<D>(planes + pl * TR * D, chunk_row0 + 16 * j, 32 * db, lane);
      acc[db] = mfma_x6(a, pb, acc[db]);
    }
  }
}

// score_tile_pf and accumulate_t_p at chunk row 0 of TR-row planes, with the addresses from
// LaneLds (tiles.hpp): the dK/dV kernel's register relief (no spills at D = 64).
template <int D, int TR>
__device__ __forceinline__ f32x16 score_tile_pfx(const bf16* planes, const float (&bf)[D / 2],
                                                 const LaneLds& lo) {
  uint32_t ra[D / 16];
  row_addr_xor<D>(ra, lo.ro);
  f32x16 acc = zero16();
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds) {
    X3 a;
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) a.v[pl] = lds_row_at(planes + pl * TR * D, ra[ds]);
    float b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      b[e] = bf[8 * ds + e];
      asm volatile("" : "+v"(b[e]));
    }
    acc = mfma_x6(a, split3(b), acc);
  }
  return acc;
}
template <int D, int TR>
__device__ __forceinline__ void accumulate_t_px(f32x16 (&acc)[D / 32], const bf16* planes,
                                                const f32x16& p, const LaneLds& lo) {
  uint32_t ta[2][D / 32];
  tr_addr_xor<D>(ta, lo.tr);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = p[8 * j + e];
    const X3 pb = split3(x);
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      X3 a;
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        a.v[pl] = lds_tr_at(planes + pl * TR * D + 16 * j * D, ta[0][db], ta[1][db]);
      acc[db] = mfma_x6(a, pb, acc[db]);
    }
  }
}

// Writes a wave's transposed accumulators (element r of lane (l32, h), block db: row l32 of
// the wave, column 32 db + c32_row(r, h)) as 32 contiguous rows of D floats through the wave's
// LDS slot `stage` (32 x (D + 4) floats), times `mul` (per lane).
template <int D>
__device__ __forceinline__ void store_rows_t(float* dst, int row0, int S,
                                             const f32x16 (&acc)[D / 32], float mul,
                                             float* stage, int lane) {
  const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      stage[l32 * Tile<D>::kPitch + 32 * db + c32_row(r, h)] = acc[db][r] * mul;
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's own LDS writes are done
  __builtin_amdgcn_wave_barrier();
  constexpr int kPieces = 32 * D / 4 / 64;
#pragma unroll
  for (int i = 0; i < kPieces; ++i) {
    const int u = lane + 64 * i, row = u / (D / 4), c = u % (D / 4);
    if (row0 + row < S)
      *reinterpret_cast<f32x4*>(dst + (size_t)(row0 + row) * D + 4 * c) =
          *reinterpret_cast<const f32x4*>(stage + row * Tile<D>::kPitch + 4 * c);
  }
}

// ------------------------------------------------------------------------------ forward

template <int D, bool DROP>
__global__ __launch_bounds__(64 * kWaves, kMinBlocks) void fwd_f32_kernel(
    float* __restrict__ out, float* __restrict__ lse, const float* __restrict__ q,
    const float* __restrict__ k, const float* __restrict__ v, int S, float scale,
    const DropParams dr) {
  // K and V tiles as three bf16 planes each; after the tile loop the first holds the
  // epilogue's fp32 staging rows
  __shared__ __attribute__((aligned(16))) bf16 skp[3 * kTile * D];
  __shared__ __attribute__((aligned(16))) bf16 svp[3 * kTile * D];
  static_assert(3 * kTile * D * 2 >= 2 * 32 * Tile<D>::kPitch * 4, "epilogue staging fits");
  const int bh = blockIdx.x;
  const int blk = gridDim.y - 1 - blockIdx.y;  // longest query blocks first
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar
  const size_t base = (size_t)bh * S * D;
  const int q0 = blk * kRows + 32 * wave;  // the wave's first query
  const int qi = q0 + l32;                 // this lane's query
  const int last = min(S, (blk + 1) * kRows) - 1;  // the workgroup's last query
  const int n_tiles = last / kTile + 1;

  X3 qb[D / 16];  // the lane's query row, split
  load_split_row<D>(qb, q + base + (size_t)min(qi, S - 1) * D, h);
  f32x16 o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) o[db] = zero16();
  float m = neg_inf(), lh = 0.f;  // running maximum; this lane half's sum of weights

  Tile<D> tk, tv;
  tk.load(k + base, 0, S);
  tv.load(v + base, 0, S);
  for (int t = 0; t < n_tiles; ++t) {
    __syncthreads();  // the previous tile's reads are done
    store_x3<D>(tk, skp);
    store_x3<D>(tv, svp);
    __syncthreads();
    if (t + 1 < n_tiles) {  // next tile in flight during this one
      tk.load(k + base, (t + 1) * kTile, S);
      tv.load(v + base, (t + 1) * kTile, S);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int key0 = t * kTile + 32 * c;
      if (key0 > q0 + 31) continue;  // wave-uniform: the whole chunk is in the future
      f32x16 s = score_tile_p<D>(skp, 32 * c, qb, lane);
      // only the chunk whose first key is the wave's first query holds keys after a query
      // (or past S); waves are 32-query aligned, so it is the one with key0 == q0
      const bool diag = key0 == q0;
      // weights against the running maximum m as it stands (natural-log units)
      float w[16], ps;
      auto weights = [&](float mref) {
#pragma unroll
        for (int u = 0; u < 16; ++u) w[u] = exp_acc(fmaf(s[u], scale, -mref));
        if (diag) {
#pragma unroll
          for (int u = 0; u < 16; ++u)
            if (key0 + reg_row(u, h) > qi) w[u] = 0.f;
        }
        ps = w[0];  // (0 + w[0] could not be folded: it maps -0 to +0)
#pragma unroll
        for (int u = 1; u < 16; ++u) ps += w[u];
      };
      weights(m);
      // The maximum moves only when a row's weights would reach 2^64 (or are inf/NaN: m is
      // -inf before a row's first chunk), compared on the bits (ps is +0, positive or NaN).
      // Both lane halves of a row take the row's decision, and only the rows that need it
      // move: the others rescale by exp(0) = 1 and recompute the same weights, so no row's
      // bits depend on another row.
      const bool need = __float_as_uint(ps) >= __float_as_uint(kMaxW);
      if (__builtin_amdgcn_ballot_w64(need) != 0) {  // wave-uniform
        float cm = neg_inf();
#pragma unroll
        for (int u = 0; u < 16; ++u)
          if (!(diag && key0 + reg_row(u, h) > qi)) cm = fmaxf(cm, s[u] * scale);
        // every row of a chunk the wave computes has a visible key: the row maximum is finite
        const float mn = or_halves(need) ? fmaxf(m, max_halves(cm)) : m;
        // 0 on a row's first chunk (exp_acc has no -inf input path)
        const float alpha = m == neg_inf() ? 0.f : exp_acc(m - mn);
        m = mn;
        lh *= alpha;
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
        weights(m);
      }
      lh += ps;
      KeepWords16 keep = {};
      if constexpr (DROP) keep = keep_words16(dr, (uint64_t)bh * S + qi, key0, h);
#pragma unroll
      for (int u = 0; u < 16; ++u) s[u] = DROP ? w[u] * keep_factor(keep, u, dr) : w[u];
      accumulate_t_p<D>(o, svp, 32 * c, s, lane);
    }
  }
  const float l = sum_halves(lh);
  if (h == 0 && qi < S) lse[(size_t)bh * S + qi] = m + logf(l);
  __syncthreads();  // every wave is done with the tiles: reuse sk as per-wave staging
  float* stage = reinterpret_cast<float*>(wave < 2 ? skp : svp) + (wave & 1) * 32 * Tile<D>::kPitch;
  store_rows_t<D>(out + base, q0, S, o, 1.0f / l, stage, lane);
}

// ----------------------------------------------------------------------------- backward

// delta[row] = sum_d dout[row][d] * out[row][d]: D/4 lanes per row, one 16-byte piece each;
// a grid-stride loop over rows (the lanes of a row share every trip, so the row's shuffles
// always see all of its lanes).
template <int D>
__global__ __launch_bounds__(256) void delta_f32_kernel(float* __restrict__ delta,
                                                        const float* __restrict__ dout,
                                                        const float* __restrict__ out,
                                                        long long rows) {
  constexpr int LPR = D / 4;
  const int c = threadIdx.x % LPR;
  const long long stride = (long long)gridDim.x * (256 / LPR);
  for (long long row = ((long long)blockIdx.x * 256 + threadIdx.x) / LPR; row < rows;
       row += stride) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(dout + row * D + 4 * c);
    const f32x4 b = *reinterpret_cast<const f32x4*>(out + row * D + 4 * c);
    float acc = a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
    acc = lanes::group_sum<LPR>(acc);
    if (c == 0) delta[row] = acc;
  }
}

template <int D, bool DROP>
__global__ __launch_bounds__(64 * kWaves, kMinBlocks) void dkdv_f32_kernel(
    float* __restrict__ dk, float* __restrict__ dv, const float* __restrict__ q,
    const float* __restrict__ k, const float* __restrict__ v, const float* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, int S, float scale,
    const DropParams dr) {
  // Q and dO tiles of TR rows as three bf16 planes each (see the forward); each array also
  // holds two waves' epilogue staging
  constexpr int TR = 32;
  constexpr int kLds = 3 * TR * D > 4 * 32 * Tile<D>::kPitch ? 3 * TR * D
                                                               : 4 * 32 * Tile<D>::kPitch;
  __shared__ __attribute__((aligned(16))) bf16 sqp[kLds];
  __shared__ __attribute__((aligned(16))) bf16 sgp[kLds];
  // per query row of the tile: lse, and delta * scale
  __shared__ __attribute__((aligned(16))) float sl[TR], sd[TR];
  const int bh = blockIdx.x, blk = blockIdx.y;  // early key blocks see the most queries: first
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar
  const size_t base = (size_t)bh * S * D;
  const int k0 = blk * kRows + 32 * wave;  // the wave's first key
  const int kj = k0 + l32;                 // this lane's key
  const int t0 = (blk * kRows) / TR;  // first query tile with a query >= the first key
  const int n_tiles = (S + TR - 1) / TR;

  // the lane's K and V rows (score-product B layout), split at each use
  float kf[D / 2], vf[D / 2];
  load_row_b<D>(kf, k + base + (size_t)min(kj, S - 1) * D, h);
  load_row_b<D>(vf, v + base + (size_t)min(kj, S - 1) * D, h);
  f32x16 dka[D / 32], dva[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) dka[db] = zero16(), dva[db] = zero16();

  static_assert(TR == 32, "one chunk per tile");
  const LaneLds lo = lane_lds<D>(lane);
  Tile<D, TR> tq, tg;
  float pl = 0.f, pd = 0.f;
  auto load_stats = [&](int row0) {
    const int r = row0 + (threadIdx.x & (TR - 1));
    pl = r < S ? lse[(size_t)bh * S + r] : 0.f;
    pd = r < S ? delta[(size_t)bh * S + r] : 0.f;
  };
  tq.load(q + base, t0 * TR, S);
  tg.load(dout + base, t0 * TR, S);
  load_stats(t0 * TR);
  for (int t = t0; t < n_tiles; ++t) {
    __syncthreads();
    store_x3<D, TR>(tq, sqp);
    store_x3<D, TR>(tg, sgp);
    if (threadIdx.x < TR) sl[threadIdx.x] = pl, sd[threadIdx.x] = pd * scale;
    __syncthreads();
    if (t + 1 < n_tiles) {
      tq.load(q + base, (t + 1) * TR, S);
      tg.load(dout + base, (t + 1) * TR, S);
      load_stats((t + 1) * TR);
    }
#pragma unroll
    for (int c = 0; c < TR / 32; ++c) {
      const int qrow0 = t * TR + 32 * c;
      if (qrow0 + 31 < k0) continue;  // wave-uniform: every query of the chunk precedes every key
      // lane (l32, h), register u: query qrow0 + reg_row(u, h), key kj
      f32x16 s = score_tile_pfx<D, TR>(sqp, kf, lo);   // Q K^T
      f32x16 dp = score_tile_pfx<D, TR>(sgp, vf, lo);  // dO V^T
      uint32_t keep = 0;
      if constexpr (DROP) keep = keep_col16(dr, (uint64_t)bh * S + qrow0, k0, lane);
      // Statistics of the chunk's rows 32c + reg_row(u, h): registers 8j..8j+7 are the 8
      // consecutive rows 32c + 16j + 8h .., two 16-byte LDS reads each.
      // keys after a query, or rows past S, only where the chunk reaches the wave's first
      // keys or S (wave-uniform)
      const bool mask = qrow0 < k0 + 31 || qrow0 + 31 >= S;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        // registers 4 g4 .. 4 g4 + 3 are the consecutive rows 32c + 16(g4/2) + 8h + 4(g4%2) ..;
        // their statistics are read here, four at a time, rather than all ahead of the loop
        const int r = 32 * c + 16 * (g4 >> 1) + 8 * h + 4 * (g4 & 1);
        asm volatile("" ::: "memory");
        const f32x4 ls = *reinterpret_cast<const f32x4*>(sl + r);
        const f32x4 ds = *reinterpret_cast<const f32x4*>(sd + r);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int u = 4 * g4 + e;
          const int qrow = qrow0 + reg_row(u, h);
          float p = exp_acc(fmaf(s[u], scale, -ls[e]));
          if (mask && !(kj <= qrow && qrow < S)) p = 0.f;
          float g = dp[u];
          if constexpr (DROP) {
            const float f = keep_factor(keep, u, dr.scale);
            g *= f;
            s[u] = p * f;  // the probability that multiplied V
          } else {
            s[u] = p;
          }
          dp[u] = p * fmaf(g, scale, -ds[e]);  // P (dP - delta) scale
        }
      }
      accumulate_t_px<D, TR>(dva, sgp, s, lo);   // dV^T += dO^T P
      accumulate_t_px<D, TR>(dka, sqp, dp, lo);  // dK^T += Q^T dS
    }
  }
  __syncthreads();
  float* stage = reinterpret_cast<float*>(wave < 2 ? sqp : sgp) + (wave & 1) * 32 * Tile<D>::kPitch;
  store_rows_t<D>(dk + base, k0, S, dka, 1.0f, stage, lane);
  store_rows_t<D>(dv + base, k0, S, dva, 1.0f, stage, lane);  // after the wave's dK reads
}

template <int D, bool DROP>
__global__ __launch_bounds__(64 * kWaves, kMinBlocks) void dq_f32_kernel(
    float* __restrict__ dq, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta, int S, float scale, const DropParams dr) {
  // K and V tiles of TR rows as three bf16 planes each (see the forward); each array also
  // holds two waves' epilogue staging
  constexpr int TR = 32;
  constexpr int kLds = 3 * TR * D > 4 * 32 * Tile<D>::kPitch ? 3 * TR * D
                                                               : 4 * 32 * Tile<D>::kPitch;
  __shared__ __attribute__((aligned(16))) bf16 skp[kLds];
  __shared__ __attribute__((aligned(16))) bf16 svp[kLds];
  const int bh = blockIdx.x;
  const int blk = gridDim.y - 1 - blockIdx.y;  // longest query blocks first
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar
  const size_t base = (size_t)bh * S * D;
  const int q0 = blk * kRows + 32 * wave;
  const int qi = q0 + l32;
  const int qc = min(qi, S - 1);
  const int last = min(S, (blk + 1) * kRows) - 1;
  const int n_tiles = last / TR + 1;

  // the lane's Q row split once, its dO row (columns 16 ds + 8 h + 0..7) split at each use
  X3 qb[D / 16];
  load_split_row<D>(qb, q + base + (size_t)qc * D, h);
  float gf[D / 2];
  load_row_b<D>(gf, dout + base + (size_t)qc * D, h);
  const float my_lse = lse[(size_t)bh * S + qc];
  const float my_dscale = delta[(size_t)bh * S + qc] * scale;
  f32x16 acc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) acc[db] = zero16();

  Tile<D, TR> tk, tv;
  tk.load(k + base, 0, S);
  tv.load(v + base, 0, S);
  for (int t = 0; t < n_tiles; ++t) {
    __syncthreads();
    store_x3<D, TR>(tk, skp);
    store_x3<D, TR>(tv, svp);
    __syncthreads();
    if (t + 1 < n_tiles) {
      tk.load(k + base, (t + 1) * TR, S);
      tv.load(v + base, (t + 1) * TR, S);
    }
#pragma unroll
    for (int c = 0; c < TR / 32; ++c) {
      const int key0 = t * TR + 32 * c;
      if (key0 > q0 + 31) continue;
      // lane (l32, h), register u: query qi, key key0 + reg_row(u, h)
      f32x16 s = score_tile_p<D, TR>(skp, 32 * c, qb, lane);   // K Q^T
      f32x16 dp = score_tile_pf<D, TR>(svp, 32 * c, gf, lane);  // V dO^T
      KeepWords16 keep = {};
      if constexpr (DROP) keep = keep_words16(dr, (uint64_t)bh * S + qi, key0, h);
      // only the chunk whose first key is the wave's first query holds keys after a query (or
      // past S): waves are 32-query aligned
      const bool diag = key0 == q0;
#pragma unroll
      for (int u = 0; u < 16; ++u) s[u] = exp_acc(fmaf(s[u], scale, -my_lse));  // P
      if (diag) {
#pragma unroll
        for (int u = 0; u < 16; ++u)
          if (key0 + reg_row(u, h) > qi) s[u] = 0.f;
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float p = s[u];
        float g = dp[u];
        if constexpr (DROP) g *= keep_factor(keep, u, dr);
        s[u] = p * fmaf(g, scale, -my_dscale);  // P (dP - delta) scale
      }
      accumulate_t_p<D, TR>(acc, skp, 32 * c, s, lane);  // dQ^T += K^T dS^T
    }
  }
  __syncthreads();
  float* stage = reinterpret_cast<float*>(wave < 2 ? skp : svp) + (wave & 1) * 32 * Tile<D>::kPitch;
  store_rows_t<D>(dq + base, q0, S, acc, 1.0f, stage, lane);
}

template <int D>
hipError_t fwd_f32_t(float* out, float* lse, const float* q, const float* k, const float* v,
                     int BH, int S, float scale, hipStream_t stream, const Dropout* drop) {
  const dim3 grid(BH, (S + kRows - 1) / kRows);
  const DropParams dr = drop_params(drop);
  if (drop != nullptr)
    fwd_f32_kernel<D, true><<<grid, 64 * kWaves, 0, stream>>>(out, lse, q, k, v, S, scale, dr);
  else
    fwd_f32_kernel<D, false><<<grid, 64 * kWaves, 0, stream>>>(out, lse, q, k, v, S, scale, dr);
  return hipGetLastError();
}

template <int D>
hipError_t bwd_f32_t(float* dq, float* dk, float* dv, float* delta, const float* dout,
                     const float* out, const float* lse, const float* q, const float* k,
                     const float* v, int BH, int S, float scale, hipStream_t stream,
                     const Dropout* drop) {
  const DropParams dr = drop_params(drop);
  const long long rows = (long long)BH * S;
  const long long blocks = (rows * (D / 4) + 255) / 256;
  delta_f32_kernel<D><<<(unsigned)(blocks < 16384 ? blocks : 16384), 256, 0, stream>>>(
      delta, dout, out, rows);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 grid(BH, (S + kRows - 1) / kRows);
  if (drop != nullptr)
    dkdv_f32_kernel<D, true><<<grid, 64 * kWaves, 0, stream>>>(dk, dv, q, k, v, dout, lse,
                                                               delta, S, scale, dr);
  else
    dkdv_f32_kernel<D, false><<<grid, 64 * kWaves, 0, stream>>>(dk, dv, q, k, v, dout, lse,
                                                                delta, S, scale, dr);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (drop != nullptr)
    dq_f32_kernel<D, true><<<grid, 64 * kWaves, 0, stream>>>(dq, q, k, v, dout, lse, delta, S,
                                                             scale, dr);
  else
    dq_f32_kernel<D, false><<<grid, 64 * kWaves, 0, stream>>>(dq, q, k, v, dout, lse, delta, S,
                                                              scale, dr);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fwd_f32(float* out, float* lse, const float* q, const float* k,
                          const float* v, int BH, int S, int D, float scale,
                          hipStream_t stream, const Dropout* drop) {
  if (D == 64) return fwd_f32_t<64>(out, lse, q, k, v, BH, S, scale, stream, drop);
  if (D == 32) return fwd_f32_t<32>(out, lse, q, k, v, BH, S, scale, stream, drop);
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_f32(float* dq, float* dk, float* dv, float* delta, const float* dout,
                          const float* out, const float* lse, const float* q, const float* k,
                          const float* v, int BH, int S, int D, float scale,
                          hipStream_t stream, const Dropout* drop) {
  if (D == 64)
    return bwd_f32_t<64>(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S, scale, stream,
                         drop);
  if (D == 32)
    return bwd_f32_t<32>(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S, scale, stream,
                         drop);
  return hipErrorInvalidValue;
}

}  // namespace dadgpt
