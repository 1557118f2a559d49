// Causal flash-attention backward for gfx950: bf16 operands, fp32 accumulation, P recomputed
// from the saved natural-log logsumexp. Covers what cuda/attention.cu:75-205 does in fp32
// (delta, dK/dV, dQ), restructured for MFMA:
//
//   dQ kernel      query-major; per 32-key chunk:  S^T = K Q^T, dP^T = V dO^T,
//                  dQ^T += K^T dS^T                                   (attention.cu:154-205)
//                  and, first, delta[r] = sum_d dO[r,d] * O[r,d] of its rows, written for
//                  the dK/dV kernel                                   (attention.cu:75-85)
//   dK/dV kernel   key-major; per 32-query block:  S = Q K^T, dP = dO V^T,
//                  P = exp(S*scale - lse), dS = P (dP - delta),
//                  dV^T += dO^T P, dK^T += Q^T dS                    (attention.cu:87-152)
//   delta kernel   delta as a pass of its own (profiling and the phase API)
//
// Both MFMA kernels own their outputs outright (no atomics, bitwise repeatable). The score
// tiles use the same sigma32 row permutation as the forward so that P and dS feed the next
// MFMA as B operands from registers; the operands that must be read along the score dimension
// (Q^T and dO^T in the dK/dV kernel, K^T in the dQ kernel) are read across the rows of the
// row-major LDS tiles with ds_read_b64_tr_b16, so every tile is staged once, row-major.
// Masking runs only in the blocks that straddle the diagonal, behind a uniform branch around
// the instructions that zero P. The streamed tiles (Q and dO for dK/dV, K and V for dQ) are
// double-buffered in LDS through direct global->LDS loads, one tile ahead of the compute.
// STRIDED and DROP instantiations as in the forward: per-tensor strides, and dropout with
// the keep bits regenerated (dV from P keep/(1-p), dS = P (dP keep/(1-p) - delta)).
#include "common.hpp"
#include "dropout.hpp"
#include "kernels.hpp"
#include "lanes.hpp"
#include "tiles.hpp"

namespace dadgpt {
namespace {

constexpr int kWaves = 4;
// Workgroups per CU the registers are sized for (4 waves each: 2 -> 256 VGPRs, 3 -> 168).
// dK/dV fits 168 with its LDS addresses derived at use (LaneLds); the dropout one keeps
// 256.
#ifndef DADGPT_DKDV_MINB
#define DADGPT_DKDV_MINB 2
#endif
#ifndef DADGPT_DKDV_MINB_NODROP
#define DADGPT_DKDV_MINB_NODROP 3
#endif
#ifndef DADGPT_DQ_MINB
#define DADGPT_DQ_MINB 3
#endif
constexpr int kDkdvMinBlocks = DADGPT_DKDV_MINB;
constexpr int kDkdvMinBlocksNoDrop = DADGPT_DKDV_MINB_NODROP;
constexpr int kDqMinBlocks = DADGPT_DQ_MINB;

// ---------------------------------------------------------------- delta
template <int D, bool STRIDED>
__global__ __launch_bounds__(256) void delta_bf16_kernel(float* __restrict__ delta,
                                                         const bf16* __restrict__ dout,
                                                         const bf16* __restrict__ out, int S,
                                                         long long rows, int row_blocks,
                                                         const AttnLayout L) {
  // 32 rows per workgroup, 8 lanes per row, 16 bytes each per step. Contiguous: rows of the
  // flat [BH*S, D] matrices (`rows` of them); strided: row_blocks workgroups per (b,h) slice.
  constexpr int LPR = 8;
  const int part = threadIdx.x % LPR;
  const bf16 *dor, *orow;
  long long drow;  // row of delta
  bool valid;
  if constexpr (STRIDED) {
    const int bh = blockIdx.x / row_blocks;
    const int row = (blockIdx.x - bh * row_blocks) * (256 / LPR) + threadIdx.x / LPR;
    const Slice<D, true> sl(L, bh, S);
    dor = sl.row(dout, kTDO, row);
    orow = sl.row(out, kTO, row);
    drow = (long long)bh * S + row;
    valid = row < S;
  } else {
    drow = (long long)blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
    dor = dout + drow * D;
    orow = out + drow * D;
    valid = drow < rows;
  }
  float acc = 0.f;
  if (valid) {
#pragma unroll
    for (int c = part; c < D / 8; c += LPR) {
      const u32x4 a = ld_g128u(dor + c * 8);
      const u32x4 b = ld_g128u(orow + c * 8);
#pragma unroll
      for (int w = 0; w < 4; ++w)
        acc += bf16_lo(a[w]) * bf16_lo(b[w]) + bf16_hi(a[w]) * bf16_hi(b[w]);
    }
  }
  acc = lanes::group_sum<LPR>(acc);
  if (valid && part == 0) delta[drow] = acc;
}

// ---------------------------------------------------------------- dK / dV
constexpr int kKW = 32;  // keys per wave

// One 32-query block (tile rows 32*qb ..) against the wave's 32 keys. Register 8j+e of lane
// half hi holds tile query 32qb + 16j + 8hi + e. The two score products start from
// accumulators that already hold the per-query statistics, read from LDS straight into them:
//   s  = -lse/scale + Q K^T         so P = exp2(c s) with c = scale log2(e)
//   dp = -delta + dO V^T            so P dp = P (dP - delta) = dS
// which leaves two multiplies and an exp2 per score on the VALU. slc holds the tile's
// -lse/scale, sdl its -delta. `mask` zeroes P for keys after the query and for tile rows past
// S (rows_left = S - r0; those rows hold copies of row S-1). It is a runtime flag, not a
// template parameter, and guards only the few instructions that zero P: with two inlined copies
// of the block the compiler gave their MFMAs different accumulator registers and copied all 64
// accumulator values back after every block.
//
// With dropout (DROP; f = keep/(1-p) from bit 8j+e of `keep`): dV accumulates (P f)^T dO and
// dS = P (dP f - delta), so dp starts from zero and -delta is read separately.
// XA: operand addresses from `lo` (LaneLds, tiles.hpp), XORed once per phase, instead of
// computed per read: what brings dK/dV (all but the dropout instantiation) to 168 VGPRs,
// three workgroups per CU, without spilling in the loop.
template <int D, bool DROP, bool XA>
__device__ __forceinline__ void dkdv_block(bool mask, f32x16 (&dkacc)[D / 32],
                                           f32x16 (&dvacc)[D / 32], const bf16x8 (&kop)[D / 16],
                                           const bf16x8 (&vop)[D / 16], const bf16* sq,
                                           const bf16* sdo, const float* slc, const float* sdl,
                                           int qb, int key_minus_r0, int rows_left, int lane,
                                           float c, uint32_t keep, float dscale,
                                           const LaneLds& lo) {
  constexpr int DS = D / 16, DB = D / 32;
  const int l32 = lane & 31, hi = lane >> 5;
  const int qr = 32 * qb + sigma32(l32);
  // Phases: S = stats + Q K^T, dP = stats + dO V^T, softmax, dV += dO^T P, dK += Q^T dS,
  // ordered by the compiler's scheduler (fencing them apart measured 2-3% slower).
  auto stats = [&](const float* row, f32x16& acc) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int qt0 = 32 * qb + 16 * j + 8 * hi;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(row + qt0 + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[8 * j + 4 * h + e] = a[e];
      }
    }
  };
  f32x16 s, dp;
  uint32_t ra[DS] = {};
  if constexpr (XA) row_addr_xor<D>(ra, lo.ro);
  {
    bf16x8 qa[DS];
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
      qa[ds] = XA ? lds_row_at(sq + 32 * qb * D, ra[ds])
                  : lds_op(sq, rm_off<D>(qr, 2 * ds + hi));
    stats(slc, s);
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) s = mfma32(qa[ds], kop[ds], s);
  }
  {
    bf16x8 da[DS];
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
      da[ds] = XA ? lds_row_at(sdo + 32 * qb * D, ra[ds])
                  : lds_op(sdo, rm_off<D>(qr, 2 * ds + hi));
    if constexpr (DROP)
      dp = f32x16{};
    else
      stats(sdl, dp);
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) dp = mfma32(da[ds], vop[ds], dp);
  }
  bf16x8 pb[2], dsb[2];
  f32x16 nd;  // -delta of the block's queries (dropout only)
  if constexpr (DROP) stats(sdl, nd);
  float pr[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) pr[i] = fast_exp2(s[i] * c);
  if (mask) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int qt0 = 32 * qb + 16 * j + 8 * hi;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        pr[8 * j + e] = (key_minus_r0 > qt0 + e || qt0 + e >= rows_left) ? 0.f : pr[8 * j + e];
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    u32x4 wp, wd;
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      float p[2], d[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int e = 2 * e2 + h;
        const float pe = pr[8 * j + e];
        if constexpr (DROP) {
          const float f = keep_factor(keep, 8 * j + e, dscale);
          p[h] = pe * f;
          d[h] = pe * fmaf(dp[8 * j + e], f, nd[8 * j + e]);
        } else {
          p[h] = pe;
          d[h] = pe * dp[8 * j + e];
        }
      }
      wp[e2] = pack_bf16x2(p[0], p[1]);
      wd[e2] = pack_bf16x2(d[0], d[1]);
    }
    pb[j] = as_bf16x8(wp);
    dsb[j] = as_bf16x8(wd);
  }
  uint32_t ta[2][DB] = {};
  if constexpr (XA) tr_addr_xor<D>(ta, lo.tr);
  {
    bf16x8 t[DB][2];  // A = dO^T: lane d = 32db + l32 gets tile queries 32qb + 16j + 8hi + 0..7
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        t[db][j] = XA ? lds_tr_at(sdo + (32 * qb + 16 * j) * D, ta[0][db], ta[1][db])
                      : lds_tr_op<D>(sdo, 32 * qb + 16 * j, 32 * db, lane);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < DB; ++db) dvacc[db] = mfma32(t[db][j], pb[j], dvacc[db]);
  }
  {
    bf16x8 t[DB][2];  // A = Q^T
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        t[db][j] = XA ? lds_tr_at(sq + (32 * qb + 16 * j) * D, ta[0][db], ta[1][db])
                      : lds_tr_op<D>(sq, 32 * qb + 16 * j, 32 * db, lane);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < DB; ++db) dkacc[db] = mfma32(t[db][j], dsb[j], dkacc[db]);
  }
}

template <int D, bool STRIDED, bool DROP>
__global__ __launch_bounds__(64 * kWaves, DROP ? kDkdvMinBlocks : kDkdvMinBlocksNoDrop) void dkdv_bf16_kernel(
    bf16* __restrict__ dk, bf16* __restrict__ dv, const bf16* __restrict__ q,
    const bf16* __restrict__ k, const bf16* __restrict__ v, const bf16* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, int S, float c,
    float lse_mul, float dk_mul, const AttnLayout L, const DropParams dr) {
  constexpr int KB = kKW * kWaves;
  constexpr int DS = D / 16, DB = D / 32;
  // Q and dO tiles, double-buffered (constant buffer indices in the unrolled loop; see the
  // forward kernel), and per wave and buffer the tile's lse and delta rows, converted in place
  // to -lse/scale and -delta: each wave loads and converts its own copy, so the conversion
  // needs no barrier.
  __shared__ __attribute__((aligned(16))) bf16 sq[2][kTileRows * D];
  __shared__ __attribute__((aligned(16))) bf16 sdo[2][kTileRows * D];
  __shared__ __attribute__((aligned(16))) float sst[kWaves][2][2][kTileRows];
  static_assert(kWaves * kKW <= 2 * kTileRows, "the epilogue stages every wave's rows in sq");

  const int bh = blockIdx.x;
  const int kblk = blockIdx.y;  // key block 0 sees the most query tiles: dispatched first
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const Slice<D, STRIDED> sl(L, bh, S);
  const bf16* qg = sl.base(q, kTQ);
  const bf16* dog = sl.base(dout, kTDO);
  const int qp = sl.pitch(kTQ), dop = sl.pitch(kTDO);  // row pitches of the streamed tiles
  const float* lseg = lse + (size_t)bh * S;
  const float* delg = delta + (size_t)bh * S;

  const int kw0 = kblk * KB + wave * kKW;
  const int key = kw0 + l32;
  const int t_first = (kblk * KB) / kTileRows;
  const int t_end = (S - 1) / kTileRows + 1;

  // B operands (K^T, V^T along D): lane holds key row `key`, columns 16*ds + 8*hi + 0..7.
  bf16x8 kop[DS], vop[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    const bool in = key < S;
    kop[ds] = in ? ld_g128(sl.row(k, kTK, key) + 16 * ds + 8 * hi)
                 : as_bf16x8(u32x4{0, 0, 0, 0});
    vop[ds] = in ? ld_g128(sl.row(v, kTV, key) + 16 * ds + 8 * hi)
                 : as_bf16x8(u32x4{0, 0, 0, 0});
  }

  f32x16 dkacc[DB], dvacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dkacc[db] = f32x16{};
    dvacc[db] = f32x16{};
  }
  constexpr bool XA = !DROP;
  LaneLds lo{};
  if constexpr (XA) lo = lane_lds<D>(lane);

  // Direct loads per wave per tile: its share of Q and dO, and its own lse and delta rows.
  using Dma = DmaTile<D, kWaves>;
  uint32_t qoff[Dma::PER_WAVE], dooff[Dma::PER_WAVE];
  Dma::offsets(qoff, wave, lane, qp);
  Dma::offsets(dooff, wave, lane, dop);
  float(*st)[2][kTileRows] = sst[wave];
  auto issue = [&](int t, bf16* nq, bf16* ndo, int buf) {
    Dma::template load_any<true>(nq, qg, t * kTileRows, S, qoff, wave, lane, qp);
    Dma::template load_any<true>(ndo, dog, t * kTileRows, S, dooff, wave, lane, dop);
    dma_row64(st[buf][0], lseg, t * kTileRows, S, lane);
    dma_row64(st[buf][1], delg, t * kTileRows, S, lane);
  };
  // The first tile loads alongside the operands above: one wait covers all of them (the
  // compiler, which does not see the direct loads, then has nothing left to wait for).
  issue(t_first, sq[0], sdo[0], 0);
  wait_vm_lds<0>();
  __builtin_amdgcn_s_barrier();

  // One query tile: prefetch tile t+1 (into the buffers of tile t-1, released by the last
  // barrier), convert this wave's statistics rows, compute tile t, wait for tile t+1 and
  // barrier.
  auto tile = [&](int t, const bf16* cq, const bf16* cdo, int cb, bf16* nq, bf16* ndo,
                  int nb) {
    const int r0 = t * kTileRows;
    if (t + 1 < t_end) issue(t + 1, nq, ndo, nb);
    if (kw0 < S && r0 + kTileRows - 1 >= kw0) {
      // -lse/scale and -delta (this wave's copy; its LDS accesses complete in order)
      st[cb][0][lane] *= lse_mul;
      st[cb][1][lane] = -st[cb][1][lane];
      const bool edge = r0 + kTileRows > S;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int qlo = r0 + 32 * qb;  // first query of the block
        if (qlo + 31 < kw0) continue;   // every key of the wave is after every query
        uint32_t keep = 0;
        if constexpr (DROP) keep = keep_col16(dr, (uint64_t)bh * S + qlo, kw0, lane);
        // some key after some query, or rows past S: mask
        dkdv_block<D, DROP, XA>(edge || qlo < kw0 + kKW - 1, dkacc, dvacc, kop, vop, cq, cdo,
                                st[cb][0], st[cb][1], qb, key - r0, S - r0, lane, c, keep,
                                dr.scale, lo);
      }
    }
    wait_vm_lds<0>();
    __builtin_amdgcn_s_barrier();
  };
  for (int t = t_first; t < t_end; t += 2) {
    tile(t, sq[0], sdo[0], 0, sq[1], sdo[1], 1);
    if (t + 1 < t_end) tile(t + 1, sq[1], sdo[1], 1, sq[0], sdo[0], 0);
  }

  // the tiles are free after the last barrier: each wave stages its 32 rows in its quarter
  // of sq (dK) and sdo (dV)
  if (kw0 < S) {
    store_rows_staged<D>(sl.row(dk, kTDK, kw0), sl.pitch(kTDK), S - kw0, dkacc, dk_mul,
                         &sq[0][0] + wave * kKW * D, lane);
    store_rows_staged<D>(sl.row(dv, kTDV, kw0), sl.pitch(kTDV), S - kw0, dvacc, 1.0f,
                         &sdo[0][0] + wave * kKW * D, lane);
  }
}

// ---------------------------------------------------------------- dQ
constexpr int kQW = 32;  // queries per wave

// One 32-key chunk (tile keys 32*kb ..) against the wave's 32 queries. Register 8j+e of lane
// half hi holds tile key 32kb + 16j + 8hi + e. With dropout (DROP), dS = P (dP * f - delta)
// with f = keep/(1-p) from register 8j+e's uniform in `keep`.
template <int D, bool DROP>
__device__ __forceinline__ void dq_chunk(bool diag, f32x16 (&dqacc)[D / 32],
                                         const bf16x8 (&qop)[D / 16],
                                         const bf16x8 (&doop)[D / 16], const bf16* sk,
                                         const bf16* sv, int kb, int qrow_minus_k0, float lse2,
                                         float dlt, int lane, float scale_log2,
                                         const KeepWords16& keep, const DropParams& dr) {
  constexpr int DS = D / 16, DB = D / 32;
  const int l32 = lane & 31, hi = lane >> 5;
  f32x16 s = f32x16{}, dp = f32x16{};
  const int krow = 32 * kb + sigma32(l32);
  bf16x8 va[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) s = mfma32(lds_op(sk, rm_off<D>(krow, 2 * ds + hi)), qop[ds], s);
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) va[ds] = lds_op(sv, rm_off<D>(krow, 2 * ds + hi));
  __builtin_amdgcn_sched_barrier(0);
  // dP runs on the matrix pipe under the exponentials of S: one dP MFMA, then 16/DS of the
  // wave's exponentials, fenced so the compiler keeps the interleave (left to itself it
  // issued all exponentials first; this order took dQ ~2% faster)
  float pr[16];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    dp = mfma32(va[ds], doop[ds], dp);
#pragma unroll
    for (int i = ds * (16 / DS); i < (ds + 1) * (16 / DS); ++i)
      pr[i] = fast_exp2(fmaf(s[i], scale_log2, -lse2));
    __builtin_amdgcn_sched_barrier(0);
  }
  if (diag) {  // runtime flag around the zeroing only (see dkdv_block)
#pragma unroll
    for (int i = 0; i < 16; ++i)
      pr[i] = 32 * kb + 16 * (i / 8) + 8 * hi + i % 8 > qrow_minus_k0 ? 0.f : pr[i];
  }
  bf16x8 dsb[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    u32x4 w;
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      float d[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int e = 2 * e2 + h;
        const float p = pr[8 * j + e];
        if constexpr (DROP)
          d[h] = p * fmaf(dp[8 * j + e], keep_factor(keep, 8 * j + e, dr), -dlt);
        else
          d[h] = p * (dp[8 * j + e] - dlt);
      }
      w[e2] = pack_bf16x2(d[0], d[1]);
    }
    dsb[j] = as_bf16x8(w);
  }
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int j = 0; j < 2; ++j)  // A = K^T: lane d = 32db + l32 gets keys 32kb + 16j + 8hi ..
      dqacc[db] = mfma32(lds_tr_op<D>(sk, 32 * kb + 16 * j, 32 * db, lane), dsb[j], dqacc[db]);
  }
}

// dQ for one query block per wave; the kernel also computes delta = rowsum(dO * O) of its
// rows (from the dO operands it holds and one load of O) and writes it for the dK/dV kernel,
// so the backward needs no separate delta pass.
template <int D, bool STRIDED, bool DROP>
__global__ __launch_bounds__(64 * kWaves, kDqMinBlocks) void dq_bf16_kernel(
    bf16* __restrict__ dq, float* __restrict__ delta, const bf16* __restrict__ q,
    const bf16* __restrict__ k, const bf16* __restrict__ v, const bf16* __restrict__ dout,
    const bf16* __restrict__ out, const float* __restrict__ lse, int S, float scale_log2,
    float scale, const AttnLayout L, const DropParams dr) {
  constexpr int QB = kQW * kWaves;
  constexpr int DS = D / 16, DB = D / 32;
  // K and V tiles, double-buffered (constant buffer indices; see the forward kernel).
  __shared__ __attribute__((aligned(16))) bf16 sk[2][kTileRows * D];
  __shared__ __attribute__((aligned(16))) bf16 sv[2][kTileRows * D];
  static_assert(kWaves * kQW <= 2 * kTileRows, "the epilogue stages every wave's rows in sk");

  const int bh = blockIdx.x;
  const int qblk = gridDim.y - 1 - blockIdx.y;  // longest (latest) query blocks dispatch first
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const Slice<D, STRIDED> sl(L, bh, S);
  const bf16* kg = sl.base(k, kTK);
  const bf16* vg = sl.base(v, kTV);
  const int kp = sl.pitch(kTK), vp = sl.pitch(kTV);  // row pitches of the streamed tiles

  const int q0 = qblk * QB + wave * kQW;
  const int qrow = q0 + l32;
  const int wg_last = min(S, (qblk + 1) * QB) - 1;
  const int n_tiles = wg_last / kTileRows + 1;

  // lane holds row qrow, columns 16*ds + 8*hi + 0..7 of Q, dO and O (zeros past S)
  bf16x8 qop[DS], doop[DS], oop[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    const bool in = qrow < S;
    const u32x4 z{0, 0, 0, 0};
    qop[ds] = in ? ld_g128(sl.row(q, kTQ, qrow) + 16 * ds + 8 * hi) : as_bf16x8(z);
    doop[ds] = in ? ld_g128(sl.row(dout, kTDO, qrow) + 16 * ds + 8 * hi) : as_bf16x8(z);
    oop[ds] = in ? ld_g128(sl.row(out, kTO, qrow) + 16 * ds + 8 * hi) : as_bf16x8(z);
  }
  // (rows past S read row S-1: a finite value for rows that are never stored)
  float lse_q = lse[(size_t)bh * S + min(qrow, S - 1)];

  f32x16 dqacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dqacc[db] = f32x16{};

  // Keys past S read row S-1; every chunk holding such keys is a diagonal chunk (the key is after
  // every valid query), so they are masked. The first tile loads alongside the operands
  // above, under one wait (see the dK/dV kernel).
  using Dma = DmaTile<D, kWaves>;
  uint32_t koff[Dma::PER_WAVE], voff[Dma::PER_WAVE];
  Dma::offsets(koff, wave, lane, kp);
  Dma::offsets(voff, wave, lane, vp);
  Dma::load_any(sk[0], kg, 0, S, koff, wave, lane, kp);
  Dma::load_any(sv[0], vg, 0, S, voff, wave, lane, vp);
  wait_vm_lds<0>();
  __builtin_amdgcn_s_barrier();
  // Use the loaded values only from here on, so their loads share the wait above.
  asm volatile("" : "+v"(lse_q));
  const float lse2 = lse_q * kLog2e;
  // delta of this lane's row: its 32 columns, then the other lane half's
  float dpart = 0.f;
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    asm volatile("" : "+v"(oop[ds]));
    const u32x4 a = as_u32x4(doop[ds]), o = as_u32x4(oop[ds]);
#pragma unroll
    for (int w = 0; w < 4; ++w)
      dpart += bf16_lo(a[w]) * bf16_lo(o[w]) + bf16_hi(a[w]) * bf16_hi(o[w]);
  }
  const float dlt = sum_halves(dpart);
  if (hi == 0 && qrow < S) delta[(size_t)bh * S + qrow] = dlt;

  auto tile = [&](int t, const bf16* ck, const bf16* cv, bf16* nk, bf16* nv) {
    const int k0 = t * kTileRows;
    if (t + 1 < n_tiles) {
      Dma::load_any(nk, kg, k0 + kTileRows, S, koff, wave, lane, kp);
      Dma::load_any(nv, vg, k0 + kTileRows, S, voff, wave, lane, vp);
    }
    if (q0 < S) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int klo = k0 + 32 * kb;        // first key of the chunk
        if (klo > q0 + kQW - 1) continue;    // every key after every query of the wave
        KeepWords16 keep = {};
        if constexpr (DROP) keep = keep_words16(dr, (uint64_t)bh * S + qrow, klo, hi);
        // some key after some query: mask
        dq_chunk<D, DROP>(klo + 31 > q0, dqacc, qop, doop, ck, cv, kb, qrow - k0, lse2, dlt,
                          lane, scale_log2, keep, dr);
      }
    }
    wait_vm_lds<0>();
    __builtin_amdgcn_s_barrier();
  };
  for (int t = 0; t < n_tiles; t += 2) {
    tile(t, sk[0], sv[0], sk[1], sv[1]);
    if (t + 1 < n_tiles) tile(t + 1, sk[1], sv[1], sk[0], sv[0]);
  }

  if (q0 < S)
    store_rows_staged<D>(sl.row(dq, kTDQ, q0), sl.pitch(kTDQ), S - q0, dqacc, scale,
                         &sk[0][0] + wave * kQW * D, lane);
}

template <int D>
hipError_t launch_bwd_bf16_t(bf16* dq, bf16* dk, bf16* dv, float* delta, const bf16* dout,
                             const bf16* out, const float* lse, const bf16* q, const bf16* k,
                             const bf16* v, int BH, int S, float scale, const AttnLayout& L,
                             hipStream_t stream, int phases, const Dropout* drop) {
  hipError_t e = hipSuccess;
  const bool contiguous = is_contiguous(L, S, D);
  const DropParams dr = drop_params(drop);  // dropout: contiguous layout only (caller checks)
  if (phases & kBwdDelta) {
    const long long rows = (long long)BH * S;
    const int row_blocks = (S + 31) / 32;
    if (contiguous)
      delta_bf16_kernel<D, false><<<(unsigned)((rows + 31) / 32), 256, 0, stream>>>(
          delta, dout, out, S, rows, row_blocks, L);
    else
      delta_bf16_kernel<D, true><<<(unsigned)BH * row_blocks, 256, 0, stream>>>(
          delta, dout, out, S, rows, row_blocks, L);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  // P = exp2(S * scale * log2(e) - lse * log2(e)) holds for either sign of the scale.
  const float sl2 = scale * kLog2e;
  if (phases & kBwdDq) {
    constexpr int QB = kQW * kWaves;
    const dim3 grid(BH, (S + QB - 1) / QB);
    if (drop != nullptr)
      dq_bf16_kernel<D, false, true><<<grid, 64 * kWaves, 0, stream>>>(
          dq, delta, q, k, v, dout, out, lse, S, sl2, scale, L, dr);
    else if (contiguous)
      dq_bf16_kernel<D, false, false><<<grid, 64 * kWaves, 0, stream>>>(
          dq, delta, q, k, v, dout, out, lse, S, sl2, scale, L, dr);
    else
      dq_bf16_kernel<D, true, false><<<grid, 64 * kWaves, 0, stream>>>(
          dq, delta, q, k, v, dout, out, lse, S, sl2, scale, L, dr);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (phases & kBwdDkdv) {
    constexpr int KB = kKW * kWaves;
    // s = S - lse/scale needs a nonzero scale: a zero one (P = exp(-lse)) runs with 1e-30,
    // whose S*scale terms are then below fp32 resolution next to lse/scale.
    const float se = scale != 0.f ? scale : 1e-30f;
    const dim3 grid(BH, (S + KB - 1) / KB);
    if (drop != nullptr)
      dkdv_bf16_kernel<D, false, true><<<grid, 64 * kWaves, 0, stream>>>(
          dk, dv, q, k, v, dout, lse, delta, S, se * kLog2e, -1.0f / se, scale, L, dr);
    else if (contiguous)
      dkdv_bf16_kernel<D, false, false><<<grid, 64 * kWaves, 0, stream>>>(
          dk, dv, q, k, v, dout, lse, delta, S, se * kLog2e, -1.0f / se, scale, L, dr);
    else
      dkdv_bf16_kernel<D, true, false><<<grid, 64 * kWaves, 0, stream>>>(
          dk, dv, q, k, v, dout, lse, delta, S, se * kLog2e, -1.0f / se, scale, L, dr);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return e;
}

}  // namespace

hipError_t launch_bwd_bf16(bf16* dq, bf16* dk, bf16* dv, float* delta, const bf16* dout,
                           const bf16* out, const float* lse, const bf16* q, const bf16* k,
                           const bf16* v, int BH, int S, int D, float scale,
                           const AttnLayout& layout, hipStream_t stream, int phases,
                           const Dropout* drop) {
  if (D == 64)
    return launch_bwd_bf16_t<64>(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S, scale,
                                 layout, stream, phases, drop);
  if (D == 32)
    return launch_bwd_bf16_t<32>(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S, scale,
                                 layout, stream, phases, drop);
  return hipErrorInvalidValue;
}

}  // namespace dadgpt
