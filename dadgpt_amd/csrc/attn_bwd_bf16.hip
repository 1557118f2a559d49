// Causal flash-attention backward for gfx950: bf16 operands, fp32 accumulation, P recomputed
// from the saved natural-log logsumexp. Covers what cuda/attention.cu:75-205 does in fp32
// (delta, dK/dV, dQ), restructured for MFMA:
//
//   delta kernel   delta[r] = sum_d dO[r,d] * O[r,d]                  (attention.cu:75-85)
//   dK/dV kernel   key-major; per 32-query block:  S = Q K^T, dP = dO V^T,
//                  P = exp(S*scale - lse), dS = P (dP - delta),
//                  dV^T += dO^T P, dK^T += Q^T dS                    (attention.cu:87-152)
//   dQ kernel      query-major; per 32-key chunk:  S^T = K Q^T, dP^T = V dO^T,
//                  dQ^T += K^T dS^T                                   (attention.cu:154-205)
//
// Both MFMA kernels own their outputs outright (no atomics, bitwise repeatable). The score
// tiles use the same sigma32 row permutation as the forward so that P and dS feed the next
// MFMA as B operands from registers; the operands that must be read along the score dimension
// (Q^T and dO^T in the dK/dV kernel, K^T in the dQ kernel) are read across the rows of the
// row-major LDS tiles with ds_read_b64_tr_b16, so every tile is staged once, row-major. Masking is compiled only into the blocks that straddle the diagonal
// (template DIAG), so the other blocks run branch-free. Registers stay under 256 per lane
// (launch bound: 2 waves per SIMD) so each SIMD interleaves two waves.
#include "common.hpp"
#include "kernels.hpp"
#include "tiles.hpp"

namespace dadgpt {
namespace {

constexpr int kWaves = 4;

// ---------------------------------------------------------------- delta
template <int D>
__global__ __launch_bounds__(256) void delta_bf16_kernel(float* __restrict__ delta,
                                                         const bf16* __restrict__ dout,
                                                         const bf16* __restrict__ out,
                                                         long rows) {
  // 8 lanes per row, 16 bytes each per step.
  constexpr int LPR = 8;
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  const long row = gid / LPR;
  const int part = (int)(gid % LPR);
  float acc = 0.f;
  if (row < rows) {
#pragma unroll
    for (int c = part; c < D / 8; c += LPR) {
      const u32x4 a = ld_g128u(dout + row * D + c * 8);
      const u32x4 b = ld_g128u(out + row * D + c * 8);
#pragma unroll
      for (int w = 0; w < 4; ++w)
        acc += bf16_lo(a[w]) * bf16_lo(b[w]) + bf16_hi(a[w]) * bf16_hi(b[w]);
    }
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  acc += __shfl_xor(acc, 4, 64);
  if (row < rows && part == 0) delta[row] = acc;
}

// Stores lanes' f32x16 accumulators C[d][row] (lane = row l32, element r = d row
// 32*db + c32_row(r, hi)) as bf16 rows of `dst`, times `mul`.
template <int DB>
__device__ __forceinline__ void store_rows_bf16(bf16* dst, const f32x16 (&acc)[DB], float mul,
                                                int hi) {
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * db + c32_row(4 * g, hi);
      u32x2 w;
      w[0] = pack_bf16x2(acc[db][4 * g] * mul, acc[db][4 * g + 1] * mul);
      w[1] = pack_bf16x2(acc[db][4 * g + 2] * mul, acc[db][4 * g + 3] * mul);
      st_g64(dst + d0, w);
    }
}

// ---------------------------------------------------------------- dK / dV
constexpr int kKW = 32;  // keys per wave

// One 32-query block (tile rows 32*qb ..) against the wave's 32 keys. Register 8j+e of lane
// half hi holds tile query 32qb + 16j + 8hi + e.
template <int D, bool DIAG>
__device__ __forceinline__ void dkdv_block(f32x16 (&dkacc)[D / 32], f32x16 (&dvacc)[D / 32],
                                           const bf16x8 (&kop)[D / 16],
                                           const bf16x8 (&vop)[D / 16], const bf16* sq,
                                           const bf16* sdo, const float* slse,
                                           const float* sdel, int qb, int key_minus_r0,
                                           int lane, float scale_log2) {
  constexpr int DS = D / 16, DB = D / 32;
  const int l32 = lane & 31, hi = lane >> 5;
  f32x16 s = f32x16{}, dp = f32x16{};
  const int qr = 32 * qb + sigma32(l32);
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    s = mfma32(lds_op(sq, rm_off<D>(qr, 2 * ds + hi)), kop[ds], s);
    dp = mfma32(lds_op(sdo, rm_off<D>(qr, 2 * ds + hi)), vop[ds], dp);
  }
  bf16x8 pb[2], dsb[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int qt0 = 32 * qb + 16 * j + 8 * hi;
    const f32x4 la = *reinterpret_cast<const f32x4*>(slse + qt0);
    const f32x4 lb = *reinterpret_cast<const f32x4*>(slse + qt0 + 4);
    const f32x4 da = *reinterpret_cast<const f32x4*>(sdel + qt0);
    const f32x4 dbv = *reinterpret_cast<const f32x4*>(sdel + qt0 + 4);
    u32x4 wp, wd;
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      float p[2], d[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int e = 2 * e2 + h;
        const float l2 = e < 4 ? la[e] : lb[e - 4];
        const float de = e < 4 ? da[e] : dbv[e - 4];
        float pe = fast_exp2(fmaf(s[8 * j + e], scale_log2, -l2));
        // key > query: masked (key - r0 > tile query index)
        if (DIAG) pe = key_minus_r0 > qt0 + e ? 0.f : pe;
        p[h] = pe;
        d[h] = pe * (dp[8 * j + e] - de);
      }
      wp[e2] = pack_bf16x2(p[0], p[1]);
      wd[e2] = pack_bf16x2(d[0], d[1]);
    }
    pb[j] = as_bf16x8(wp);
    dsb[j] = as_bf16x8(wd);
  }
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      // A = dO^T / Q^T: lane d = 32db + l32 gets tile queries 32qb + 16j + 8hi + 0..7
      dvacc[db] = mfma32(lds_tr_op<D>(sdo, 32 * qb + 16 * j, 32 * db, lane), pb[j], dvacc[db]);
      dkacc[db] = mfma32(lds_tr_op<D>(sq, 32 * qb + 16 * j, 32 * db, lane), dsb[j], dkacc[db]);
    }
  }
}

template <int D>
__global__ __launch_bounds__(64 * kWaves, 2) void dkdv_bf16_kernel(
    bf16* __restrict__ dk, bf16* __restrict__ dv, const bf16* __restrict__ q,
    const bf16* __restrict__ k, const bf16* __restrict__ v, const bf16* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, int S, float scale_log2,
    float scale) {
  constexpr int NT = 64 * kWaves;
  constexpr int KB = kKW * kWaves;
  constexpr int DS = D / 16, DB = D / 32;
  __shared__ __attribute__((aligned(16))) bf16 sq[2][kTileRows * D];
  __shared__ __attribute__((aligned(16))) bf16 sdo[2][kTileRows * D];
  __shared__ __attribute__((aligned(16))) float slse[2][kTileRows];
  __shared__ __attribute__((aligned(16))) float sdel[2][kTileRows];

  const int bh = blockIdx.x;
  const int kblk = blockIdx.y;  // key block 0 sees the most query tiles: dispatched first
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const size_t base = (size_t)bh * S * D;
  const bf16* qg = q + base;
  const bf16* dog = dout + base;
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
    kop[ds] = in ? ld_g128(k + base + (size_t)key * D + 16 * ds + 8 * hi)
                 : as_bf16x8(u32x4{0, 0, 0, 0});
    vop[ds] = in ? ld_g128(v + base + (size_t)key * D + 16 * ds + 8 * hi)
                 : as_bf16x8(u32x4{0, 0, 0, 0});
  }

  f32x16 dkacc[DB], dvacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dkacc[db] = f32x16{};
    dvacc[db] = f32x16{};
  }

  RowTile<D, NT> qt, dot;
  float lse_r = 0.f, del_r = 0.f;
  auto load_rows = [&](int row0) {
    qt.load(qg, row0, S, tid);
    dot.load(dog, row0, S, tid);
    if (tid < kTileRows) {
      const int r = row0 + tid;
      // Padded query rows get lse = +inf so their recomputed P is exactly 0.
      lse_r = r < S ? lseg[r] * kLog2e : __builtin_inff();
      del_r = r < S ? delg[r] : 0.f;
    }
  };
  auto store_rows = [&](int st) {
    qt.store(sq[st], tid);
    dot.store(sdo[st], tid);
    if (tid < kTileRows) {
      slse[st][tid] = lse_r;
      sdel[st][tid] = del_r;
    }
  };
  load_rows(t_first * kTileRows);
  store_rows(0);
  __syncthreads();

  for (int t = t_first; t < t_end; ++t) {
    const int st = (t - t_first) & 1;
    const int r0 = t * kTileRows;
    if (t + 1 < t_end) load_rows(r0 + kTileRows);
    if (kw0 < S && r0 + kTileRows - 1 >= kw0) {
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int qlo = r0 + 32 * qb;  // first query of the block
        if (qlo + 31 < kw0) continue;   // every key of the wave is after every query
        if (qlo < kw0 + kKW - 1)        // some key after some query: mask
          dkdv_block<D, true>(dkacc, dvacc, kop, vop, sq[st], sdo[st], slse[st], sdel[st], qb,
                              key - r0, lane, scale_log2);
        else
          dkdv_block<D, false>(dkacc, dvacc, kop, vop, sq[st], sdo[st], slse[st], sdel[st], qb,
                               key - r0, lane, scale_log2);
      }
    }
    if (t + 1 < t_end) store_rows(st ^ 1);
    __syncthreads();
  }

  if (key < S) {
    store_rows_bf16<DB>(dk + base + (size_t)key * D, dkacc, scale, hi);
    store_rows_bf16<DB>(dv + base + (size_t)key * D, dvacc, 1.0f, hi);
  }
}

// ---------------------------------------------------------------- dQ
constexpr int kQW = 32;  // queries per wave

// One 32-key chunk (tile keys 32*kb ..) against the wave's 32 queries. Register 8j+e of lane
// half hi holds tile key 32kb + 16j + 8hi + e.
template <int D, bool DIAG>
__device__ __forceinline__ void dq_chunk(f32x16 (&dqacc)[D / 32], const bf16x8 (&qop)[D / 16],
                                         const bf16x8 (&doop)[D / 16], const bf16* sk,
                                         const bf16* sv, int kb, int qrow_minus_k0, float lse2,
                                         float dlt, int lane, float scale_log2) {
  constexpr int DS = D / 16, DB = D / 32;
  const int l32 = lane & 31, hi = lane >> 5;
  f32x16 s = f32x16{}, dp = f32x16{};
  const int krow = 32 * kb + sigma32(l32);
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    s = mfma32(lds_op(sk, rm_off<D>(krow, 2 * ds + hi)), qop[ds], s);
    dp = mfma32(lds_op(sv, rm_off<D>(krow, 2 * ds + hi)), doop[ds], dp);
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
        float p = fast_exp2(fmaf(s[8 * j + e], scale_log2, -lse2));
        if (DIAG) p = 32 * kb + 16 * j + 8 * hi + e > qrow_minus_k0 ? 0.f : p;
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

template <int D>
__global__ __launch_bounds__(64 * kWaves, 2) void dq_bf16_kernel(
    bf16* __restrict__ dq, const bf16* __restrict__ q, const bf16* __restrict__ k,
    const bf16* __restrict__ v, const bf16* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta, int S, float scale_log2, float scale) {
  constexpr int NT = 64 * kWaves;
  constexpr int QB = kQW * kWaves;
  constexpr int DS = D / 16, DB = D / 32;
  __shared__ __attribute__((aligned(16))) bf16 sk[2][kTileRows * D];
  __shared__ __attribute__((aligned(16))) bf16 sv[2][kTileRows * D];

  const int bh = blockIdx.x;
  const int qblk = gridDim.y - 1 - blockIdx.y;  // longest (latest) query blocks dispatch first
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const size_t base = (size_t)bh * S * D;
  const bf16* kg = k + base;
  const bf16* vg = v + base;

  const int q0 = qblk * QB + wave * kQW;
  const int qrow = q0 + l32;
  const int wg_last = min(S, (qblk + 1) * QB) - 1;
  const int n_tiles = wg_last / kTileRows + 1;

  bf16x8 qop[DS], doop[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    const bool in = qrow < S;
    qop[ds] = in ? ld_g128(q + base + (size_t)qrow * D + 16 * ds + 8 * hi)
                 : as_bf16x8(u32x4{0, 0, 0, 0});
    doop[ds] = in ? ld_g128(dout + base + (size_t)qrow * D + 16 * ds + 8 * hi)
                  : as_bf16x8(u32x4{0, 0, 0, 0});
  }
  const float lse2 = qrow < S ? lse[(size_t)bh * S + qrow] * kLog2e : 0.f;
  const float dlt = qrow < S ? delta[(size_t)bh * S + qrow] : 0.f;

  f32x16 dqacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dqacc[db] = f32x16{};

  RowTile<D, NT> kt, vt;
  kt.load(kg, 0, S, tid);
  vt.load(vg, 0, S, tid);
  kt.store(sk[0], tid);
  vt.store(sv[0], tid);
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int st = t & 1;
    const int k0 = t * kTileRows;
    if (t + 1 < n_tiles) {
      kt.load(kg, k0 + kTileRows, S, tid);
      vt.load(vg, k0 + kTileRows, S, tid);
    }
    if (q0 < S) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int klo = k0 + 32 * kb;        // first key of the chunk
        if (klo > q0 + kQW - 1) continue;    // every key after every query of the wave
        if (klo + 31 > q0)                   // some key after some query: mask
          dq_chunk<D, true>(dqacc, qop, doop, sk[st], sv[st], kb, qrow - k0, lse2, dlt, lane,
                            scale_log2);
        else
          dq_chunk<D, false>(dqacc, qop, doop, sk[st], sv[st], kb, qrow - k0, lse2, dlt, lane,
                             scale_log2);
      }
    }
    if (t + 1 < n_tiles) {
      kt.store(sk[st ^ 1], tid);
      vt.store(sv[st ^ 1], tid);
    }
    __syncthreads();
  }

  if (qrow < S) store_rows_bf16<DB>(dq + base + (size_t)qrow * D, dqacc, scale, hi);
}

template <int D>
hipError_t launch_bwd_bf16_t(bf16* dq, bf16* dk, bf16* dv, float* delta, const bf16* dout,
                             const bf16* out, const float* lse, const bf16* q, const bf16* k,
                             const bf16* v, int BH, int S, float scale, hipStream_t stream,
                             int phases) {
  hipError_t e = hipSuccess;
  if (phases & kBwdDelta) {
    const long rows = (long)BH * S;
    const long threads = rows * 8;
    delta_bf16_kernel<D><<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(delta, dout,
                                                                               out, rows);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  // P = exp2(S * scale * log2(e) - lse * log2(e)) holds for either sign of the scale.
  const float sl2 = scale * kLog2e;
  if (phases & kBwdDq) {
    constexpr int QB = kQW * kWaves;
    dq_bf16_kernel<D><<<dim3(BH, (S + QB - 1) / QB), 64 * kWaves, 0, stream>>>(
        dq, q, k, v, dout, lse, delta, S, sl2, scale);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (phases & kBwdDkdv) {
    constexpr int KB = kKW * kWaves;
    dkdv_bf16_kernel<D><<<dim3(BH, (S + KB - 1) / KB), 64 * kWaves, 0, stream>>>(
        dk, dv, q, k, v, dout, lse, delta, S, sl2, scale);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return e;
}

}  // namespace

hipError_t launch_bwd_bf16(bf16* dq, bf16* dk, bf16* dv, float* delta, const bf16* dout,
                           const bf16* out, const float* lse, const bf16* q, const bf16* k,
                           const bf16* v, int BH, int S, int D, float scale,
                           hipStream_t stream, int phases) {
  if (D == 64)
    return launch_bwd_bf16_t<64>(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S, scale,
                                 stream, phases);
  if (D == 32)
    return launch_bwd_bf16_t<32>(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S, scale,
                                 stream, phases);
  return hipErrorInvalidValue;
}

}  // namespace dadgpt
