// Causal flash-attention backward for gfx950: bf16 operands, fp32 accumulation, P recomputed
// from the saved natural-log logsumexp. Covers what cuda/attention.cu:75-205 does in fp32
// (delta, dK/dV, dQ), restructured for MFMA:
//
//   delta kernel   delta[r] = sum_d dO[r,d] * O[r,d]                  (attention.cu:75-85)
//   dQ kernel      query-major; per 64-key tile:  S^T = K Q^T, dP^T = V dO^T,
//                  dS = P (dP - delta), dQ^T += K^T dS^T              (attention.cu:154-205)
//   dK/dV kernel   key-major; per 64-query tile: S = Q K^T, dP = dO V^T,
//                  dV^T += dO^T P, dK^T += Q^T dS                    (attention.cu:87-152)
//
// Both kernels own their outputs outright (no atomics, bitwise repeatable). The score
// tiles use the same sigma32 row permutation as the forward so that P and dS feed the next
// MFMA as B operands from registers; the operands that must be read along the score
// dimension (K^T in the dQ kernel, Q^T and dO^T in the dK/dV kernel) come from transposed
// LDS tiles built during staging.
#include "common.hpp"
#include "kernels.hpp"
#include "tiles.hpp"

namespace dadgpt {
namespace {

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

// ---------------------------------------------------------------- dQ
constexpr int kQWb = 32;  // queries per wave in the dQ kernel

template <int D, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void dq_bf16_kernel(
    bf16* __restrict__ dq, const bf16* __restrict__ q, const bf16* __restrict__ k,
    const bf16* __restrict__ v, const bf16* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta, int S, float scale_log2, float scale) {
  constexpr int NT = 64 * WAVES;
  constexpr int QB = kQWb * WAVES;
  constexpr int DS = D / 16, DB = D / 32;
  __shared__ __attribute__((aligned(16))) bf16 sk[2][kTileRows * D];
  __shared__ __attribute__((aligned(16))) bf16 skt[2][D * kTileRows];
  __shared__ __attribute__((aligned(16))) bf16 sv[2][kTileRows * D];

  const int bh = blockIdx.x;
  const int qblk = gridDim.y - 1 - blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const size_t base = (size_t)bh * S * D;
  const bf16* kg = k + base;
  const bf16* vg = v + base;

  const int q0 = qblk * QB + wave * kQWb;
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

  PairTile<D, NT> kt;
  RowTile<D, NT> vt;
  kt.load(kg, 0, S, tid);
  vt.load(vg, 0, S, tid);
  kt.store_rm(sk[0], tid);
  kt.store_tr(skt[0], tid);
  vt.store_rm(sv[0], tid);
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int st = t & 1;
    const int k0 = t * kTileRows;
    if (t + 1 < n_tiles) {
      kt.load(kg, k0 + kTileRows, S, tid);
      vt.load(vg, k0 + kTileRows, S, tid);
    }
    if (q0 < S && k0 <= q0 + kQWb - 1) {
      f32x16 s[2], dp[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s[kb] = f32x16{};
        dp[kb] = f32x16{};
        const int krow = 32 * kb + sigma32(l32);
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
          s[kb] = mfma32(lds_op(sk[st], rm_off<D>(krow, 2 * ds + hi)), qop[ds], s[kb]);
          dp[kb] = mfma32(lds_op(sv[st], rm_off<D>(krow, 2 * ds + hi)), doop[ds], dp[kb]);
        }
      }
      const bool diag = k0 + kTileRows - 1 > q0;
      bf16x8 dsb[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = fast_exp2(s[kb][r] * scale_log2 - lse2);
          if (diag) {
            const int key = k0 + 32 * kb + 16 * (r >> 3) + 8 * hi + (r & 7);
            if (key > qrow) p = 0.f;
          }
          s[kb][r] = p * (dp[kb][r] - dlt);
        }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f32x16& src = s[ks >> 1];
        const int r0 = (ks & 1) * 8;
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = pack_bf16x2(src[r0 + 2 * e], src[r0 + 2 * e + 1]);
        dsb[ks] = as_bf16x8(w);
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int col = 32 * db + l32;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          dqacc[db] = mfma32(lds_op(skt[st], tr_off(col, 2 * ks + hi)), dsb[ks], dqacc[db]);
      }
    }
    if (t + 1 < n_tiles) {
      kt.store_rm(sk[st ^ 1], tid);
      kt.store_tr(skt[st ^ 1], tid);
      vt.store_rm(sv[st ^ 1], tid);
    }
    __syncthreads();
  }

  if (qrow < S) {
    bf16* orow = dq + base + (size_t)qrow * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * db + c32_row(4 * g, hi);
        u32x2 w;
        w[0] = pack_bf16x2(dqacc[db][4 * g] * scale, dqacc[db][4 * g + 1] * scale);
        w[1] = pack_bf16x2(dqacc[db][4 * g + 2] * scale, dqacc[db][4 * g + 3] * scale);
        st_g64(orow + d0, w);
      }
  }
}

// ---------------------------------------------------------------- dK / dV
constexpr int kKWb = 32;  // keys per wave in the dK/dV kernel

template <int D, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void dkdv_bf16_kernel(
    bf16* __restrict__ dk, bf16* __restrict__ dv, const bf16* __restrict__ q,
    const bf16* __restrict__ k, const bf16* __restrict__ v, const bf16* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, int S, float scale_log2,
    float scale) {
  constexpr int NT = 64 * WAVES;
  constexpr int KB = kKWb * WAVES;
  constexpr int DS = D / 16, DB = D / 32;
  __shared__ __attribute__((aligned(16))) bf16 sq[2][kTileRows * D];
  __shared__ __attribute__((aligned(16))) bf16 sqt[2][D * kTileRows];
  __shared__ __attribute__((aligned(16))) bf16 sdo[2][kTileRows * D];
  __shared__ __attribute__((aligned(16))) bf16 sdot[2][D * kTileRows];
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

  const int kw0 = kblk * KB + wave * kKWb;
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

  PairTile<D, NT> qt, dot;
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
    qt.store_rm(sq[st], tid);
    qt.store_tr(sqt[st], tid);
    dot.store_rm(sdo[st], tid);
    dot.store_tr(sdot[st], tid);
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
      const bool diag = r0 < kw0 + kKWb - 1;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        f32x16 s = f32x16{}, dp = f32x16{};
        const int qr = 32 * qb + sigma32(l32);
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
          s = mfma32(lds_op(sq[st], rm_off<D>(qr, 2 * ds + hi)), kop[ds], s);
          dp = mfma32(lds_op(sdo[st], rm_off<D>(qr, 2 * ds + hi)), vop[ds], dp);
        }
        bf16x8 pb[2], dsb[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          // Registers 8j..8j+7 of lane half hi hold tile queries 32qb + 16j + 8hi + 0..7.
          const int qt0 = 32 * qb + 16 * j + 8 * hi;
          const f32x4 la = *reinterpret_cast<const f32x4*>(&slse[st][qt0]);
          const f32x4 lb = *reinterpret_cast<const f32x4*>(&slse[st][qt0 + 4]);
          const f32x4 da = *reinterpret_cast<const f32x4*>(&sdel[st][qt0]);
          const f32x4 dbv = *reinterpret_cast<const f32x4*>(&sdel[st][qt0 + 4]);
          float p[8], d[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float l2 = e < 4 ? la[e] : lb[e - 4];
            const float de = e < 4 ? da[e] : dbv[e - 4];
            float pe = fast_exp2(s[8 * j + e] * scale_log2 - l2);
            if (diag && key > r0 + qt0 + e) pe = 0.f;
            p[e] = pe;
            d[e] = pe * (dp[8 * j + e] - de);
          }
          u32x4 wp, wd;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            wp[e] = pack_bf16x2(p[2 * e], p[2 * e + 1]);
            wd[e] = pack_bf16x2(d[2 * e], d[2 * e + 1]);
          }
          pb[j] = as_bf16x8(wp);
          dsb[j] = as_bf16x8(wd);
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int col = 32 * db + l32;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int chunk = 4 * qb + 2 * j + hi;  // tile queries 32qb + 16j + 8hi ..
            dvacc[db] = mfma32(lds_op(sdot[st], tr_off(col, chunk)), pb[j], dvacc[db]);
            dkacc[db] = mfma32(lds_op(sqt[st], tr_off(col, chunk)), dsb[j], dkacc[db]);
          }
        }
      }
    }
    if (t + 1 < t_end) store_rows(st ^ 1);
    __syncthreads();
  }

  if (key < S) {
    bf16* krow = dk + base + (size_t)key * D;
    bf16* vrow = dv + base + (size_t)key * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * db + c32_row(4 * g, hi);
        u32x2 wk, wv;
        wk[0] = pack_bf16x2(dkacc[db][4 * g] * scale, dkacc[db][4 * g + 1] * scale);
        wk[1] = pack_bf16x2(dkacc[db][4 * g + 2] * scale, dkacc[db][4 * g + 3] * scale);
        wv[0] = pack_bf16x2(dvacc[db][4 * g], dvacc[db][4 * g + 1]);
        wv[1] = pack_bf16x2(dvacc[db][4 * g + 2], dvacc[db][4 * g + 3]);
        st_g64(krow + d0, wk);
        st_g64(vrow + d0, wv);
      }
  }
}

template <int D, int WAVES>
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
  const float sl2 = scale * kLog2e;
  if (phases & kBwdDq) {
    constexpr int QB = kQWb * WAVES;
    dq_bf16_kernel<D, WAVES><<<dim3(BH, (S + QB - 1) / QB), 64 * WAVES, 0, stream>>>(
        dq, q, k, v, dout, lse, delta, S, sl2, scale);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (phases & kBwdDkdv) {
    constexpr int KB = kKWb * WAVES;
    dkdv_bf16_kernel<D, WAVES><<<dim3(BH, (S + KB - 1) / KB), 64 * WAVES, 0, stream>>>(
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
    return launch_bwd_bf16_t<64, 4>(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S, scale,
                                    stream, phases);
  if (D == 32)
    return launch_bwd_bf16_t<32, 4>(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S, scale,
                                    stream, phases);
  return hipErrorInvalidValue;
}

}  // namespace dadgpt
