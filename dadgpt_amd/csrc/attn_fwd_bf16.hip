// Causal flash-attention forward for gfx950: bf16 Q/K/V/O, fp32 accumulation and softmax,
// fp32 natural-log logsumexp. Replaces the role of flash_fwd_kernel (cuda/attention.cu:17-73)
// at bf16; the fp32 path is attn_f32.hip.
//
// Work decomposition: one workgroup = WAVES waves x 64 queries of one (b,h) slice; it walks
// the 64-key tiles up to its last query (causal tile skipping). Each wave owns 64 queries as
// two 32-query MFMA blocks.
//
// Per 64-key tile and wave, on v_mfma_f32_32x32x16_bf16:
//   S^T[key][query] = K . Q^T   A = K rows from LDS (rows loaded through sigma32), B = Q
//                               held in registers for the whole kernel
//   online softmax in registers: each lane owns one query, so the row max is an in-lane
//                               max3 chain plus one exchange with the other lane half, and the
//                               row sum is kept per lane half until the epilogue
//   O^T[d][query] += V^T . P^T  A = V^T from the transposed LDS tile, B = P straight from the
//                               score registers (bf16), no lane exchange
// K and V^T tiles are double-buffered in LDS: the next tile's global loads are in flight
// while the current tile is on the MFMA pipes; one barrier per tile.
#include "common.hpp"
#include "kernels.hpp"
#include "tiles.hpp"

namespace dadgpt {
namespace {

constexpr int kQW = 64;  // queries per wave

template <int D, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void fwd_bf16_kernel(
    bf16* __restrict__ out, float* __restrict__ lse, const bf16* __restrict__ q,
    const bf16* __restrict__ k, const bf16* __restrict__ v, int S, float scale_log2) {
  constexpr int NT = 64 * WAVES;
  constexpr int QB = kQW * WAVES;
  constexpr int DS = D / 16;  // 16-wide K-steps along D
  constexpr int DB = D / 32;  // 32-row blocks of O^T
  __shared__ __attribute__((aligned(16))) bf16 sk[2][kTileRows * D];
  __shared__ __attribute__((aligned(16))) bf16 svt[2][D * kTileRows];

  const int bh = blockIdx.x;
  const int qblk = gridDim.y - 1 - blockIdx.y;  // longest (latest) query blocks dispatch first
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const size_t base = (size_t)bh * S * D;
  const bf16* qg = q + base;
  const bf16* kg = k + base;
  const bf16* vg = v + base;

  const int q0 = qblk * QB + wave * kQW;
  const int wg_last = min(S, (qblk + 1) * QB) - 1;
  const int n_tiles = wg_last / kTileRows + 1;

  // B operands of S^T: lane holds query q0 + 32i + l32, columns 16*ds + 8*hi + 0..7.
  bf16x8 qop[2][DS];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = q0 + 32 * i + l32;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      qop[i][ds] = row < S ? ld_g128(qg + (size_t)row * D + 16 * ds + 8 * hi)
                           : as_bf16x8(u32x4{0, 0, 0, 0});
    }
  }

  f32x16 oacc[2][DB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[i][db] = f32x16{};
  float mrun[2] = {neg_inf(), neg_inf()};
  float lrun[2] = {0.f, 0.f};

  RowTile<D, NT> kt;
  PairTile<D, NT> vt;
  kt.load(kg, 0, S, tid);
  vt.load(vg, 0, S, tid);
  kt.store_rm(sk[0], tid);
  vt.store_tr(svt[0], tid);
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int st = t & 1;
    const int k0 = t * kTileRows;
    if (t + 1 < n_tiles) {
      kt.load(kg, k0 + kTileRows, S, tid);
      vt.load(vg, k0 + kTileRows, S, tid);
    }
    if (q0 < S && k0 <= q0 + kQW - 1) {
      const bf16* lk = sk[st];
      const bf16* lv = svt[st];
      // ---- S^T = K Q^T for both query blocks; each K operand read once ----
      f32x16 s[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s[0][kb] = f32x16{};
        s[1][kb] = f32x16{};
        const int krow = 32 * kb + sigma32(l32);
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
          const bf16x8 a = lds_op(lk, rm_off<D>(krow, 2 * ds + hi));
          s[0][kb] = mfma32(a, qop[0][ds], s[0][kb]);
          s[1][kb] = mfma32(a, qop[1][ds], s[1][kb]);
        }
      }
      // ---- online softmax (log2 domain), per query = per lane ----
      const bool diag = k0 + kTileRows - 1 > q0;
      bf16x8 pb[2][4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int qrow = q0 + 32 * i + l32;
        float mx = neg_inf();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float x = s[i][kb][r] * scale_log2;
            if (diag) {
              const int key = k0 + 32 * kb + 16 * (r >> 3) + 8 * hi + (r & 7);
              if (key > qrow) x = neg_inf();
            }
            s[i][kb][r] = x;
            mx = fmaxf(mx, x);
          }
        mx = fmaxf(mx, other_half(mx));
        const float mnew = fmaxf(mrun[i], mx);
        const float corr = fast_exp2(mrun[i] - mnew);
        mrun[i] = mnew;
        float ls = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float p = fast_exp2(s[i][kb][r] - mnew);
            s[i][kb][r] = p;
            ls += p;
          }
        lrun[i] = lrun[i] * corr + ls;
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[i][db] *= corr;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const f32x16& src = s[i][ks >> 1];
          const int r0 = (ks & 1) * 8;
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = pack_bf16x2(src[r0 + 2 * e], src[r0 + 2 * e + 1]);
          pb[i][ks] = as_bf16x8(w);
        }
      }
      // ---- O^T += V^T P^T; each V^T operand read once for both query blocks ----
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int col = 32 * db + l32;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 a = lds_op(lv, tr_off(col, 2 * ks + hi));
          oacc[0][db] = mfma32(a, pb[0][ks], oacc[0][db]);
          oacc[1][db] = mfma32(a, pb[1][ks], oacc[1][db]);
        }
      }
    }
    if (t + 1 < n_tiles) {
      kt.store_rm(sk[st ^ 1], tid);
      vt.store_tr(svt[st ^ 1], tid);
    }
    __syncthreads();
  }

  // ---- epilogue: O = O^T / l, lse = ln2 * (m + log2 l) ----
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int qrow = q0 + 32 * i + l32;
    const float l = lrun[i] + other_half(lrun[i]);
    const float inv = 1.0f / l;
    if (qrow < S) {
      bf16* orow = out + base + (size_t)qrow * D;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 32 * db + c32_row(4 * g, hi);
          u32x2 w;
          w[0] = pack_bf16x2(oacc[i][db][4 * g] * inv, oacc[i][db][4 * g + 1] * inv);
          w[1] = pack_bf16x2(oacc[i][db][4 * g + 2] * inv, oacc[i][db][4 * g + 3] * inv);
          st_g64(orow + d0, w);
        }
      if (hi == 0) lse[(size_t)bh * S + qrow] = (mrun[i] + __log2f(l)) * kLn2;
    }
  }
}

template <int D, int WAVES>
hipError_t launch_fwd_bf16_t(bf16* out, float* lse, const bf16* q, const bf16* k, const bf16* v,
                             int BH, int S, float scale, hipStream_t stream) {
  constexpr int QB = kQW * WAVES;
  dim3 grid(BH, (S + QB - 1) / QB);
  fwd_bf16_kernel<D, WAVES><<<grid, 64 * WAVES, 0, stream>>>(out, lse, q, k, v, S,
                                                              scale * kLog2e);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fwd_bf16(bf16* out, float* lse, const bf16* q, const bf16* k, const bf16* v,
                           int BH, int S, int D, float scale, hipStream_t stream) {
  if (D == 64) return launch_fwd_bf16_t<64, 4>(out, lse, q, k, v, BH, S, scale, stream);
  if (D == 32) return launch_fwd_bf16_t<32, 2>(out, lse, q, k, v, BH, S, scale, stream);
  return hipErrorInvalidValue;
}

}  // namespace dadgpt
