// fp32 causal flash attention (the reference's precision, cuda/attention.cu:1): forward with
// online softmax and saved natural-log logsumexp, backward recomputing P from it. Accurate
// expf/logf, fp32 FMA; the result matches the fp32 CPU path to ~1e-6. The DROP instantiations
// add attention-probability dropout with the keep bits of dropout.hpp.
//
// gfx950 has no fp32 MFMA rate worth the layout work at this precision's use (tests, greedy
// parity), so these are SIMT kernels: one lane per query row (forward, dQ) or key row
// (dK/dV), 64-row tiles of the other operand staged in LDS and read as broadcast float4.
#include "common.hpp"
#include "dropout.hpp"
#include "kernels.hpp"

namespace dadgpt {
namespace {

constexpr int kT = 64;  // rows per block and per LDS tile

template <int D>
__device__ __forceinline__ void stage_rows_f32(float (*dst)[D], const float* src, int row0,
                                               int S) {
  // 64 threads, 16-byte pieces, consecutive threads on consecutive pieces.
  constexpr int C = D / 4;
  for (int u = threadIdx.x; u < kT * C; u += kT) {
    const int r = u / C, c = u % C;
    f32x4 x = f32x4{0.f, 0.f, 0.f, 0.f};
    if (row0 + r < S) x = *reinterpret_cast<const f32x4*>(src + (size_t)(row0 + r) * D + 4 * c);
    *reinterpret_cast<f32x4*>(&dst[r][4 * c]) = x;
  }
}

template <int D>
__device__ __forceinline__ float dot_row(const float* a, const float (*tile)[D], int j) {
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < D; c += 4) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(&tile[j][c]);
    acc = fmaf(a[c], t[0], acc);
    acc = fmaf(a[c + 1], t[1], acc);
    acc = fmaf(a[c + 2], t[2], acc);
    acc = fmaf(a[c + 3], t[3], acc);
  }
  return acc;
}

template <int D, bool DROP>
__global__ __launch_bounds__(kT) void fwd_f32_kernel(float* __restrict__ out,
                                                     float* __restrict__ lse,
                                                     const float* __restrict__ q,
                                                     const float* __restrict__ k,
                                                     const float* __restrict__ v, int S,
                                                     float scale, const DropParams dr) {
  __shared__ __attribute__((aligned(16))) float sk[kT][D];
  __shared__ __attribute__((aligned(16))) float sv[kT][D];
  const int bh = blockIdx.x;
  const int blk = gridDim.y - 1 - blockIdx.y;
  const int row = blk * kT + threadIdx.x;
  const size_t base = (size_t)bh * S * D;
  const bool valid = row < S;

  float qr[D], o[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    qr[d] = valid ? q[base + (size_t)row * D + d] : 0.f;
    o[d] = 0.f;
  }
  float m = neg_inf(), l = 0.f;
  const int last = min(S, (blk + 1) * kT) - 1;
  for (int k0 = 0; k0 <= last; k0 += kT) {
    __syncthreads();
    stage_rows_f32<D>(sk, k + base, k0, S);
    stage_rows_f32<D>(sv, v + base, k0, S);
    __syncthreads();
    if (!valid) continue;
    const int nj = min(kT, row - k0 + 1);  // keys k0 .. row are visible
    if (nj <= 0) continue;
    uint64_t keep = 0;  // keep bits of keys k0 .. k0+63 of this row
    if constexpr (DROP) {
#pragma unroll 1
      for (int j8 = 0; j8 < nj; j8 += 8)
        keep |= (uint64_t)keep8(dr, (uint64_t)bh * S + row, (uint32_t)(k0 + j8) >> 3) << j8;
    }
    float s[kT];
    float mx = neg_inf();
#pragma unroll
    for (int j = 0; j < kT; ++j) {
      s[j] = j < nj ? dot_row<D>(qr, sk, j) * scale : neg_inf();
      mx = fmaxf(mx, s[j]);
    }
    const float mnew = fmaxf(m, mx);
    const float corr = expf(m - mnew);
    l *= corr;
#pragma unroll
    for (int d = 0; d < D; ++d) o[d] *= corr;
#pragma unroll
    for (int j = 0; j < kT; ++j) {
      if (j < nj) {
        const float p = expf(s[j] - mnew);
        l += p;  // the normaliser of the undropped row
        float pv = p;
        if constexpr (DROP) pv = p * ((keep >> j) & 1u ? dr.scale : 0.0f);
#pragma unroll
        for (int d = 0; d < D; ++d) o[d] = fmaf(pv, sv[j][d], o[d]);
      }
    }
    m = mnew;
  }
  if (valid) {
    const float inv = 1.0f / l;
#pragma unroll
    for (int d = 0; d < D; ++d) out[base + (size_t)row * D + d] = o[d] * inv;
    lse[(size_t)bh * S + row] = m + logf(l);
  }
}

__global__ __launch_bounds__(256) void delta_f32_kernel(float* __restrict__ delta,
                                                        const float* __restrict__ dout,
                                                        const float* __restrict__ out,
                                                        long rows, int D) {
  const long r = (long)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  float acc = 0.f;
  for (int d = 0; d < D; ++d) acc = fmaf(dout[r * D + d], out[r * D + d], acc);
  delta[r] = acc;
}

// One lane per key j: dV_j = sum_{r>=j} P_rj dO_r, dK_j = scale * sum_{r>=j} dS_rj Q_r.
// With dropout: dV_j = sum_r P_rj f_rj dO_r and dS_rj = P_rj (dP_rj f_rj - delta_r), f = keep/(1-p).
template <int D, bool DROP>
__global__ __launch_bounds__(kT) void dkdv_f32_kernel(
    float* __restrict__ dk, float* __restrict__ dv, const float* __restrict__ q,
    const float* __restrict__ k, const float* __restrict__ v, const float* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, int S, float scale,
    const DropParams dr) {
  __shared__ __attribute__((aligned(16))) float sq[kT][D];
  __shared__ __attribute__((aligned(16))) float sdo[kT][D];
  __shared__ float slse[kT], sdel[kT];
  const int bh = blockIdx.x;
  const int blk = blockIdx.y;
  const int key = blk * kT + threadIdx.x;
  const size_t base = (size_t)bh * S * D;
  const bool valid = key < S;
  float kr[D], vr[D], dka[D], dva[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    kr[d] = valid ? k[base + (size_t)key * D + d] : 0.f;
    vr[d] = valid ? v[base + (size_t)key * D + d] : 0.f;
    dka[d] = dva[d] = 0.f;
  }
  for (int r0 = blk * kT; r0 < S; r0 += kT) {
    __syncthreads();
    stage_rows_f32<D>(sq, q + base, r0, S);
    stage_rows_f32<D>(sdo, dout + base, r0, S);
    {
      const int r = r0 + threadIdx.x;
      slse[threadIdx.x] = r < S ? lse[(size_t)bh * S + r] : 0.f;
      sdel[threadIdx.x] = r < S ? delta[(size_t)bh * S + r] : 0.f;
    }
    __syncthreads();
    // keep bits of this lane's key for the tile's 64 rows (every lane, before any exits: the
    // bits of 8 rows come from one Philox block per lane of an 8-lane group, then a transpose)
    uint64_t keep = 0;
    if constexpr (DROP) {
      const int t = threadIdx.x & 7;
      const uint32_t j8 = (uint32_t)(blk * kT + (threadIdx.x & ~7)) >> 3;
#pragma unroll 1
      for (int i8 = 0; i8 < kT; i8 += 8) {
        const uint32_t m = keep8(dr, (uint64_t)bh * S + r0 + i8 + t, j8);  // row i8 + t
        keep |= (uint64_t)transpose8_bits(m, t) << i8;  // bit e: row i8 + e, this lane's key
      }
    }
    if (!valid) continue;
    const int i_begin = max(0, key - r0);
    const int i_end = min(kT, S - r0);
    for (int i = i_begin; i < i_end; ++i) {
      const float s = dot_row<D>(kr, sq, i);
      const float dp = dot_row<D>(vr, sdo, i);
      const float p = expf(s * scale - slse[i]);
      float pv = p, ds;
      if constexpr (DROP) {
        const float f = (keep >> i) & 1u ? dr.scale : 0.0f;
        pv = p * f;
        ds = p * (dp * f - sdel[i]) * scale;
      } else {
        ds = p * (dp - sdel[i]) * scale;
      }
#pragma unroll
      for (int d = 0; d < D; ++d) {
        dva[d] = fmaf(pv, sdo[i][d], dva[d]);
        dka[d] = fmaf(ds, sq[i][d], dka[d]);
      }
    }
  }
  if (valid) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      dk[base + (size_t)key * D + d] = dka[d];
      dv[base + (size_t)key * D + d] = dva[d];
    }
  }
}

// One lane per query r: dQ_r = scale * sum_{j<=r} dS_rj K_j.
template <int D, bool DROP>
__global__ __launch_bounds__(kT) void dq_f32_kernel(
    float* __restrict__ dq, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta, int S, float scale, const DropParams dr) {
  __shared__ __attribute__((aligned(16))) float sk[kT][D];
  __shared__ __attribute__((aligned(16))) float sv[kT][D];
  const int bh = blockIdx.x;
  const int blk = gridDim.y - 1 - blockIdx.y;
  const int row = blk * kT + threadIdx.x;
  const size_t base = (size_t)bh * S * D;
  const bool valid = row < S;
  float qr[D], dor[D], dqa[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    qr[d] = valid ? q[base + (size_t)row * D + d] : 0.f;
    dor[d] = valid ? dout[base + (size_t)row * D + d] : 0.f;
    dqa[d] = 0.f;
  }
  const float rl = valid ? lse[(size_t)bh * S + row] : 0.f;
  const float rd = valid ? delta[(size_t)bh * S + row] : 0.f;
  const int last = min(S, (blk + 1) * kT) - 1;
  for (int k0 = 0; k0 <= last; k0 += kT) {
    __syncthreads();
    stage_rows_f32<D>(sk, k + base, k0, S);
    stage_rows_f32<D>(sv, v + base, k0, S);
    __syncthreads();
    if (!valid) continue;
    const int nj = min(kT, row - k0 + 1);
    uint32_t keep = 0;
    for (int j = 0; j < nj; ++j) {
      const float s = dot_row<D>(qr, sk, j);
      const float dp = dot_row<D>(dor, sv, j);
      const float p = expf(s * scale - rl);
      float ds;
      if constexpr (DROP) {
        if ((j & 7) == 0) keep = keep8(dr, (uint64_t)bh * S + row, (uint32_t)(k0 + j) >> 3);
        ds = p * (dp * keep_factor(keep, j & 7, dr.scale) - rd) * scale;
      } else {
        ds = p * (dp - rd) * scale;
      }
#pragma unroll
      for (int d = 0; d < D; ++d) dqa[d] = fmaf(ds, sk[j][d], dqa[d]);
    }
  }
  if (valid) {
#pragma unroll
    for (int d = 0; d < D; ++d) dq[base + (size_t)row * D + d] = dqa[d];
  }
}

template <int D>
hipError_t fwd_f32_t(float* out, float* lse, const float* q, const float* k, const float* v,
                     int BH, int S, float scale, hipStream_t stream, const Dropout* drop) {
  const dim3 grid(BH, (S + kT - 1) / kT);
  const DropParams dr = drop_params(drop);
  if (drop != nullptr)
    fwd_f32_kernel<D, true><<<grid, kT, 0, stream>>>(out, lse, q, k, v, S, scale, dr);
  else
    fwd_f32_kernel<D, false><<<grid, kT, 0, stream>>>(out, lse, q, k, v, S, scale, dr);
  return hipGetLastError();
}

template <int D>
hipError_t bwd_f32_t(float* dq, float* dk, float* dv, float* delta, const float* dout,
                     const float* out, const float* lse, const float* q, const float* k,
                     const float* v, int BH, int S, float scale, hipStream_t stream,
                     const Dropout* drop) {
  const DropParams dr = drop_params(drop);
  const long rows = (long)BH * S;
  delta_f32_kernel<<<(unsigned)((rows + 255) / 256), 256, 0, stream>>>(delta, dout, out, rows, D);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 grid(BH, (S + kT - 1) / kT);
  if (drop != nullptr)
    dkdv_f32_kernel<D, true><<<grid, kT, 0, stream>>>(dk, dv, q, k, v, dout, lse, delta, S,
                                                      scale, dr);
  else
    dkdv_f32_kernel<D, false><<<grid, kT, 0, stream>>>(dk, dv, q, k, v, dout, lse, delta, S,
                                                       scale, dr);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (drop != nullptr)
    dq_f32_kernel<D, true><<<grid, kT, 0, stream>>>(dq, q, k, v, dout, lse, delta, S, scale, dr);
  else
    dq_f32_kernel<D, false><<<grid, kT, 0, stream>>>(dq, q, k, v, dout, lse, delta, S, scale,
                                                     dr);
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
