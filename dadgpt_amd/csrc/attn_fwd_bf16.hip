// Causal flash-attention forward for gfx950: bf16 Q/K/V/O, fp32 accumulation and softmax,
// fp32 natural-log logsumexp. Replaces the role of flash_fwd_kernel (cuda/attention.cu:17-73)
// at bf16; the fp32 path is attn_f32.hip.
//
// Work decomposition: one workgroup = WAVES waves x NQB*32 queries of one (b,h) slice; it
// walks the 64-key tiles up to its last query (causal tile skipping). Each wave owns NQB
// 32-query MFMA blocks and handles each key tile as two 32-key chunks. Per chunk and wave, on
// v_mfma_f32_32x32x16_bf16:
//   S^T[key][query] = K . Q^T   A = K rows from LDS (rows loaded through sigma32), B = Q held
//                               in registers for the whole kernel; one K operand read feeds
//                               every query block of the wave
//   online softmax in registers: each lane owns one query, so the row max is an in-lane max3
//                               chain plus one exchange with the other lane half
//   O^T[d][query] += V^T . P^T  A = V^T read across the rows of the row-major V tile with
//                               ds_read_b64_tr_b16, B = P straight from the score registers
//                               (bf16), no lane exchange
//
// VALU per score, the forward's other bound at d_head 64: the scale is folded into the
// exponent (one FMA: exp2(s*c - m)), the max takes half a v_max3 per score, the bf16 pack
// half a v_cvt_pk, and the row sum one fp32 add (in fp32, before the bf16 rounding, so the
// saved logsumexp keeps fp32 accuracy). Rescaling is lazy: the running max m only moves when
// a row's new maximum exceeds it by more than kRescale (log2 units), so the O accumulators are rescaled
// on a few chunks per row instead of every chunk; P stays below 2^kRescale, and O and l carry
// the same factor, which the epilogue's division removes.
//
// The launch bound caps registers so that several waves share each SIMD, which interleaves
// one wave's softmax with another's MFMAs and covers LDS latency. K and V tiles are
// triple-buffered in LDS and staged by direct global->LDS loads (no registers, no LDS-store
// instructions): tiles t+1 and t+2 are in flight while tile t is on the MFMA pipes; one
// barrier per tile.
#include "common.hpp"
#include "kernels.hpp"
#include "tiles.hpp"

namespace dadgpt {
namespace {

// Geometry: NQB 32-query blocks per wave, WAVES waves per workgroup, MINB workgroups per CU
// (the register budget: 512 / (MINB * WAVES / 4) per lane). One wave with one query block and
// 8 waves per workgroup keeps 4 waves on each SIMD to cover LDS and MFMA latencies; two query
// blocks per wave halve the LDS reads per MFMA instead.
#ifndef DADGPT_FWD_NQB
#define DADGPT_FWD_NQB 1
#endif
#ifndef DADGPT_FWD_WAVES
#define DADGPT_FWD_WAVES 4
#endif
#ifndef DADGPT_FWD_MINB
#define DADGPT_FWD_MINB 3
#endif
constexpr int kNQB = DADGPT_FWD_NQB;
constexpr int kQW = 32 * kNQB;            // queries per wave
constexpr int kWaves = DADGPT_FWD_WAVES;  // waves per workgroup
constexpr int kMinBlocks = DADGPT_FWD_MINB;
constexpr float kRescale = 8.0f;          // lazy-rescale threshold, log2 units

// K operands of one 32-key chunk (tile keys 32*kb ..): A operands of S^T = K Q^T, K rows read
// through sigma32 so that register r of lane half hi holds key 32kb + 16*(r>>3) + 8*hi + (r&7).
template <int D>
__device__ __forceinline__ void fwd_k_ops(bf16x8 (&ka)[D / 16], const bf16* lk, int kb,
                                          int lane) {
  const int l32 = lane & 31, hi = lane >> 5;
  const int krow = 32 * kb + sigma32(l32);
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds) ka[ds] = lds_op(lk, rm_off<D>(krow, 2 * ds + hi));
}

// s[i] = K[chunk] Q_i^T for the wave's NQB query blocks; each K operand feeds every block.
template <int D, int NQB>
__device__ __forceinline__ void fwd_scores(f32x16 (&s)[NQB], const bf16x8 (&qop)[NQB][D / 16],
                                           const bf16x8 (&ka)[D / 16]) {
#pragma unroll
  for (int i = 0; i < NQB; ++i) s[i] = f32x16{};
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds)
#pragma unroll
    for (int i = 0; i < NQB; ++i) s[i] = mfma32(ka[ds], qop[i][ds], s[i]);
}

// V^T operands of one chunk (A of O^T += V^T P^T), read across the rows of the V tile.
template <int D>
__device__ __forceinline__ void fwd_v_ops(bf16x8 (&va)[D / 32][2], const bf16* lv, int kb,
                                          int lane) {
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 2; ++j) va[db][j] = lds_tr_op<D>(lv, 32 * kb + 16 * j, 32 * db, lane);
}

// Online softmax of one chunk's scores and O^T += V^T[:, chunk] P^T. DIAG chunks mask keys
// after the query.
template <int D, int NQB, bool DIAG>
__device__ __forceinline__ void fwd_softmax_pv(f32x16 (&s)[NQB], f32x16 (&oacc)[NQB][D / 32],
                                               float (&mrun)[NQB], float (&lrun)[NQB],
                                               const bf16x8 (&va)[D / 32][2], int qrow_minus_c0,
                                               int lane, float scale_log2) {
  const int hi = lane >> 5;
  constexpr int DB = D / 32;
  // ---- online softmax, per query = per lane ----
  bf16x8 pb[NQB][2];
#pragma unroll
  for (int i = 0; i < NQB; ++i) {
    // key offset within the chunk minus (query - c0): > 0 means masked
    const int rel = qrow_minus_c0 + 32 * i - 8 * hi;
    if (DIAG) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        s[i][r] = 16 * (r >> 3) + (r & 7) > rel ? neg_inf() : s[i][r];
    }
    float mx = s[i][0];
#pragma unroll
    for (int r = 1; r < 15; r += 2) mx = fmaxf(fmaxf(mx, s[i][r]), s[i][r + 1]);
    mx = max_halves(fmaxf(mx, s[i][15]));
    if (DIAG) mx = mx == neg_inf() ? mx : mx * scale_log2;  // a fully masked row stays -inf
    else mx *= scale_log2;
    // Lazy rescale (wave-uniform branch): move m only when some row's max exceeds it by more
    // than kRescale. A row whose chunk is fully masked has mx = -inf: no change.
    if (__builtin_amdgcn_ballot_w64(mx > mrun[i] + kRescale) != 0) {
      const float mnew = fmaxf(mrun[i], mx);
      // 0 on a row's first chunk (mrun = -inf); 1 while a row has seen no key
      const float corr = mnew == neg_inf() ? 1.0f : fast_exp2(mrun[i] - mnew);
      mrun[i] = mnew;
      lrun[i] *= corr;
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[i][db] *= corr;
    }
    const float mneg = -mrun[i];
    float ls = lrun[i];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 8 * j + 2 * e;
        float p0 = fast_exp2(fmaf(s[i][r], scale_log2, mneg));
        float p1 = fast_exp2(fmaf(s[i][r + 1], scale_log2, mneg));
        if (DIAG) {  // exact zeros for masked keys, whatever the scale
          p0 = 16 * j + 2 * e > rel ? 0.f : p0;
          p1 = 16 * j + 2 * e + 1 > rel ? 0.f : p1;
        }
        w[e] = pack_bf16x2(p0, p1);
        ls += p0 + p1;
      }
      pb[i][j] = as_bf16x8(w);
    }
    lrun[i] = ls;
  }
  // ---- O^T += V^T[:, chunk] P^T; each V^T operand read once for every query block ----
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < NQB; ++i) oacc[i][db] = mfma32(va[db][j], pb[i][j], oacc[i][db]);
}

template <int D>
__global__ __launch_bounds__(64 * kWaves, kMinBlocks)
__attribute__((amdgpu_num_vgpr(512 / (kMinBlocks * kWaves / 4)))) void fwd_bf16_kernel(
    bf16* __restrict__ out, float* __restrict__ lse, const bf16* __restrict__ q,
    const bf16* __restrict__ k, const bf16* __restrict__ v, int S, float scale_log2,
    int negate_q) {
  // scale_log2 = |scale| * log2(e); a negative scale is applied by negating Q (exact in bf16),
  // so the row max of the raw scores is the row max of the scaled ones.
  constexpr int QB = kQW * kWaves;
  constexpr int DS = D / 16;  // 16-wide K-steps along D
  constexpr int DB = D / 32;  // 32-row blocks of O^T
  // K and V tiles, triple-buffered: tile t is read while t+1 and t+2 are in flight. With the
  // tile loop unrolled by three every access names its buffer by a constant index, so the
  // compiler addresses all three from one register and knows that a pending direct load into
  // one buffer does not alias reads of another (it inserts no wait for it).
  __shared__ __attribute__((aligned(16))) bf16 sk[3][kTileRows * D];
  __shared__ __attribute__((aligned(16))) bf16 sv[3][kTileRows * D];

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
  bf16x8 qop[kNQB][DS];
#pragma unroll
  for (int i = 0; i < kNQB; ++i) {
    const int row = q0 + 32 * i + l32;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      qop[i][ds] = row < S ? ld_g128(qg + (size_t)row * D + 16 * ds + 8 * hi)
                           : as_bf16x8(u32x4{0, 0, 0, 0});
      if (negate_q) qop[i][ds] = neg_bf16x8(qop[i][ds]);
    }
  }

  f32x16 oacc[kNQB][DB];
  float mrun[kNQB], lrun[kNQB];  // running max (scaled log2 units); per-half row sums
#pragma unroll
  for (int i = 0; i < kNQB; ++i) {
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[i][db] = f32x16{};
    mrun[i] = neg_inf();
    lrun[i] = 0.f;
  }

  // Land the Q loads before the first direct load: the compiler does not see those, so a
  // wait it placed later for qop would also wait for every tile in flight.
  wait_vm_lds<0>();
  using Dma = DmaTile<D, kWaves>;
  constexpr int NI = 2 * Dma::PER_WAVE;  // DMA instructions per wave per tile (K and V)
  Dma::load(sk[0], kg, 0, S, wave, lane);
  Dma::load(sv[0], vg, 0, S, wave, lane);
  if (n_tiles > 1) {
    Dma::load(sk[1], kg, kTileRows, S, wave, lane);
    Dma::load(sv[1], vg, kTileRows, S, wave, lane);
    wait_vm_lds<NI>();
  } else {
    wait_vm_lds<0>();
  }
  __builtin_amdgcn_s_barrier();

  // One key tile: prefetch tile t+2 into (nk, nv) (it held tile t-1, released by the last
  // barrier), compute tile t from (ck, cv), then wait for tile t+1 (only tile t+2's loads may
  // still be in flight) and barrier, which also ends every wave's reads of tile t.
  auto tile = [&](int t, const bf16* ck, const bf16* cv, bf16* nk, bf16* nv) {
    const int k0 = t * kTileRows;
    const bool prefetch = t + 2 < n_tiles;
    if (prefetch) {
      Dma::load(nk, kg, k0 + 2 * kTileRows, S, wave, lane);
      Dma::load(nv, vg, k0 + 2 * kTileRows, S, wave, lane);
    }
    // Issue order is pinned with scheduling barriers: all K operand reads, then both chunks'
    // score MFMAs, then each chunk's V^T reads ahead of its softmax, so no MFMA waits on an
    // LDS read issued just before it and the second chunk's MFMAs run under the first
    // chunk's softmax.
    if (q0 < S && k0 <= q0 + kQW - 1) {  // some key of the tile at or before a query
      const bool live1 = k0 + 32 <= q0 + kQW - 1;  // likewise for chunk 1
      bf16x8 ka0[DS], ka1[DS], va[DB][2];
      f32x16 s0[kNQB], s1[kNQB];
      fwd_k_ops<D>(ka0, ck, 0, lane);
      if (live1) fwd_k_ops<D>(ka1, ck, 1, lane);
      __builtin_amdgcn_sched_barrier(0);
      fwd_scores<D, kNQB>(s0, qop, ka0);
      if (live1) fwd_scores<D, kNQB>(s1, qop, ka1);
      fwd_v_ops<D>(va, cv, 0, lane);
      __builtin_amdgcn_sched_barrier(0);
      const int rel0 = q0 + l32 - k0;
      if (k0 + 31 > q0)  // some key after some query: mask
        fwd_softmax_pv<D, kNQB, true>(s0, oacc, mrun, lrun, va, rel0, lane, scale_log2);
      else
        fwd_softmax_pv<D, kNQB, false>(s0, oacc, mrun, lrun, va, rel0, lane, scale_log2);
      if (live1) {
        fwd_v_ops<D>(va, cv, 1, lane);
        __builtin_amdgcn_sched_barrier(0);
        if (k0 + 63 > q0)
          fwd_softmax_pv<D, kNQB, true>(s1, oacc, mrun, lrun, va, rel0 - 32, lane, scale_log2);
        else
          fwd_softmax_pv<D, kNQB, false>(s1, oacc, mrun, lrun, va, rel0 - 32, lane, scale_log2);
      }
    }
    if (prefetch)
      wait_vm_lds<NI>();
    else
      wait_vm_lds<0>();
    __builtin_amdgcn_s_barrier();
  };
  for (int t = 0; t < n_tiles; t += 3) {
    tile(t, sk[0], sv[0], sk[2], sv[2]);
    if (t + 1 < n_tiles) tile(t + 1, sk[1], sv[1], sk[0], sv[0]);
    if (t + 2 < n_tiles) tile(t + 2, sk[2], sv[2], sk[1], sv[1]);
  }

  // ---- epilogue: O = O^T / l, lse = ln2 * (m + log2 l) ----
#pragma unroll
  for (int i = 0; i < kNQB; ++i) {
    const int qrow = q0 + 32 * i + l32;
    const float l = sum_halves(lrun[i]);
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

template <int D>
hipError_t launch_fwd_bf16_t(bf16* out, float* lse, const bf16* q, const bf16* k, const bf16* v,
                             int BH, int S, float scale, hipStream_t stream) {
  constexpr int QB = kQW * kWaves;
  dim3 grid(BH, (S + QB - 1) / QB);
  fwd_bf16_kernel<D><<<grid, 64 * kWaves, 0, stream>>>(out, lse, q, k, v, S,
                                                       fabsf(scale) * kLog2e, scale < 0.f);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fwd_bf16(bf16* out, float* lse, const bf16* q, const bf16* k, const bf16* v,
                           int BH, int S, int D, float scale, hipStream_t stream) {
  if (D == 64) return launch_fwd_bf16_t<64>(out, lse, q, k, v, BH, S, scale, stream);
  if (D == 32) return launch_fwd_bf16_t<32>(out, lse, q, k, v, BH, S, scale, stream);
  return hipErrorInvalidValue;
}

}  // namespace dadgpt
