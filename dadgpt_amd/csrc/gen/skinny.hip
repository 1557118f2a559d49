// Decode-step projections for at most 16 rows (one token per sequence): out[M,N] = A[M,K] W
// with W stored transposed, W^T [N, K] bf16, so that every MFMA operand is a contiguous
// 16-byte load straight from HBM (no LDS staging of the weights). These GEMMs are weight
// streams (M <= 16) far smaller than the bytes HBM needs in flight to reach its bandwidth,
// so each one takes about one memory latency if all its weight loads are issued at once, on
// many CUs; the work around each projection is folded into it, because at this size every
// dependent kernel costs its launch plus a memory round trip.
//
// Workgroup = 16 output columns (4 or 8 for narrow projections, below) x W waves: wave w takes
// the K range [w K/W, (w+1) K/W) (W = 4, 8 for the LayerNorm prologue at K a multiple of 256,
// 16 for K >= 2048) and issues all its weight loads up front; the partial products are summed
// through LDS and the epilogue runs in the same workgroup, so no result crosses workgroups.
// The grid is N/16 workgroups for the LayerNorm projections (144 for the QKV projection of
// GPT-2 124M, 192 for fc1) and N/4 for Wo and fc2 (192 instead of 48, which spreads their
// weight streams over most CUs). The epilogue's own
// inputs (bias, residual, cache row) are loaded first, so their latency hides under the
// weight stream.
// v_mfma_f32_16x16x32_bf16: lane l supplies A[l%16][8(l/16)+e] and B[8(l/16)+e][l%16] and
// holds D[4(l/16)+r][l%16]. Here A = W^T (rows = output columns n) and B = the activations
// transposed (columns = rows m of the batch), so D = out^T.
//
// Prologues (where the B operands come from):
//   kProRows  bf16 activations act [M][K], read straight from global memory (L2-resident)
//   kProLn    A = bf16(LayerNorm(x) w + b) of the fp32 residual stream x [M][K], computed by
//             every workgroup into LDS (two-pass mean and variance, eps 1e-5) with 16 or 32
//             threads per row, row sums on DPP and permlane swaps; the weight loads are
//             issued right after its inputs, so the stream runs under it
//   kProRowsF32  fp32 activations act32 [M][K] (the fp32 attention output), rounded to bf16
//             in registers as the operands are loaded: no separate conversion launch
//   kProRowsBlocked  bf16 activations stored K-blocked, [K/32][16][32] (the kEpiGelu layout):
//             each operand load of a wave is 1 KiB contiguous instead of 64 bytes of 16 rows,
//             which halves the cache lines every workgroup pulls through its CU for fc2
// Epilogues (per output element, after the bias):
//   kEpiStore     out [M][N] fp32                                       (logits)
//                 and, if cand is set, the workgroup's greedy candidate of each row (best
//                 column, its value, the runner-up value), so the pick reads 1/16 of the
//                 logits' columns instead of re-reading all of them
//   kEpiQkv       q -> q [M, H, dh]; k, v -> the caches [.., H, max_len, dh] at row pos[m]
//   kEpiGelu      g = bf16(gelu(.)), K-blocked for the next projection: element (m, n) at
//                 ((n/32)*16 + m)*32 + n%32 (the buffer holds 16 rows)       (fc1)
//   kEpiResidual  x [M][N] += .  (the residual stream, in place)        (Wo, fc2)
#include <hip/hip_runtime.h>

#include "gen_internal.hpp"
#include "pick.hpp"
#include "lanes.hpp"

namespace dadgpt::gen {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kRows = kSkinnyRows;  // batch rows of the skinny path
constexpr int kPad = 8;        // LDS row padding (16 bytes): conflict-free operand reads
constexpr int kMaxLnK = 1024;  // kProLn: the prologue holds a row's values in registers

// GELU, tanh form (src/tensor_ops.cpp:86-95): 0.5 x (1 + tanh(u)) = x / (1 + exp(-2u)), one
// exponential and one reciprocal instead of tanhf (the result is rounded to bf16).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float u = 0.7978845608f * (x + 0.044715f * x * x * x);
  return x / (1.0f + __expf(-2.0f * u));
}

__device__ __forceinline__ f32x4 ld_bf16x4(const bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}

template <int TPR>
__device__ __forceinline__ float sum_row(float v) {  // over the TPR lanes of a row group
  return lanes::group_sum<TPR>(v);                   // DPP and permlane swaps, no LDS trips
}

template <int EPI>
struct Epi {  // the epilogue's per-lane inputs, loaded (not yet converted) before the weights
  f32x4 bias_f = {0.f, 0.f, 0.f, 0.f};
  bf16x4 bias = {};
  f32x4 x = {0.f, 0.f, 0.f, 0.f};
  int pos = 0;
};

// WAVES waves, each over a K range of KW (K = WAVES * KW); COLS (16, 8 or 4) output columns
// per workgroup, so that a projection with few columns still spreads its weight stream over
// most CUs (the MFMA's other rows are zero and never stored).
template <int PRO, int EPI, int KW, int WAVES, int COLS>
__global__ __launch_bounds__(64 * WAVES) void skinny_kernel(SkinnyArgs a) {
  constexpr int K = WAVES * KW, NT = KW / 32;  // MFMA k-steps per wave
  constexpr int LDS_K = PRO == kProLn ? K : 1;
  constexpr int TPR = 64 * WAVES / kRows;  // LayerNorm threads per row (16 or 32)
  __shared__ __attribute__((aligned(16))) bf16 act[kRows][LDS_K + kPad];
  __shared__ f32x4 red[WAVES - 1][64];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  static_assert(COLS == 16 || COLS == 8 || COLS == 4, "column tile");
  const int n0 = blockIdx.x * COLS, kw0 = wave * KW;
  const int M = a.M, N = a.N;
  const int m = lane & 15, nl = n0 + 4 * (lane >> 4);  // this lane's row and first column
  const bool mine = 4 * (lane >> 4) < COLS;            // its columns belong to this workgroup
  const bool full4 = nl + 3 < N;                       // its 4 columns all exist

  // 0. the epilogue's inputs (wave 0 finishes the outputs), first in the load queue
  Epi<EPI> ep;
  if (wave == 0 && mine && m < M && nl < N) {
    if constexpr (EPI == kEpiQkv) {
      ep.pos = a.pos[m];
      ep.bias_f = *reinterpret_cast<const f32x4*>(a.bias_f + nl);  // 3d is a multiple of 16
    } else if constexpr (EPI != kEpiStore) {
      if (full4) {
        ep.bias = *reinterpret_cast<const bf16x4*>(a.bias + nl);
        if constexpr (EPI == kEpiResidual)
          ep.x = *reinterpret_cast<const f32x4*>(a.x_out + (size_t)m * N + nl);
      } else {
        for (int r = 0; nl + r < N; ++r) {
          ep.bias[r] = a.bias[nl + r];
          if constexpr (EPI == kEpiResidual) ep.x[r] = a.x_out[(size_t)m * N + nl + r];
        }
      }
    }
  }

  // 0b. the LayerNorm prologue's rows and parameters (TPR threads per row, pieces of 8
  //     columns: one 16-byte load of each parameter per piece), also ahead of the weights
  constexpr int NV = PRO == kProLn ? K / (8 * TPR) : 1;  // 8-column pieces per thread
  const int lr = tid / TPR, lj = tid % TPR;
  f32x4 xv[NV][2];
  bf16x8 lw[NV], lb[NV];
  if constexpr (PRO == kProLn) {
    static_assert(K % (8 * TPR) == 0 && K <= kMaxLnK, "row fits the registers");
    const int rr = min(lr, M - 1);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = 8 * (lj + TPR * i);
      xv[i][0] = *reinterpret_cast<const f32x4*>(a.x + (size_t)rr * K + c);
      xv[i][1] = *reinterpret_cast<const f32x4*>(a.x + (size_t)rr * K + c + 4);
      lw[i] = *reinterpret_cast<const bf16x8*>(a.ln_w + c);
      lb[i] = *reinterpret_cast<const bf16x8*>(a.ln_b + c);
    }
  }

  // 1. this wave's weight operands: row n of W^T (clamped to N-1 past the edge; those columns
  //    are not stored), 8 k per lane and step; all issued before anything waits
  bf16x8 w[NT];
  if (COLS == 16 || (lane & 15) < COLS) {
    const bf16* wp = a.wt + (size_t)min(n0 + (lane & 15), N - 1) * K + kw0 + 8 * (lane >> 4);
#pragma unroll
    for (int t = 0; t < NT; ++t) w[t] = *reinterpret_cast<const bf16x8*>(wp + 32 * t);
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t) w[t] = bf16x8{};
  }
  // (nothing that consumes a load moves above here: every load is in flight before the first
  // wait)
  __builtin_amdgcn_sched_barrier(0);

  // 2. B operands: lane holds batch row m = lane%16 (rows m >= M are zero), k = 8(lane/16) ..
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if constexpr (PRO != kProLn) {
    bf16x8 b[NT];
    if constexpr (PRO == kProRowsBlocked) {  // 16 rows x 32 k per 1 KiB block
      const bf16* ap = a.act + ((size_t)(kw0 / 32) * kRows + m) * 32 + 8 * (lane >> 4);
#pragma unroll
      for (int t = 0; t < NT; ++t) b[t] = *reinterpret_cast<const bf16x8*>(ap + 32 * kRows * t);
    } else if constexpr (PRO == kProRowsF32) {
      const float* ap = a.act32 + (size_t)min(m, M - 1) * K + kw0 + 8 * (lane >> 4);
      f32x4 lo[NT], hi[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        lo[t] = *reinterpret_cast<const f32x4*>(ap + 32 * t);
        hi[t] = *reinterpret_cast<const f32x4*>(ap + 32 * t + 4);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          b[t][e] = static_cast<bf16>(lo[t][e]);
          b[t][4 + e] = static_cast<bf16>(hi[t][e]);
        }
    } else {
      const bf16* ap = a.act + (size_t)min(m, M - 1) * K + kw0 + 8 * (lane >> 4);
#pragma unroll
      for (int t = 0; t < NT; ++t) b[t] = *reinterpret_cast<const bf16x8*>(ap + 32 * t);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w[t], m < M ? b[t] : bf16x8{}, acc, 0, 0,
                                                    0);
  } else {
    // LayerNorm of the 16 rows into LDS (two-pass mean and variance in fp32, eps 1e-5)
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += xv[i][e >> 2][e & 3];
    const float mean = sum_row<TPR>(sum) / (float)K;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float dv = xv[i][e >> 2][e & 3] - mean;
        sq += dv * dv;
      }
    const float inv_std = 1.0f / sqrtf(sum_row<TPR>(sq) / (float)K + 1e-5f);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o[e] = static_cast<bf16>(lr < M ? (xv[i][e >> 2][e & 3] - mean) * inv_std *
                                                  (float)lw[i][e] +
                                              (float)lb[i][e]
                                        : 0.0f);
      *reinterpret_cast<bf16x8*>(&act[lr][8 * (lj + TPR * i)]) = o;
    }
    __syncthreads();
    const bf16* ap = &act[m][kw0 + 8 * (lane >> 4)];
#pragma unroll
    for (int t = 0; t < NT; ++t)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          w[t], *reinterpret_cast<const bf16x8*>(ap + 32 * t), acc, 0, 0, 0);
  }

  // 3. sum the waves' products (wave 0 keeps the result): lane holds out[m][nl + r]
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int i = 0; i < WAVES - 1; ++i) acc += red[i][lane];
  if constexpr (EPI == kEpiStore) {
    if (a.cand != nullptr) {  // all 64 lanes take part: the 4 lanes of row m are 16 apart
      Pick p = pick_none();
      if (mine && m < M) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nl + r < N) p = pick_combine(p, Pick{acc[r], nl + r, -__builtin_inff()});
      }
      p = pick_combine(p, pick_shfl_xor(p, 16));
      p = pick_combine(p, pick_shfl_xor(p, 32));
      if (lane < 16 && m < M) {
        const size_t plane = (size_t)kRows * gridDim.x, i = (size_t)m * gridDim.x + blockIdx.x;
        a.cand[i] = p.v1;
        reinterpret_cast<int*>(a.cand)[plane + i] = p.i1;
        a.cand[2 * plane + i] = p.v2;
      }
    }
  }
  if (!mine || m >= M || nl >= N) return;
  if constexpr (EPI == kEpiStore) {
    float* o = a.out + (size_t)m * N + nl;
    if (full4 && (((size_t)m * N + nl) & 3) == 0)
      *reinterpret_cast<f32x4*>(o) = acc;
    else
      for (int r = 0; nl + r < N && r < 4; ++r) o[r] = acc[r];
  } else if constexpr (EPI == kEpiGelu) {
    bf16x4 o;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      o[r] = static_cast<bf16>(gelu_tanh(acc[r] + (float)ep.bias[r]));
    // K-blocked for kProRowsBlocked: the 4 columns lie in one 32-column block
    bf16* g = a.g + ((size_t)(nl / 32) * kRows + m) * 32 + nl % 32;
    if (full4)
      *reinterpret_cast<bf16x4*>(g) = o;
    else
      for (int r = 0; nl + r < N; ++r) g[r] = o[r];
  } else if constexpr (EPI == kEpiResidual) {
    const f32x4 xn = ep.x + acc +
                     f32x4{(float)ep.bias[0], (float)ep.bias[1], (float)ep.bias[2], (float)ep.bias[3]};
    float* x = a.x_out + (size_t)m * N + nl;
    if (full4)
      *reinterpret_cast<f32x4*>(x) = xn;
    else
      for (int r = 0; nl + r < N; ++r) x[r] = xn[r];
  } else {  // kEpiQkv: the 4 columns lie in one head (d_head is a multiple of 4)
    const f32x4 val = acc + ep.bias_f;
    const int d = N / 3, which = nl / d, c = nl % d, hh = c / a.dh, ee = c % a.dh;
    const size_t head = (size_t)m * a.H + hh;
    const size_t idx = which == 0 ? head * a.dh + ee : (head * a.max_len + ep.pos) * a.dh + ee;
    void* dst = which == 0 ? a.q : which == 1 ? a.kcache : a.vcache;
    if (a.qkv_fp32) {
      *reinterpret_cast<f32x4*>(static_cast<float*>(dst) + idx) = val;
    } else {
      bf16x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = static_cast<bf16>(val[r]);
      *reinterpret_cast<bf16x4*>(static_cast<bf16*>(dst) + idx) = o;
    }
  }
}

__global__ void transpose_kernel(bf16* out, const bf16* in, int rows, int cols) {
  __shared__ bf16 tile[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  for (int i = threadIdx.y; i < 32; i += blockDim.y) {
    const int r = r0 + i, c = c0 + threadIdx.x;
    if (r < rows && c < cols) tile[i][threadIdx.x] = in[(size_t)r * cols + c];
  }
  __syncthreads();
  for (int i = threadIdx.y; i < 32; i += blockDim.y) {
    const int c = c0 + i, r = r0 + threadIdx.x;
    if (r < rows && c < cols) out[(size_t)c * rows + r] = tile[threadIdx.x][i];
  }
}

// Column tile of a launch: 16 columns per workgroup, or 8 / 4 for the row-prologue
// projections while 16-column tiles would leave most of the 256 CUs idle (Wo and fc2 of
// GPT-2: 48 workgroups). The LayerNorm prologue stays at 16 columns: every workgroup
// recomputes the rows' statistics, and more workgroups made QKV slower (8.4 against 6.7 us at
// 8 columns).
int col_tile(int pro, int N) {
  if (pro == kProLn || N >= 16 * 160) return 16;
  return N >= 8 * 160 ? 8 : 4;
}

template <int PRO, int EPI, int KW, int WAVES>
hipError_t launch_kw(const SkinnyArgs& a, hipStream_t s) {
  constexpr int K = WAVES * KW;
  if constexpr (PRO == kProLn && (K > kMaxLnK || K % (8 * 64 * WAVES / kRows) != 0)) {
    return hipErrorInvalidValue;
  } else {
    const int cols = col_tile(PRO, a.N);
    if (cols == 16) {
      skinny_kernel<PRO, EPI, KW, WAVES, 16><<<dim3((a.N + 15) / 16), 64 * WAVES, 0, s>>>(a);
    } else if (cols == 8) {
      skinny_kernel<PRO, EPI, KW, WAVES, 8><<<dim3((a.N + 7) / 8), 64 * WAVES, 0, s>>>(a);
    } else {
      skinny_kernel<PRO, EPI, KW, WAVES, 4><<<dim3((a.N + 3) / 4), 64 * WAVES, 0, s>>>(a);
    }
    return hipGetLastError();
  }
}

// The row prologues keep each wave's range at 128-256 (so all of a wave's loads fit in
// registers at once) with up to 16 waves. The LayerNorm prologue runs on 8 waves (32 threads
// per row) where K is a multiple of 256: its per-thread share of the row statistics is half
// that of 4 waves, which took the GPT-2 QKV and fc1 LayerNorm from ~1.9 to ~1.1 us past the
// arrival of x (with the 16-byte parameter loads).
template <int PRO, int EPI>
hipError_t launch_k(const SkinnyArgs& a, hipStream_t s) {
  constexpr bool ln = PRO == kProLn;
  switch (a.K) {  // the reduction lengths of the supported configurations
    case 128: return launch_kw<PRO, EPI, 32, 4>(a, s);
    case 512: return ln ? launch_kw<PRO, EPI, 64, 8>(a, s) : launch_kw<PRO, EPI, 128, 4>(a, s);
    case 768: return ln ? launch_kw<PRO, EPI, 96, 8>(a, s) : launch_kw<PRO, EPI, 192, 4>(a, s);
    case 1024: return ln ? launch_kw<PRO, EPI, 128, 8>(a, s) : launch_kw<PRO, EPI, 256, 4>(a, s);
    case 2048: return launch_kw<PRO, EPI, 128, 16>(a, s);
    case 3072: return launch_kw<PRO, EPI, 192, 16>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int skinny_store_parts(int N) {
  const int cols = col_tile(kProRows, N);  // the same tile for kProRowsBlocked
  return (N + cols - 1) / cols;
}

bool skinny_supported(int M, int K) {
  return M >= 1 && M <= kRows &&
         (K == 128 || K == 512 || K == 768 || K == 1024 || K == 2048 || K == 3072);
}

hipError_t skinny_gemm(int pro, int epi, const SkinnyArgs& a, hipStream_t s) {
  if (!skinny_supported(a.M, a.K) || a.N < 1) return hipErrorInvalidValue;
  if (pro == kProLn && a.K > kMaxLnK) return hipErrorInvalidValue;
  if (epi == kEpiQkv && (a.N % 3 || (a.N / 3) % a.dh)) return hipErrorInvalidValue;
  if (epi == kEpiGelu && a.N % 32) return hipErrorInvalidValue;  // whole K-blocks
  if (pro == kProRows) {
    switch (epi) {
      case kEpiStore: return launch_k<kProRows, kEpiStore>(a, s);
      case kEpiResidual: return launch_k<kProRows, kEpiResidual>(a, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (pro == kProRowsBlocked) {
    switch (epi) {
      case kEpiStore: return launch_k<kProRowsBlocked, kEpiStore>(a, s);
      case kEpiResidual: return launch_k<kProRowsBlocked, kEpiResidual>(a, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (pro == kProRowsF32)
    return epi == kEpiResidual ? launch_k<kProRowsF32, kEpiResidual>(a, s)
                               : hipErrorInvalidValue;
  switch (epi) {
    case kEpiQkv: return launch_k<kProLn, kEpiQkv>(a, s);
    case kEpiGelu: return launch_k<kProLn, kEpiGelu>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t transpose(bf16* out, const bf16* in, int rows, int cols, hipStream_t s) {
  transpose_kernel<<<dim3((cols + 31) / 32, (rows + 31) / 32), dim3(32, 8), 0, s>>>(out, in,
                                                                                  rows, cols);
  return hipGetLastError();
}

}  // namespace dadgpt::gen
