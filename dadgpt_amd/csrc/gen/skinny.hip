// Decode-step projections for at most 16 rows (one token per sequence): out[M,N] = A[M,K] W
// with W stored transposed, W^T [N, K] bf16, so that every MFMA operand is a contiguous
// 16-byte load straight from HBM (no LDS staging of the weights). These GEMMs are weight
// streams (M <= 16): the point is to have the whole weight matrix in flight at once and to
// fold the elementwise work around each projection into it, because at this size every
// dependent kernel costs its launch plus a memory round trip.
//
// Workgroup = 4 waves x 16 output columns; wave w owns columns n0 + 16w .. +15 and one
// K-chunk of KC (blockIdx.y selects the chunk; partial sums go to parts[chunk], summed by the
// consumer in chunk order). v_mfma_f32_16x16x32_bf16: lane l supplies A[l%16][8(l/16)+e] and
// B[8(l/16)+e][l%16] and holds D[4(l/16)+r][l%16]. Here A = W^T (rows = output columns n) and
// B = the activations transposed (columns = rows m of the batch), so D = out^T.
//
// The activations reach the MFMA through LDS, produced by a prologue (one of):
//   kProRows    A = bf16 rows act[m][k]                                   (Wo, logits)
//   kProLayerNorm  x' = x + sum_s parts_s + bias (the residual add of the previous
//               projection), A = LayerNorm(x') * w + b over the full row (K = the chunk,
//               <= 768); workgroup (0,0) also stores x' (the next residual stream) (QKV, fc1)
//   kProGelu    A = gelu(sum_s parts_s + bias) for this chunk's columns    (fc2)
#include <hip/hip_runtime.h>

#include "gen_internal.hpp"

namespace dadgpt::gen {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 16;         // batch rows of the skinny path
constexpr int kMaxLnVals = 48;    // LayerNorm prologue: K <= 16 * 48 = 768
constexpr int kPad = 8;           // LDS row padding (16 bytes): conflict-free operand reads

// GELU, tanh form (src/tensor_ops.cpp:86-95): 0.5 x (1 + tanh(u)) = x / (1 + exp(-2u)), one
// exponential and one reciprocal instead of tanhf (the result is rounded to bf16).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float u = 0.7978845608f * (x + 0.044715f * x * x * x);
  return x / (1.0f + __expf(-2.0f * u));
}

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4 ld_bf16x4(const bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}

__device__ __forceinline__ float sum16(float v) {  // over the 16 lanes of a row group
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int PRO, int KC>
__global__ __launch_bounds__(256) void skinny_gemm_kernel(SkinnyArgs a) {
  constexpr int NT = KC / 32;  // MFMA k-steps of a chunk
  __shared__ __attribute__((aligned(16))) bf16 act[kRows][KC + kPad];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n0 = blockIdx.x * 64 + wave * 16;
  const int chunk = blockIdx.y, k0 = chunk * KC;

  // Issue order: the prologue's (small) loads first, then this wave's weight operands, so
  // the prologue math waits only for its own data (loads complete in order) while the
  // weights keep streaming.
  bf16x8 w[NT];
  auto load_weights = [&] {
    // row n of W^T (clamped to N-1 past the edge; those columns are not stored), 8 k per lane
    const int n = min(n0 + (lane & 15), a.N - 1);
    const bf16* wp = a.wt + (size_t)n * a.K + k0 + 8 * (lane >> 4);
#pragma unroll
    for (int t = 0; t < NT; ++t) w[t] = *reinterpret_cast<const bf16x8*>(wp + 32 * t);
  };

  // prologue: the activations of this chunk into LDS (rows m >= M are zero); loads use
  // clamped, always-valid addresses
  if constexpr (PRO == kProRows) {
    constexpr int PER = kRows * KC / 8 / 256;  // 16-byte pieces per thread
    static_assert(PER * 256 * 8 == kRows * KC, "whole pieces per thread");
    bf16x8 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int p = tid + 256 * i, m = p / (KC / 8), j = 8 * (p % (KC / 8));
      v[i] = *reinterpret_cast<const bf16x8*>(a.act + (size_t)min(m, a.M - 1) * a.K + k0 + j);
    }
    load_weights();
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int p = tid + 256 * i, m = p / (KC / 8), j = 8 * (p % (KC / 8));
      if (m >= a.M) v[i] = bf16x8{};
      *reinterpret_cast<bf16x8*>(&act[m][j]) = v[i];
    }
  } else if constexpr (PRO == kProGelu) {
    constexpr int PER = kRows * KC / 4 / 256;  // 4-float pieces per thread
    static_assert(PER * 256 * 4 == kRows * KC, "whole pieces per thread");
    f32x4 v[PER], bias[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int p = tid + 256 * i, m = p / (KC / 4), j = 4 * (p % (KC / 4));
      v[i] = *reinterpret_cast<const f32x4*>(a.in_parts + (size_t)min(m, a.M - 1) * a.K + k0 + j);
      bias[i] = ld_bf16x4(a.in_bias + k0 + j);
    }
    for (int sp = 1; sp < a.in_splits; ++sp) {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int p = tid + 256 * i, m = p / (KC / 4), j = 4 * (p % (KC / 4));
        v[i] += *reinterpret_cast<const f32x4*>(
            a.in_parts + ((size_t)sp * a.M + min(m, a.M - 1)) * a.K + k0 + j);
      }
    }
    load_weights();
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int p = tid + 256 * i, m = p / (KC / 4), j = 4 * (p % (KC / 4));
#pragma unroll
      for (int e = 0; e < 4; ++e)
        act[m][j + e] = static_cast<bf16>(m < a.M ? gelu_tanh(v[i][e] + bias[i][e]) : 0.0f);
    }
  } else {  // kProLayerNorm: 16 threads per row, the whole row (K = KC) in registers
    static_assert(KC % 64 == 0 && KC / 64 <= kMaxLnVals / 4, "row fits the registers");
    constexpr int NV = KC / 64;  // float4 pieces per thread
    const int m = tid >> 4, j = tid & 15, mm = min(m, a.M - 1);
    f32x4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i)
      v[i] = *reinterpret_cast<const f32x4*>(a.x_in + (size_t)mm * a.K + 4 * (j + 16 * i));
    for (int sp = 0; sp < a.in_splits; ++sp) {
#pragma unroll
      for (int i = 0; i < NV; ++i)
        v[i] += *reinterpret_cast<const f32x4*>(a.in_parts + ((size_t)sp * a.M + mm) * a.K +
                                                4 * (j + 16 * i));
    }
    if (a.in_bias) {
#pragma unroll
      for (int i = 0; i < NV; ++i) v[i] += ld_bf16x4(a.in_bias + 4 * (j + 16 * i));
    }
    load_weights();
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) sum += v[i][0] + v[i][1] + v[i][2] + v[i][3];
    const float mean = sum16(sum) / (float)a.K;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) sq += (v[i][e] - mean) * (v[i][e] - mean);
    const float inv_std = 1.0f / sqrtf(sum16(sq) / (float)a.K + 1e-5f);
    const bool store_x = a.x_out && blockIdx.x == 0 && blockIdx.y == 0 && m < a.M;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = 4 * (j + 16 * i);
      if (store_x) *reinterpret_cast<f32x4*>(a.x_out + (size_t)m * a.K + c) = v[i];
      const f32x4 g = ld_bf16x4(a.ln_w + c), b = ld_bf16x4(a.ln_b + c);
      bf16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = static_cast<bf16>(m < a.M ? (v[i][e] - mean) * inv_std * g[e] + b[e] : 0.0f);
      *reinterpret_cast<bf16x4*>(&act[m][c]) = o;
    }
  }
  __syncthreads();

  // 3. D = W^T A^T over the chunk
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const bf16* arow = &act[lane & 15][8 * (lane >> 4)];
#pragma unroll
  for (int t = 0; t < NT; ++t)
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        w[t], *reinterpret_cast<const bf16x8*>(arow + 32 * t), acc, 0, 0, 0);

  // 4. lane holds out[m = lane%16][n0 + 4(lane/16) + r]
  const int m = lane & 15;
  if (m < a.M) {
    float* out = a.parts + ((size_t)chunk * a.M + m) * a.N;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = n0 + 4 * (lane >> 4) + r;
      if (n < a.N) out[n] = acc[r];
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

}  // namespace

bool skinny_supported(int M, int K) {
  return M >= 1 && M <= kRows && K % 128 == 0 && K >= 128;
}

// The K-chunk of a reduction: the largest of 768, 512, 384, 256, 128 that divides K.
int skinny_chunk(int K) {
  for (int kc : {768, 512, 384, 256, 128})
    if (K % kc == 0) return kc;
  return 128;
}

namespace {
template <int PRO>
hipError_t launch_pro(const SkinnyArgs& a, dim3 grid, hipStream_t s) {
  switch (a.kc) {
    case 128: skinny_gemm_kernel<PRO, 128><<<grid, 256, 0, s>>>(a); break;
    case 256: skinny_gemm_kernel<PRO, 256><<<grid, 256, 0, s>>>(a); break;
    case 384: skinny_gemm_kernel<PRO, 384><<<grid, 256, 0, s>>>(a); break;
    case 512: skinny_gemm_kernel<PRO, 512><<<grid, 256, 0, s>>>(a); break;
    case 768: skinny_gemm_kernel<PRO, 768><<<grid, 256, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

hipError_t skinny_gemm(int pro, const SkinnyArgs& args, hipStream_t s) {
  if (!skinny_supported(args.M, args.K) || args.K % args.kc ||
      (pro == kProLayerNorm && args.kc != args.K))
    return hipErrorInvalidValue;
  const dim3 grid((args.N + 63) / 64, args.K / args.kc);
  if (pro == kProRows) return launch_pro<kProRows>(args, grid, s);
  if (pro == kProLayerNorm) return launch_pro<kProLayerNorm>(args, grid, s);
  return launch_pro<kProGelu>(args, grid, s);
}

hipError_t transpose(bf16* out, const bf16* in, int rows, int cols, hipStream_t s) {
  transpose_kernel<<<dim3((cols + 31) / 32, (rows + 31) / 32), dim3(32, 8), 0, s>>>(out, in,
                                                                                  rows, cols);
  return hipGetLastError();
}

}  // namespace dadgpt::gen
