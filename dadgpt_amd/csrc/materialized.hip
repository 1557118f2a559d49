// Row kernels of the materialized attention path (the [BH, S, S] probability matrix in HBM):
// the reference's own elementwise operators, and one-pass fusions of the chains it runs
// between its batched GEMMs (src/model.cpp:395-420 forward, :575-616 backward, :765-790
// decode).
//
// Every kernel walks rows with one wave per row (four rows per 256-lane workgroup); a lane
// holds columns lane, lane + 64, ... (16-byte pieces 4 floats wide when the row allows), so
// each load instruction of a wave covers 256 or 1024 contiguous bytes. Row maxima and sums
// are wave reductions through lane shuffles. The matrices are fp32, as the reference's.
//
// Arithmetic order per element follows the reference's operators: scores are multiplied by
// the scale, then masked to -1e9 (src/model.cpp:407-408; cuda/gpu_ops.cu:476-525), the
// softmax subtracts the row max, exponentiates with expf and divides by the row sum
// (cuda/gpu_ops.cu:147-193), and the softmax backward is p * (dp - sum(dp * p))
// (cuda/gpu_ops.cu:542-563), masked, then scaled (src/model.cpp:601-607). Only the order of
// the row sums differs (a wave tree instead of a block tree).
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "dropout.hpp"
#include "lanes.hpp"
#include "kernels.hpp"

namespace dadgpt {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr float kMaskValue = -1e9f;  // cuda/gpu_ops.cu:482

__device__ __forceinline__ float wave_max(float x) { return lanes::group_max<64>(x); }
__device__ __forceinline__ float wave_sum(float x) { return lanes::group_sum<64>(x); }

template <int V, typename F>
__device__ __forceinline__ void read_row(const float* row, int cols, int lane, F f) {
  if constexpr (V == 4) {
    for (int c = lane * 4; c < cols; c += 256) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(row + c);
      f(c, v.x), f(c + 1, v.y), f(c + 2, v.z), f(c + 3, v.w);
    }
  } else {
    for (int c = lane; c < cols; c += 64) f(c, row[c]);
  }
}

// What a softmax row sees of its input: the raw value (kPlain), scale then causal mask
// (kCausal: row r of a head is query r % S), or scale then a length mask (kLength: keys at or
// past lens[r / H] are masked; an empty cache gives a zero row).
enum RowMode { kPlain, kCausal, kLength };

template <int MODE, int V>
__global__ __launch_bounds__(64 * kRowsPerBlock) void softmax_rows_kernel(
    float* out, const float* in, long long rows, int cols, int S,
    float scale, const int* __restrict__ lens, int H) {
  const int lane = threadIdx.x & 63;
  const long long r = (long long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* src = in + r * cols;
  float* dst = out + r * cols;
  int limit = cols;  // columns at or past `limit` are masked
  if constexpr (MODE == kCausal) limit = (int)(r % S) + 1;
  if constexpr (MODE == kLength) {
    const int L = lens[r / H];
    limit = L < 0 ? 0 : (L > cols ? cols : L);
    if (limit == 0) {  // no keys: a zero row (o = 0, as the decode kernel returns)
      for (int c = lane; c < cols; c += 64) dst[c] = 0.f;
      return;
    }
  }
  auto value = [&](int c, float x) {
    if constexpr (MODE == kPlain) return x;
    const float s = x * scale;
    return c < limit ? s : kMaskValue;
  };
  float mx = -1e30f;  // the reference's initial max (cuda/gpu_ops.cu:156)
  read_row<V>(src, cols, lane, [&](int c, float x) { mx = fmaxf(mx, value(c, x)); });
  mx = wave_max(mx);
  float sum = 0.f;
  read_row<V>(src, cols, lane, [&](int c, float x) { sum += expf(value(c, x) - mx); });
  sum = wave_sum(sum);
  // in == out is allowed: each lane writes exactly the columns it reads, after reading them
  if constexpr (V == 4) {
    for (int c = lane * 4; c < cols; c += 256) {
      f32x4 v = *reinterpret_cast<const f32x4*>(src + c);
      v.x = expf(value(c, v.x) - mx) / sum;
      v.y = expf(value(c + 1, v.y) - mx) / sum;
      v.z = expf(value(c + 2, v.z) - mx) / sum;
      v.w = expf(value(c + 3, v.w) - mx) / sum;
      *reinterpret_cast<f32x4*>(dst + c) = v;
    }
  } else {
    for (int c = lane; c < cols; c += 64) dst[c] = expf(value(c, src[c]) - mx) / sum;
  }
}

// Softmax backward per row: g = p * (dp - sum_j dp_j p_j). ACCUMULATE: din += g (the
// reference's operator). Otherwise the attention form: din = g, zero past the causal
// diagonal, times scale (din may be dout).
template <bool ACCUMULATE>
__global__ __launch_bounds__(64 * kRowsPerBlock) void softmax_backward_rows_kernel(
    float* din, const float* dout, const float* __restrict__ p, long long rows, int cols, int S,
    float scale) {
  const int lane = threadIdx.x & 63;
  const long long r = (long long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* g = dout + r * cols;
  const float* pr = p + r * cols;
  float* d = din + r * cols;
  float dot = 0.f;
  for (int c = lane; c < cols; c += 64) dot += g[c] * pr[c];
  dot = wave_sum(dot);
  const int limit = ACCUMULATE ? cols : (int)(r % S) + 1;
  for (int c = lane; c < cols; c += 64) {
    const float v = pr[c] * (g[c] - dot);
    if constexpr (ACCUMULATE)
      d[c] += v;
    else
      d[c] = c < limit ? v * scale : 0.0f;
  }
}

// scores[h][i][j] = value for j > i over n_blocks blocks of S x S.
__global__ void causal_fill_kernel(float* __restrict__ m, long long rows, int S, float value) {
  const long long r = (long long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  float* row = m + r * S;
  for (int c = (int)(r % S) + 1 + (threadIdx.x & 63); c < S; c += 64) row[c] = value;
}

__global__ void scale_kernel(float* __restrict__ x, long long n, float scale) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x)
    x[i] *= scale;
}

// Attention-probability dropout on the materialized path, with the flash kernels' mask
// (dropout.hpp): element (r, c) of the [BH*S, S] probabilities is row r = bh*S + query and key
// c. Each lane owns 8 consecutive columns per step, whose keep bits are one Philox block;
// rows whose columns are not 16-byte pieces take the per-element path (V = 1).
template <int V, typename F>
__device__ __forceinline__ void row_groups(const float* row, int cols, int lane,
                                           const DropParams& dr, long long r, F f) {
  for (int c0 = 8 * lane; c0 < cols; c0 += 512) {
    const uint32_t bits = keep8(dr, (uint64_t)r, (uint32_t)c0 >> 3);
    if constexpr (V == 4) {  // cols % 8 == 0: the group is whole
      const f32x4 a = *reinterpret_cast<const f32x4*>(row + c0);
      const f32x4 b = *reinterpret_cast<const f32x4*>(row + c0 + 4);
      f(c0, a, b, bits);
    } else {
      f32x4 a, b;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[e] = c0 + e < cols ? row[c0 + e] : 0.f;
        b[e] = c0 + 4 + e < cols ? row[c0 + 4 + e] : 0.f;
      }
      f(c0, a, b, bits);
    }
  }
}

template <int V>
__device__ __forceinline__ void store_group(float* row, int cols, int c0, const f32x4& a,
                                            const f32x4& b) {
  if constexpr (V == 4) {
    *reinterpret_cast<f32x4*>(row + c0) = a;
    *reinterpret_cast<f32x4*>(row + c0 + 4) = b;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (c0 + e < cols) row[c0 + e] = a[e];
      if (c0 + 4 + e < cols) row[c0 + 4 + e] = b[e];
    }
  }
}

// out = p * keep / (1 - p_drop) (the reference's gpu_dropout_forward, cuda/gpu_ops.cu:712-733,
// with this mask). out may be p.
template <int V>
__global__ __launch_bounds__(64 * kRowsPerBlock) void dropout_rows_kernel(
    float* out, const float* p, long long rows, int cols, DropParams dr) {
  const int lane = threadIdx.x & 63;
  const long long r = (long long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  float* dst = out + r * cols;
  row_groups<V>(p + r * cols, cols, lane, dr, r, [&](int c0, f32x4 a, f32x4 b, uint32_t bits) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] *= keep_factor(bits, e, dr.scale);
      b[e] *= keep_factor(bits, 4 + e, dr.scale);
    }
    store_group<V>(dst, cols, c0, a, b);
  });
}

// The attention backward's row pass with dropout (src/model.cpp:594-607): dP = dPd * keep /
// (1 - p_drop) (gpu_dropout_backward, cuda/gpu_ops.cu:736-749), then the softmax backward
// against the undropped P, zero past the causal diagonal, times scale. ds may be dpd.
template <int V>
__global__ __launch_bounds__(64 * kRowsPerBlock) void attn_probs_backward_dropout_kernel(
    float* ds, const float* dpd, const float* __restrict__ p, long long rows, int S,
    float scale, DropParams dr) {
  const int lane = threadIdx.x & 63;
  const long long r = (long long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* g = dpd + r * S;
  const float* pr = p + r * S;
  float* d = ds + r * S;
  float dot = 0.f;
  row_groups<V>(g, S, lane, dr, r, [&](int c0, f32x4 a, f32x4 b, uint32_t bits) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (c0 + e < S) dot += a[e] * keep_factor(bits, e, dr.scale) * pr[c0 + e];
      if (c0 + 4 + e < S) dot += b[e] * keep_factor(bits, 4 + e, dr.scale) * pr[c0 + 4 + e];
    }
  });
  dot = wave_sum(dot);
  const int limit = (int)(r % S) + 1;
  row_groups<V>(g, S, lane, dr, r, [&](int c0, f32x4 a, f32x4 b, uint32_t bits) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ca = c0 + e, cb = c0 + 4 + e;
      a[e] = ca < limit ? pr[ca] * (a[e] * keep_factor(bits, e, dr.scale) - dot) * scale : 0.f;
      b[e] = cb < limit ? pr[cb] * (b[e] * keep_factor(bits, 4 + e, dr.scale) - dot) * scale
                        : 0.f;
    }
    store_group<V>(d, S, c0, a, b);
  });
}

// The head split and merge (cuda/gpu_ops.cu:426-474), a pure permutation between the
// token-major [B*S, H*dh] layout and [B*H, S, dh]. One workgroup per token row (b, s): its
// threads walk the row in W-float pieces (16 bytes when dh and both buffers allow), so the
// token-major side is one contiguous run and the head-major side one contiguous run of dh
// floats per head. MERGE runs the other direction.
template <bool MERGE, int W>
__global__ __launch_bounds__(256) void heads_kernel(float* __restrict__ out,
                                                    const float* __restrict__ in, int S, int H,
                                                    int dh) {
  using V = std::conditional_t<W == 4, f32x4, float>;
  const int row = blockIdx.x;  // b * S + s
  const int b = row / S, s = row - b * S;
  const int D = H * dh;
  const size_t tok = (size_t)row * D;
  for (int c = W * threadIdx.x; c < D; c += W * blockDim.x) {
    const int h = c / dh, x = c - h * dh;
    const size_t head = (((size_t)b * H + h) * S + s) * dh + x;
    const size_t src = MERGE ? head : tok + c, dst = MERGE ? tok + c : head;
    *reinterpret_cast<V*>(out + dst) = *reinterpret_cast<const V*>(in + src);
  }
}

template <bool MERGE>
hipError_t launch_heads(float* out, const float* in, int B, int S, int H, int dh,
                        hipStream_t stream) {
  const bool wide = dh % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(in) % 16 == 0;
  const int pieces = wide ? H * dh / 4 : H * dh;
  const int threads = std::min(256, (pieces + 63) / 64 * 64);
  const unsigned rows = (unsigned)((long long)B * S);
  if (wide)
    heads_kernel<MERGE, 4><<<rows, threads, 0, stream>>>(out, in, S, H, dh);
  else
    heads_kernel<MERGE, 1><<<rows, threads, 0, stream>>>(out, in, S, H, dh);
  return hipGetLastError();
}

unsigned row_blocks(long long rows) {
  return (unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock);
}

bool vec4(const void* a, const void* b, int cols) {
  return cols % 4 == 0 && reinterpret_cast<uintptr_t>(a) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(b) % 16 == 0;
}

template <int MODE>
hipError_t launch_softmax(float* out, const float* in, long long rows, int cols, int S,
                          float scale, const int* lens, int H, hipStream_t stream) {
  if (vec4(out, in, cols))
    softmax_rows_kernel<MODE, 4><<<row_blocks(rows), 64 * kRowsPerBlock, 0, stream>>>(
        out, in, rows, cols, S, scale, lens, H);
  else
    softmax_rows_kernel<MODE, 1><<<row_blocks(rows), 64 * kRowsPerBlock, 0, stream>>>(
        out, in, rows, cols, S, scale, lens, H);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_softmax_rows(float* out, const float* in, long long rows, int cols,
                               hipStream_t stream) {
  return launch_softmax<kPlain>(out, in, rows, cols, 1, 1.0f, nullptr, 1, stream);
}

hipError_t launch_softmax_backward_rows(float* din, const float* dout, const float* p,
                                        long long rows, int cols, hipStream_t stream) {
  softmax_backward_rows_kernel<true><<<row_blocks(rows), 64 * kRowsPerBlock, 0, stream>>>(
      din, dout, p, rows, cols, 1, 1.0f);
  return hipGetLastError();
}

hipError_t launch_causal_fill(float* m, int n_blocks, int S, float value, hipStream_t stream) {
  const long long rows = (long long)n_blocks * S;
  causal_fill_kernel<<<row_blocks(rows), 64 * kRowsPerBlock, 0, stream>>>(m, rows, S, value);
  return hipGetLastError();
}

hipError_t launch_scale(float* x, long long n, float scale, hipStream_t stream) {
  const long long blocks = (n + 255) / 256;
  scale_kernel<<<(unsigned)(blocks < 8192 ? blocks : 8192), 256, 0, stream>>>(x, n, scale);
  return hipGetLastError();
}

hipError_t launch_attention_probs(float* p, int BH, int S, float scale, hipStream_t stream) {
  return launch_softmax<kCausal>(p, p, (long long)BH * S, S, S, scale, nullptr, 1, stream);
}

hipError_t launch_attention_probs_backward(float* ds, const float* dp, const float* p, int BH,
                                           int S, float scale, hipStream_t stream) {
  const long long rows = (long long)BH * S;
  softmax_backward_rows_kernel<false><<<row_blocks(rows), 64 * kRowsPerBlock, 0, stream>>>(
      ds, dp, p, rows, S, S, scale);
  return hipGetLastError();
}

hipError_t launch_decode_probs(float* p, const int* lens, int n_seq, int H, int max_len,
                               float scale, hipStream_t stream) {
  return launch_softmax<kLength>(p, p, (long long)n_seq * H, max_len, 1, scale, lens, H,
                                 stream);
}

hipError_t launch_attention_dropout(float* out, const float* p, int BH, int S,
                                   const Dropout& drop, hipStream_t stream) {
  const long long rows = (long long)BH * S;
  const DropParams dr = drop_params(&drop);
  if (S % 8 == 0 && vec4(out, p, S))
    dropout_rows_kernel<4><<<row_blocks(rows), 64 * kRowsPerBlock, 0, stream>>>(out, p, rows, S,
                                                                                dr);
  else
    dropout_rows_kernel<1><<<row_blocks(rows), 64 * kRowsPerBlock, 0, stream>>>(out, p, rows, S,
                                                                                dr);
  return hipGetLastError();
}

hipError_t launch_attention_probs_backward_dropout(float* ds, const float* dpd, const float* p,
                                                   int BH, int S, float scale,
                                                   const Dropout& drop, hipStream_t stream) {
  const long long rows = (long long)BH * S;
  const DropParams dr = drop_params(&drop);
  if (S % 8 == 0 && vec4(ds, dpd, S) && vec4(p, p, S))
    attn_probs_backward_dropout_kernel<4><<<row_blocks(rows), 64 * kRowsPerBlock, 0, stream>>>(
        ds, dpd, p, rows, S, scale, dr);
  else
    attn_probs_backward_dropout_kernel<1><<<row_blocks(rows), 64 * kRowsPerBlock, 0, stream>>>(
        ds, dpd, p, rows, S, scale, dr);
  return hipGetLastError();
}

hipError_t launch_split_heads(float* out, const float* in, int B, int S, int H, int dh,
                              hipStream_t stream) {
  return launch_heads<false>(out, in, B, S, H, dh, stream);
}

hipError_t launch_merge_heads(float* out, const float* in, int B, int S, int H, int dh,
                              hipStream_t stream) {
  return launch_heads<true>(out, in, B, S, H, dh, stream);
}

}  // namespace dadgpt
