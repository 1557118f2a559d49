// Elementwise kernels of the GPT-2 generation driver (the non-GEMM, non-attention steps of
// src/model.cpp:334-475 and :687-825): embedding, LayerNorm, the QKV split with the KV-cache
// append fused in, bias + residual, bias + GELU, head merge, last-row gather and the greedy
// pick. All memory-bound; one row per block or wave, contiguous accesses along the row.
#include <hip/hip_runtime.h>

#include "gen_internal.hpp"

namespace dadgpt::gen {

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

__device__ __forceinline__ uint64_t splitmix_at(uint64_t seed, uint64_t k) {
  uint64_t z = seed + k * kGolden;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ double uniform_at(uint64_t seed, uint64_t k) {
  return ((double)(splitmix_at(seed, k) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

__global__ void init_normal_kernel(bf16* p, size_t n, uint64_t seed, float stddev) {
  const size_t pairs = (n + 1) / 2;
  for (size_t j = blockIdx.x * (size_t)blockDim.x + threadIdx.x; j < pairs;
       j += (size_t)gridDim.x * blockDim.x) {
    const double u1 = uniform_at(seed, 2 * j + 1), u2 = uniform_at(seed, 2 * j + 2);
    const double r = sqrt(-2.0 * log(u1)), t = 6.283185307179586 * u2;
    p[2 * j] = static_cast<bf16>((float)(r * cos(t)) * stddev);
    if (2 * j + 1 < n) p[2 * j + 1] = static_cast<bf16>((float)(r * sin(t)) * stddev);
  }
}

__global__ void fill_kernel(bf16* p, size_t n, float value) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = static_cast<bf16>(value);
}

__global__ void embed_kernel(float* x, const int* tok, const int* pos0, const bf16* wte,
                             const bf16* wpe, int S, int d) {
  const int r = blockIdx.x, b = r / S, s = r % S;
  const bf16* te = wte + (size_t)tok[r] * d;
  const bf16* pe = wpe + (size_t)(pos0[b] + s) * d;
  for (int c = threadIdx.x; c < d; c += blockDim.x)
    x[(size_t)r * d + c] = (float)te[c] + (float)pe[c];
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One wave per row, four rows per block.
__global__ __launch_bounds__(256) void layernorm_kernel(bf16* out, const float* x,
                                                        const bf16* w, const bf16* b, int rows,
                                                        int d) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + (size_t)row * d;
  float sum = 0.f;
  for (int c = lane; c < d; c += 64) sum += xr[c];
  const float mean = wave_sum(sum) / (float)d;
  float sq = 0.f;
  for (int c = lane; c < d; c += 64) {
    const float diff = xr[c] - mean;
    sq += diff * diff;
  }
  const float inv_std = 1.0f / sqrtf(wave_sum(sq) / (float)d + 1e-5f);
  bf16* orow = out + (size_t)row * d;
  for (int c = lane; c < d; c += 64)
    orow[c] = static_cast<bf16>((xr[c] - mean) * inv_std * (float)w[c] + (float)b[c]);
}

template <typename T>
__global__ void qkv_split_kernel(T* qh, T* kh, T* vh, T* kcache, T* vcache, const float* qkv,
                                 const float* bqkv, const int* pos0, const int* nvalid, int S,
                                 int H, int dh, int max_len) {
  const int r = blockIdx.x, b = r / S, s = r % S;
  const int d = H * dh;
  const float* row = qkv + (size_t)r * 3 * d;
  const bool append = s < nvalid[b];
  const int p = pos0[b] + s;
  for (int c = threadIdx.x; c < d; c += blockDim.x) {
    const int h = c / dh, e = c % dh;
    const size_t head = (size_t)b * H + h;
    const T kval = static_cast<T>(row[d + c] + bqkv[d + c]);
    const T vval = static_cast<T>(row[2 * d + c] + bqkv[2 * d + c]);
    qh[(head * S + s) * dh + e] = static_cast<T>(row[c] + bqkv[c]);
    if (kh) {
      kh[(head * S + s) * dh + e] = kval;
      vh[(head * S + s) * dh + e] = vval;
    }
    if (append) {
      kcache[(head * max_len + p) * dh + e] = kval;
      vcache[(head * max_len + p) * dh + e] = vval;
    }
  }
}

template <typename T>
__global__ void merge_heads_kernel(bf16* out, const T* heads, int S, int H, int dh) {
  const int r = blockIdx.x, b = r / S, s = r % S;
  const int d = H * dh;
  for (int c = threadIdx.x; c < d; c += blockDim.x) {
    const int h = c / dh, e = c % dh;
    out[(size_t)r * d + c] = static_cast<bf16>((float)heads[(((size_t)b * H + h) * S + s) * dh + e]);
  }
}

__global__ void to_bf16_kernel(bf16* out, const float* in, size_t count) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = static_cast<bf16>(in[i]);
}

__global__ void bias_residual_kernel(float* x, const float* y, const bf16* bias, int rows,
                                     int cols) {
  const size_t n = (size_t)rows * cols;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    x[i] += y[i] + (float)bias[i % cols];
}

// GELU, tanh form (cuda/gpu_ops.cu:250-256, src/tensor_ops.cpp:86-95).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float inner = 0.7978845608f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

__global__ void bias_gelu_kernel(bf16* out, const float* y, const bf16* bias, int rows,
                                 int cols) {
  const size_t n = (size_t)rows * cols;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = static_cast<bf16>(gelu_tanh(y[i] + (float)bias[i % cols]));
}

__global__ void gather_last_kernel(float* out, const float* x, const int* len, int S, int d) {
  const int b = blockIdx.x;
  const float* src = x + ((size_t)b * S + len[b] - 1) * d;
  for (int c = threadIdx.x; c < d; c += blockDim.x) out[(size_t)b * d + c] = src[c];
}

struct Pick {
  float v1;
  int i1;
  float v2;
};

// The better of two candidates (higher value, then lower index) keeps its index; the runner-up
// value is the larger of the loser's best and the winner's runner-up.
__device__ __forceinline__ Pick combine(Pick a, Pick b) {
  const bool b_wins = b.v1 > a.v1 || (b.v1 == a.v1 && b.i1 < a.i1);
  const Pick& w = b_wins ? b : a;
  const Pick& l = b_wins ? a : b;
  return Pick{w.v1, w.i1, fmaxf(l.v1, w.v2)};
}

__global__ __launch_bounds__(256) void argmax_advance_kernel(int* tokens, float* margins,
                                                             int* tok, int* pos, int* cache_len,
                                                             const float* logits, int n, int V,
                                                             int step, int advance) {
  __shared__ float s_v1[256], s_v2[256];
  __shared__ int s_i1[256];
  const int b = blockIdx.x, t = threadIdx.x;
  const float* row = logits + (size_t)b * V;
  Pick p{-__builtin_inff(), 0x7fffffff, -__builtin_inff()};
  for (int v = t; v < V; v += 256) p = combine(p, Pick{row[v], v, -__builtin_inff()});
  s_v1[t] = p.v1;
  s_i1[t] = p.i1;
  s_v2[t] = p.v2;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (t < w) {
      const Pick q = combine(Pick{s_v1[t], s_i1[t], s_v2[t]},
                             Pick{s_v1[t + w], s_i1[t + w], s_v2[t + w]});
      s_v1[t] = q.v1;
      s_i1[t] = q.i1;
      s_v2[t] = q.v2;
    }
    __syncthreads();
  }
  if (t == 0) {
    const int pick = s_i1[0];
    tokens[(size_t)step * n + b] = pick;
    margins[(size_t)step * n + b] = s_v1[0] - s_v2[0];
    tok[b] = pick;
    pos[b] += advance;
    cache_len[b] = pos[b] + 1;
  }
}

__global__ void pack_bias_kernel(float* bqkv, const bf16* bq, const bf16* bk, const bf16* bv,
                                 int d) {
  for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < d; c += gridDim.x * blockDim.x) {
    bqkv[c] = (float)bq[c];
    bqkv[d + c] = (float)bk[c];
    bqkv[2 * d + c] = (float)bv[c];
  }
}

unsigned grid_for(size_t n, unsigned threads = 256, unsigned cap = 65536) {
  const size_t g = (n + threads - 1) / threads;
  return (unsigned)(g < 1 ? 1 : (g > cap ? cap : g));
}

}  // namespace

hipError_t init_normal(bf16* p, size_t n, uint64_t seed, float stddev, hipStream_t s) {
  init_normal_kernel<<<grid_for((n + 1) / 2), 256, 0, s>>>(p, n, seed, stddev);
  return hipGetLastError();
}

hipError_t fill(bf16* p, size_t n, float value, hipStream_t s) {
  fill_kernel<<<grid_for(n), 256, 0, s>>>(p, n, value);
  return hipGetLastError();
}

hipError_t embed(float* x, const int* tok, const int* pos0, const bf16* wte, const bf16* wpe,
                 int n, int S, int d, hipStream_t s) {
  embed_kernel<<<n * S, 256, 0, s>>>(x, tok, pos0, wte, wpe, S, d);
  return hipGetLastError();
}

hipError_t layernorm(bf16* out, const float* x, const bf16* w, const bf16* b, int rows, int d,
                     hipStream_t s) {
  layernorm_kernel<<<(rows + 3) / 4, 256, 0, s>>>(out, x, w, b, rows, d);
  return hipGetLastError();
}

template <typename T>
hipError_t qkv_split(T* qh, T* kh, T* vh, T* kcache, T* vcache, const float* qkv,
                     const float* bqkv, const int* pos0, const int* nvalid, int n, int S, int H,
                     int dh, int max_len, hipStream_t s) {
  qkv_split_kernel<T><<<n * S, 256, 0, s>>>(qh, kh, vh, kcache, vcache, qkv, bqkv, pos0, nvalid,
                                            S, H, dh, max_len);
  return hipGetLastError();
}
template hipError_t qkv_split<bf16>(bf16*, bf16*, bf16*, bf16*, bf16*, const float*,
                                    const float*, const int*, const int*, int, int, int, int,
                                    int, hipStream_t);
template hipError_t qkv_split<float>(float*, float*, float*, float*, float*, const float*,
                                     const float*, const int*, const int*, int, int, int, int,
                                     int, hipStream_t);

template <typename T>
hipError_t merge_heads(bf16* out, const T* heads, int n, int S, int H, int dh, hipStream_t s) {
  merge_heads_kernel<T><<<n * S, 256, 0, s>>>(out, heads, S, H, dh);
  return hipGetLastError();
}
template hipError_t merge_heads<bf16>(bf16*, const bf16*, int, int, int, int, hipStream_t);
template hipError_t merge_heads<float>(bf16*, const float*, int, int, int, int, hipStream_t);

hipError_t to_bf16(bf16* out, const float* in, size_t count, hipStream_t s) {
  to_bf16_kernel<<<grid_for(count), 256, 0, s>>>(out, in, count);
  return hipGetLastError();
}

hipError_t bias_residual(float* x, const float* y, const bf16* bias, int rows, int cols,
                         hipStream_t s) {
  bias_residual_kernel<<<grid_for((size_t)rows * cols), 256, 0, s>>>(x, y, bias, rows, cols);
  return hipGetLastError();
}

hipError_t bias_gelu(bf16* out, const float* y, const bf16* bias, int rows, int cols,
                     hipStream_t s) {
  bias_gelu_kernel<<<grid_for((size_t)rows * cols), 256, 0, s>>>(out, y, bias, rows, cols);
  return hipGetLastError();
}

hipError_t gather_last(float* out, const float* x, const int* len, int n, int S, int d,
                       hipStream_t s) {
  gather_last_kernel<<<n, 256, 0, s>>>(out, x, len, S, d);
  return hipGetLastError();
}

hipError_t argmax_advance(int* tokens, float* margins, int* tok, int* pos, int* cache_len,
                          const float* logits, int n, int V, int step, int advance,
                          hipStream_t s) {
  argmax_advance_kernel<<<n, 256, 0, s>>>(tokens, margins, tok, pos, cache_len, logits, n, V,
                                          step, advance);
  return hipGetLastError();
}

hipError_t pack_bias(float* bqkv, const bf16* bq, const bf16* bk, const bf16* bv, int d,
                     hipStream_t s) {
  pack_bias_kernel<<<grid_for(d), 256, 0, s>>>(bqkv, bq, bk, bv, d);
  return hipGetLastError();
}

}  // namespace dadgpt::gen
