// Elementwise kernels of the GPT-2 generation driver (the non-GEMM, non-attention steps of
// src/model.cpp:334-475 and :687-825): embedding, LayerNorm, the QKV split with the KV-cache
// append fused in, bias + residual, bias + GELU, head merge, last-row gather and the greedy
// pick. All memory-bound; one row per block or wave, contiguous accesses along the row.
#include <hip/hip_runtime.h>

#include "gen_internal.hpp"
#include "pick.hpp"
#include "lanes.hpp"

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
                             const bf16* wpe, const int* rowmap, int S, int d) {
  // packed row r holds padded position p = b*S + s (rowmap), or r = p without a map
  const int r = blockIdx.x, p = rowmap ? rowmap[r] : r, b = p / S, s = p % S;
  const bf16* te = wte + (size_t)tok[p] * d;
  const bf16* pe = wpe + (size_t)(pos0[b] + s) * d;
  for (int c = threadIdx.x; c < d; c += blockDim.x)
    x[(size_t)r * d + c] = (float)te[c] + (float)pe[c];
}

__device__ __forceinline__ float wave_sum(float v) { return lanes::group_sum<64>(v); }

// Sum over the 256 threads of a block (4 waves): wave shuffles, then the 4 partials via LDS.
__device__ __forceinline__ float block_sum(float v, float* sm) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();  // sm may still be read from a previous reduction
  if (lane == 0) sm[wave] = v;
  __syncthreads();
  return sm[0] + sm[1] + sm[2] + sm[3];
}

constexpr int kLnMaxPerThread = 8;  // d <= 2048

// One row per 256-thread block, the row held in registers: optionally x += y + bias (the
// residual add of the previous projection), then out = O(LayerNorm(x) * w + b) (O bf16 or
// fp32) with eps 1e-5 and two-pass mean and variance in fp32 (src/tensor_ops.cpp:57-84).
// w == nullptr: residual only.
template <typename O>
__global__ __launch_bounds__(256) void residual_layernorm_kernel(float* x, const float* y,
                                                                 const bf16* bias, O* out,
                                                                 const bf16* w, const bf16* b,
                                                                 int d, int splits,
                                                                 int blocked) {
  __shared__ float sm[4];
  float* xr = x + (size_t)blockIdx.x * d;
  float v[kLnMaxPerThread];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kLnMaxPerThread; ++i) {
    const int c = threadIdx.x + 256 * i;
    v[i] = 0.f;
    if (c < d) {
      v[i] = xr[c];
      if (y) {
        for (int sp = 0; sp < splits; ++sp)
          v[i] += y[((size_t)sp * gridDim.x + blockIdx.x) * d + c];
        v[i] += (float)bias[c];
        xr[c] = v[i];
      }
      sum += v[i];
    }
  }
  if (!w) return;
  const float mean = block_sum(sum, sm) / (float)d;
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < kLnMaxPerThread; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c < d) sq += (v[i] - mean) * (v[i] - mean);
  }
  const float inv_std = 1.0f / sqrtf(block_sum(sq, sm) / (float)d + 1e-5f);
  O* orow = out + (size_t)blockIdx.x * (blocked ? 32 : d);
#pragma unroll
  for (int i = 0; i < kLnMaxPerThread; ++i) {
    const int c = threadIdx.x + 256 * i;
    // blocked: element (r, c) at ((c/32)*16 + r)*32 + c%32 (the skinny K-blocked layout)
    if (c < d)
      orow[blocked ? (c / 32) * 32 * kSkinnyRows + c % 32 : c] =
          static_cast<O>((v[i] - mean) * inv_std * (float)w[c] + (float)b[c]);
  }
}

template <typename T>
__global__ void qkv_split_kernel(T* qh, T* kh, T* vh, T* kcache, T* vcache, const float* qkv,
                                 const float* bqkv, const int* pos0, const int* nvalid,
                                 const int* rowmap, int S, int H, int dh, int max_len) {
  // qkv row r is padded position p = b*S + s (rowmap), or r = p without a map
  const int r = blockIdx.x, pr = rowmap ? rowmap[r] : r, b = pr / S, s = pr % S;
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

template <typename T, typename O>
__global__ void merge_heads_kernel(O* out, const T* heads, const int* rowmap, int S, int H,
                                   int dh) {
  // output row r is padded position p = b*S + s (rowmap), or r = p without a map
  const int r = blockIdx.x, p = rowmap ? rowmap[r] : r, b = p / S, s = p % S;
  const int d = H * dh;
  for (int c = threadIdx.x; c < d; c += blockDim.x) {
    const int h = c / dh, e = c % dh;
    out[(size_t)r * d + c] = static_cast<O>((float)heads[(((size_t)b * H + h) * S + s) * dh + e]);
  }
}

__global__ void to_f32_kernel(float* out, const bf16* in, size_t count) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = static_cast<float>(in[i]);
}

__global__ void to_bf16_kernel(bf16* out, const float* in, size_t count) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = static_cast<bf16>(in[i]);
}

// GELU, tanh form (cuda/gpu_ops.cu:250-256, src/tensor_ops.cpp:86-95).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float inner = 0.7978845608f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

template <typename O>
__global__ void bias_gelu_kernel(O* out, const float* y, const bf16* bias, int rows, int cols) {
  const size_t n = (size_t)rows * cols;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = static_cast<O>(gelu_tanh(y[i] + (float)bias[i % cols]));
}

template <typename T>
__global__ void gather_rows_kernel(T* out, const T* in, const int* idx, int d) {
  const int r = blockIdx.x;
  const T* src = in + (size_t)idx[r] * d;
  for (int c = threadIdx.x; c < d; c += blockDim.x) out[(size_t)r * d + c] = src[c];
}

constexpr int kPickParts = 32;  // blocks per row in the first stage of the greedy pick

// Stage 1: block (b, part) reduces a contiguous slice of row b to one candidate.
__global__ __launch_bounds__(256) void pick_partial_kernel(float* pv1, int* pi1, float* pv2,
                                                           const float* logits, int V) {
  __shared__ float s_v1[256], s_v2[256];
  __shared__ int s_i1[256];
  const int b = blockIdx.x, part = blockIdx.y, t = threadIdx.x;
  const int span = (V + kPickParts - 1) / kPickParts;
  const int lo = part * span, hi = min(V, lo + span);
  const float* row = logits + (size_t)b * V;
  Pick p = pick_none();
  for (int v = lo + t; v < hi; v += 256) p = pick_combine(p, Pick{row[v], v, -__builtin_inff()});
  s_v1[t] = p.v1;
  s_i1[t] = p.i1;
  s_v2[t] = p.v2;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (t < w) {
      const Pick q = pick_combine(Pick{s_v1[t], s_i1[t], s_v2[t]},
                                  Pick{s_v1[t + w], s_i1[t + w], s_v2[t + w]});
      s_v1[t] = q.v1;
      s_i1[t] = q.i1;
      s_v2[t] = q.v2;
    }
    __syncthreads();
  }
  if (t == 0) {
    const int k = b * kPickParts + part;
    pv1[k] = s_v1[0];
    pi1[k] = s_i1[0];
    pv2[k] = s_v2[0];
  }
}

// Stage 2: one 256-thread block per row merges the row's `parts` candidates (stage 1's, or
// those of the logits projection's epilogue), stores the pick, advances, and embeds the
// picked token at its new position as the next decode step's input row (the step's first
// launch would otherwise be that embedding).
__global__ __launch_bounds__(256) void pick_final_kernel(int* tokens, float* margins, int* tok,
                                                         int* pos, int* cache_len,
                                                         const int* prompt_len, RowStop rs,
                                                         const float* pv1, const int* pi1,
                                                         const float* pv2, int parts, int n,
                                                         int V, float* x, const bf16* wte,
                                                         const bf16* wpe, int d, int ctx) {
  __shared__ Pick s_wave[4];
  const int b = blockIdx.x, t = threadIdx.x;
  if (rs.done[b]) {
    // a stopped row: re-feed its last token at its last position (set by the pick that
    // stopped it, so both are in range); nothing is emitted and no state advances
    const int p0 = pos[b];
    const bf16* te = wte + (size_t)tok[b] * d;
    const bf16* pe = wpe + (size_t)p0 * d;
    if (p0 >= 0 && p0 < ctx)
      for (int c = t; c < d; c += 256) x[(size_t)b * d + c] = (float)te[c] + (float)pe[c];
    return;
  }
  Pick p = pick_none();
  // kPer candidates per thread are loaded before any is merged: one memory round trip per
  // batch instead of one per candidate (the merge order does not change the result)
  constexpr int kPer = 16;
  for (int k0 = 0; k0 < parts; k0 += 256 * kPer) {
    Pick c[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int k = k0 + 256 * j + t;
      const size_t i = (size_t)b * parts + k;
      c[j] = k < parts ? Pick{pv1[i], pi1[i], pv2[i]} : pick_none();
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) p = pick_combine(p, c[j]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) p = pick_combine(p, pick_shfl_xor(p, off));
  if ((t & 63) == 0) s_wave[t >> 6] = p;
  __syncthreads();
  p = pick_combine(pick_combine(s_wave[0], s_wave[1]), pick_combine(s_wave[2], s_wave[3]));
  // A row with no comparable logit (all NaN) leaves no candidate's column: it picks column 0,
  // as std::max_element does, so the token and the embedding row below stay in range.
  const int pick = p.i1 >= 0 && p.i1 < V ? p.i1 : 0;
  // pos[b] is read by every thread before thread 0 advances it (after the barrier below)
  const int pos_old = pos[b];
  __syncthreads();
  if (t == 0) {
    // pos[b] is the position of the last token fed: prompt_len-1 for the pick after the
    // prompt (step 0), prompt_len-1+t for step t. The state lives on the device, so one
    // captured decode step replays for every t. (0 <= step < ctx while the host keeps
    // prompt + new tokens within the context; the token buffers hold ctx rows of n.)
    const int step = pos_old - (prompt_len[b] - 1);
    if (step >= 0 && step < ctx) {
      tokens[(size_t)step * n + b] = pick;
      margins[(size_t)step * n + b] = p.v1 - p.v2;
    }
    tok[b] = pick;
    pos[b] = pos_old + 1;
    cache_len[b] = pos_old + 2;
    // src/generate.cpp:131: the stop token ends the row, and so does its length limit
    // (pos_old + 2 tokens: the prompt and the picks so far, this one included)
    if (pick == rs.stop[b] || pos_old + 2 >= rs.limit[b]) {
      rs.done[b] = 1;
      atomicAdd(rs.ndone, 1);
    }
  }
  const int np = pos_old + 1;
  if (np >= 0 && np < ctx) {  // the input row of the step that feeds this pick
    const bf16* te = wte + (size_t)pick * d;
    const bf16* pe = wpe + (size_t)np * d;
    for (int c = t; c < d; c += 256) x[(size_t)b * d + c] = (float)te[c] + (float)pe[c];
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
                 const int* rowmap, int rows, int S, int d, hipStream_t s) {
  embed_kernel<<<rows, 256, 0, s>>>(x, tok, pos0, wte, wpe, rowmap, S, d);
  return hipGetLastError();
}

template <typename O>
hipError_t residual_layernorm(float* x, const float* y, const bf16* bias, O* out,
                              const bf16* w, const bf16* b, int rows, int d, hipStream_t s,
                              int splits, bool blocked) {
  if (d > 256 * kLnMaxPerThread) return hipErrorInvalidValue;
  if (blocked && (rows > kSkinnyRows || d % 32 != 0)) return hipErrorInvalidValue;
  residual_layernorm_kernel<O><<<rows, 256, 0, s>>>(x, y, bias, out, w, b, d, splits, blocked);
  return hipGetLastError();
}
template hipError_t residual_layernorm<bf16>(float*, const float*, const bf16*, bf16*,
                                             const bf16*, const bf16*, int, int, hipStream_t,
                                             int, bool);
template hipError_t residual_layernorm<float>(float*, const float*, const bf16*, float*,
                                              const bf16*, const bf16*, int, int, hipStream_t,
                                              int, bool);

template <typename T>
hipError_t qkv_split(T* qh, T* kh, T* vh, T* kcache, T* vcache, const float* qkv,
                     const float* bqkv, const int* pos0, const int* nvalid, const int* rowmap,
                     int rows, int S, int H, int dh, int max_len, hipStream_t s) {
  qkv_split_kernel<T><<<rows, 256, 0, s>>>(qh, kh, vh, kcache, vcache, qkv, bqkv, pos0, nvalid,
                                           rowmap, S, H, dh, max_len);
  return hipGetLastError();
}
template hipError_t qkv_split<bf16>(bf16*, bf16*, bf16*, bf16*, bf16*, const float*,
                                    const float*, const int*, const int*, const int*, int, int,
                                    int, int, int, hipStream_t);
template hipError_t qkv_split<float>(float*, float*, float*, float*, float*, const float*,
                                     const float*, const int*, const int*, const int*, int, int,
                                     int, int, int, hipStream_t);

template <typename T, typename O>
hipError_t merge_heads(O* out, const T* heads, const int* rowmap, int rows, int S, int H, int dh,
                       hipStream_t s) {
  merge_heads_kernel<T, O><<<rows, 256, 0, s>>>(out, heads, rowmap, S, H, dh);
  return hipGetLastError();
}
template hipError_t merge_heads<float, bf16>(bf16*, const float*, const int*, int, int, int,
                                             int, hipStream_t);
template hipError_t merge_heads<float, float>(float*, const float*, const int*, int, int, int,
                                              int, hipStream_t);

hipError_t to_f32(float* out, const bf16* in, size_t count, hipStream_t s) {
  to_f32_kernel<<<grid_for(count), 256, 0, s>>>(out, in, count);
  return hipGetLastError();
}

hipError_t to_bf16(bf16* out, const float* in, size_t count, hipStream_t s) {
  to_bf16_kernel<<<grid_for(count), 256, 0, s>>>(out, in, count);
  return hipGetLastError();
}

template <typename O>
hipError_t bias_gelu(O* out, const float* y, const bf16* bias, int rows, int cols,
                     hipStream_t s) {
  bias_gelu_kernel<O><<<grid_for((size_t)rows * cols), 256, 0, s>>>(out, y, bias, rows, cols);
  return hipGetLastError();
}
template hipError_t bias_gelu<bf16>(bf16*, const float*, const bf16*, int, int, hipStream_t);
template hipError_t bias_gelu<float>(float*, const float*, const bf16*, int, int, hipStream_t);

template <typename T>
hipError_t gather_rows(T* out, const T* in, const int* idx, int rows, int d, hipStream_t s) {
  gather_rows_kernel<T><<<rows, 256, 0, s>>>(out, in, idx, d);
  return hipGetLastError();
}
template hipError_t gather_rows<float>(float*, const float*, const int*, int, int, hipStream_t);
template hipError_t gather_rows<bf16>(bf16*, const bf16*, const int*, int, int, hipStream_t);

size_t pick_scratch_floats(int n, int parts) {
  return (size_t)3 * n * (parts > kPickParts ? parts : kPickParts);
}

hipError_t argmax_advance(int* tokens, float* margins, int* tok, int* pos, int* cache_len,
                          const int* prompt_len, RowStop rs, const float* logits,
                          float* scratch, int n, int V, float* x, const bf16* wte,
                          const bf16* wpe, int d, int ctx, hipStream_t s) {
  float* pv1 = scratch;
  int* pi1 = reinterpret_cast<int*>(scratch + (size_t)n * kPickParts);
  float* pv2 = scratch + (size_t)2 * n * kPickParts;
  pick_partial_kernel<<<dim3(n, kPickParts), 256, 0, s>>>(pv1, pi1, pv2, logits, V);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  pick_final_kernel<<<n, 256, 0, s>>>(tokens, margins, tok, pos, cache_len, prompt_len, rs, pv1,
                                      pi1, pv2, kPickParts, n, V, x, wte, wpe, d, ctx);
  return hipGetLastError();
}

hipError_t pick_advance(int* tokens, float* margins, int* tok, int* pos, int* cache_len,
                        const int* prompt_len, RowStop rs, const float* cand, int parts,
                        int rows, int n, int V, float* x, const bf16* wte, const bf16* wpe,
                        int d, int ctx, hipStream_t s) {
  const float* pv1 = cand;
  const int* pi1 = reinterpret_cast<const int*>(cand + (size_t)rows * parts);
  const float* pv2 = cand + (size_t)2 * rows * parts;
  pick_final_kernel<<<n, 256, 0, s>>>(tokens, margins, tok, pos, cache_len, prompt_len, rs, pv1,
                                      pi1, pv2, parts, n, V, x, wte, wpe, d, ctx);
  return hipGetLastError();
}

hipError_t pack_bias(float* bqkv, const bf16* bq, const bf16* bk, const bf16* bv, int d,
                     hipStream_t s) {
  pack_bias_kernel<<<grid_for(d), 256, 0, s>>>(bqkv, bq, bk, bv, d);
  return hipGetLastError();
}

}  // namespace dadgpt::gen
