// KV-cache decode attention for gfx950: one query token per (sequence, head) against a
// ragged cache, split along the keys so every CU streams. Replaces the per-head GEMV chain of
// model_forward_cached (src/model.cpp:758-790: q K^T, *scale, softmax, P V) with one launch
// for all sequences and heads.
//
// Cache layout [n_seq, H, max_len, D] (for n_seq = 1 this is the reference's per-layer
// [H, max_len, d_head] cache, src/model.cpp:659-675); only the first lens[s] rows are read.
//
// Grid (ceil(max_len/256), H, n_seq); a workgroup is 4 waves x 64 keys. Workgroups past a
// sequence's length return at once. Within a wave, each 16-byte load instruction covers
// whole key rows (8 lanes x 16 B per bf16 row of 64), so every load is a fully used 1 KiB
// contiguous read; all K and V loads of the chunk are issued before any arithmetic. The
// 4 waves merge in LDS; when a sequence needs several workgroups, each writes an fp32
// partial (max, sum, unnormalised o) and the last to arrive — counted with an agent-scope
// atomic — merges them with the logsumexp rule and resets the counter to zero.
#include "common.hpp"
#include "kernels.hpp"

namespace dadgpt {
namespace {

constexpr int kChunk = 64;            // keys per wave
constexpr int kWaves = 4;             // waves per workgroup
constexpr int kWgKeys = kChunk * kWaves;

template <typename T>
struct Elem;
template <>
struct Elem<bf16> {
  static constexpr int kPer16B = 8;
  static __device__ __forceinline__ void unpack(const u32x4& w, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf16_lo(w[i]);
      f[2 * i + 1] = bf16_hi(w[i]);
    }
  }
  static __device__ __forceinline__ bf16 from(float x) { return static_cast<bf16>(x); }
};
template <>
struct Elem<float> {
  static constexpr int kPer16B = 4;
  static __device__ __forceinline__ void unpack(const u32x4& w, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(w[i]);
  }
  static __device__ __forceinline__ float from(float x) { return x; }
};

template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves) void decode_kernel(
    T* __restrict__ out, const T* __restrict__ q, const T* __restrict__ kc,
    const T* __restrict__ vc, const int* __restrict__ lens, int H, int max_len,
    float scale_log2, float* __restrict__ part, unsigned* __restrict__ counters, int n_wg_max) {
  constexpr int EPL = Elem<T>::kPer16B;  // elements per 16-byte load
  constexpr int LPR = D / EPL;           // lanes per key row
  constexpr int KPL = 64 / LPR;          // key rows per wave-wide load
  constexpr int NLD = kChunk / KPL;      // loads per chunk
  __shared__ float sm_o[kWaves][D];
  __shared__ float sm_m[kWaves], sm_l[kWaves];
  __shared__ int sm_last;

  const int seq = blockIdx.z, head = blockIdx.y, wg = blockIdx.x;
  int L = lens[seq];
  L = L < 0 ? 0 : (L > max_len ? max_len : L);
  const int n_wg = max(1, (L + kWgKeys - 1) / kWgKeys);
  if (wg >= n_wg) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane % LPR, grp = lane / LPR;
  const size_t hrow = (size_t)seq * H + head;
  const T* kh = kc + hrow * max_len * D + sub * EPL;
  const T* vh = vc + hrow * max_len * D + sub * EPL;
  const int key0 = wg * kWgKeys + wave * kChunk;

  u32x4 kr[NLD], vr[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    const int key = key0 + i * KPL + grp;
    kr[i] = u32x4{0, 0, 0, 0};
    if (key < L) kr[i] = ld_g128u(kh + (size_t)key * D);
  }
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    const int key = key0 + i * KPL + grp;
    vr[i] = u32x4{0, 0, 0, 0};
    if (key < L) vr[i] = ld_g128u(vh + (size_t)key * D);
  }
  float qf[EPL];
  Elem<T>::unpack(ld_g128u(q + hrow * D + sub * EPL), qf);

  // scores of keys key0 + i*KPL + grp (every lane of a row group ends with the full dot)
  float s[NLD];
  float mx = neg_inf();
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    float kf[EPL];
    Elem<T>::unpack(kr[i], kf);
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc = fmaf(qf[e], kf[e], acc);
#pragma unroll
    for (int off = 1; off < LPR; off <<= 1) acc += __shfl_xor(acc, off, 64);
    const int key = key0 + i * KPL + grp;
    s[i] = key < L ? acc * scale_log2 : neg_inf();
    mx = fmaxf(mx, s[i]);
  }
#pragma unroll
  for (int off = LPR; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));

  float lsum = 0.f;
  float o[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) o[e] = 0.f;
  if (mx != neg_inf()) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const float p = fast_exp2(s[i] - mx);
      lsum += p;
      float vf[EPL];
      Elem<T>::unpack(vr[i], vf);
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[e] = fmaf(p, vf[e], o[e]);
    }
  }
#pragma unroll
  for (int off = LPR; off < 64; off <<= 1) {
    lsum += __shfl_xor(lsum, off, 64);
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[e] += __shfl_xor(o[e], off, 64);
  }
  if (grp == 0) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) sm_o[wave][sub * EPL + e] = o[e];
  }
  if (lane == 0) {
    sm_m[wave] = mx;
    sm_l[wave] = lsum;
  }
  __syncthreads();

  // merge the waves of this workgroup (threads 0..D-1 own one output column each)
  float wm = neg_inf(), wl = 0.f, wo = 0.f;
  if (tid < D) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wm = fmaxf(wm, sm_m[w]);
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = sm_m[w] == neg_inf() ? 0.f : fast_exp2(sm_m[w] - wm);
      wl += sm_l[w] * f;
      wo += sm_o[w][tid] * f;
    }
  }
  if (n_wg == 1) {
    if (tid < D) out[hrow * D + tid] = Elem<T>::from(wl > 0.f ? wo / wl : 0.f);
    return;
  }

  float* my = part + (hrow * n_wg_max + wg) * (D + 2);
  if (tid < D) my[2 + tid] = wo;
  if (tid == 0) {
    my[0] = wm;
    my[1] = wl;
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = atomicAdd(&counters[hrow], 1u);
    sm_last = prev == (unsigned)(n_wg - 1);
  }
  __syncthreads();
  if (!sm_last) return;
  __threadfence();
  if (tid < D) {
    const float* ph = part + hrow * n_wg_max * (D + 2);
    float gm = neg_inf();
    for (int w = 0; w < n_wg; ++w) gm = fmaxf(gm, ph[w * (D + 2)]);
    float gl = 0.f, go = 0.f;
    for (int w = 0; w < n_wg; ++w) {
      const float* pw = ph + w * (D + 2);
      const float f = pw[0] == neg_inf() ? 0.f : fast_exp2(pw[0] - gm);
      gl += pw[1] * f;
      go += pw[2 + tid] * f;
    }
    out[hrow * D + tid] = Elem<T>::from(gl > 0.f ? go / gl : 0.f);
  }
  if (tid == 0) atomicExch(&counters[hrow], 0u);
}

int n_wg_max_for(int max_len) { return (max_len + kWgKeys - 1) / kWgKeys; }

template <typename T>
hipError_t launch_decode_t(T* out, const T* q, const T* kc, const T* vc, const int* lens,
                           int n_seq, int H, int max_len, int D, float scale, void* workspace,
                           hipStream_t stream) {
  const int nw = n_wg_max_for(max_len);
  float* part = static_cast<float*>(workspace);
  unsigned* counters = reinterpret_cast<unsigned*>(part + (size_t)n_seq * H * nw * (D + 2));
  const dim3 grid(nw, H, n_seq);
  const float sl2 = scale * kLog2e;
  if (D == 64)
    decode_kernel<T, 64><<<grid, 64 * kWaves, 0, stream>>>(out, q, kc, vc, lens, H, max_len, sl2,
                                                           part, counters, nw);
  else if (D == 32)
    decode_kernel<T, 32><<<grid, 64 * kWaves, 0, stream>>>(out, q, kc, vc, lens, H, max_len, sl2,
                                                           part, counters, nw);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace

size_t decode_workspace_bytes(int n_seq, int H, int max_len, int D) {
  const size_t nw = (size_t)n_wg_max_for(max_len);
  return sizeof(float) * (size_t)n_seq * H * nw * (D + 2) + sizeof(unsigned) * (size_t)n_seq * H;
}

hipError_t launch_decode_bf16(bf16* out, const bf16* q, const bf16* k_cache,
                              const bf16* v_cache, const int* lens, int n_seq, int H,
                              int max_len, int D, float scale, void* workspace,
                              hipStream_t stream) {
  return launch_decode_t<bf16>(out, q, k_cache, v_cache, lens, n_seq, H, max_len, D, scale,
                               workspace, stream);
}

hipError_t launch_decode_f32(float* out, const float* q, const float* k_cache,
                             const float* v_cache, const int* lens, int n_seq, int H,
                             int max_len, int D, float scale, void* workspace,
                             hipStream_t stream) {
  return launch_decode_t<float>(out, q, k_cache, v_cache, lens, n_seq, H, max_len, D, scale,
                                workspace, stream);
}

}  // namespace dadgpt
