// KV-cache decode attention for gfx950: one query token per (sequence, head) against a
// ragged cache. Replaces the per-head GEMV chain of model_forward_cached
// (src/model.cpp:758-790: q K^T, *scale, softmax, P V) with one launch for all sequences and
// heads. Decode is a GEMV: it is bound by HBM, so it uses no MFMA.
//
// Cache layout [n_seq, H, max_len, D] (for n_seq = 1 this is the reference's per-layer
// [H, max_len, d_head] cache, src/model.cpp:659-675); only the first lens[s] rows are read.
//
// One workgroup of 16 waves covers a span of 16*KW keys of one (sequence, head): wave w owns
// keys [span0 + w*KW, span0 + (w+1)*KW). Every 16-byte load instruction of a wave covers whole
// key rows (for bf16 D=64: 8 lanes x 16 B per row, 8 rows per instruction, a contiguous 1 KiB),
// and all K and V loads of a wave are issued before any arithmetic, so a workgroup keeps its
// whole span in flight. The 16 waves merge (max, sum, o) in LDS with the logsumexp rule.
//
// Spans are 1024 keys (bf16) or 512 keys (fp32). When max_len fits one span, the workgroup
// writes the output directly: one kernel, no workspace, no inter-workgroup communication. A
// longer cache splits into n_split spans: each workgroup writes an fp32 partial
// (max, sum, unnormalised o) and a second kernel merges them. The kernel boundary orders the
// two; no device-scope fence is used (on this part an agent-scope release writes back the
// whole L2, because the L2s of the 8 XCDs are not coherent with each other).
#include "common.hpp"
#include "kernels.hpp"

namespace dadgpt {
namespace {

constexpr int kWaves = 16;

template <typename T>
struct Elem;
template <>
struct Elem<bf16> {
  static constexpr int kPer16B = 8;
  static constexpr int kKeysPerWave = 64;
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
  static constexpr int kKeysPerWave = 32;
  static __device__ __forceinline__ void unpack(const u32x4& w, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(w[i]);
  }
  static __device__ __forceinline__ float from(float x) { return x; }
};

template <typename T>
constexpr int span_keys() {
  return kWaves * Elem<T>::kKeysPerWave;
}

__device__ __forceinline__ int clamp_len(int L, int max_len) {
  return L < 0 ? 0 : (L > max_len ? max_len : L);
}

// part: [n_seq*H][n_split][D+2] fp32 (max in log2 units, sum, o[D]); used when n_split > 1.
template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves) void decode_kernel(
    T* __restrict__ out, const T* __restrict__ q, const T* __restrict__ kc,
    const T* __restrict__ vc, const int* __restrict__ lens, int H, int max_len,
    float scale_log2, float* __restrict__ part, int n_split) {
  constexpr int EPL = Elem<T>::kPer16B;       // elements per 16-byte load
  constexpr int KW = Elem<T>::kKeysPerWave;   // keys per wave
  constexpr int LPR = D / EPL;                // lanes per key row
  constexpr int KPL = 64 / LPR;               // key rows per wave-wide load
  constexpr int NLD = KW / KPL;               // loads per wave, per tensor
  __shared__ float sm_o[kWaves][D];
  __shared__ float sm_m[kWaves], sm_l[kWaves];

  const int seq = blockIdx.z, head = blockIdx.y, split = blockIdx.x;
  const int L = clamp_len(lens[seq], max_len);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane % LPR, grp = lane / LPR;
  const size_t hrow = (size_t)seq * H + head;
  const T* kh = kc + hrow * max_len * D + sub * EPL;
  const T* vh = vc + hrow * max_len * D + sub * EPL;
  const int key0 = split * span_keys<T>() + wave * KW;

  float mx = neg_inf(), lsum = 0.f;
  float o[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) o[e] = 0.f;

  if (key0 < L) {  // wave-uniform: waves past the length skip their loads
    // Rows past the length load row L-1 instead (valid, since key0 < L) and are masked out
    // below: the loads stay unconditional, so the compiler issues all of them back to back.
    u32x4 kr[NLD], vr[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int key = min(key0 + i * KPL + grp, L - 1);
      kr[i] = ld_g128u(kh + (size_t)key * D);
    }
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int key = min(key0 + i * KPL + grp, L - 1);
      vr[i] = ld_g128u(vh + (size_t)key * D);
    }
    float qf[EPL];
    Elem<T>::unpack(ld_g128u(q + hrow * D + sub * EPL), qf);
    // Keep the scheduler from sinking loads towards their uses: all of them stay in flight.
    __builtin_amdgcn_sched_barrier(0);

    // score of key key0 + i*KPL + grp: every lane of a row group ends with the full dot
    float s[NLD];
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
    // key0 < L, so key key0 is valid and mx is finite
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const float p = fast_exp2(s[i] - mx);  // exactly 0 for masked rows
      lsum += p;
      float vf[EPL];
      Elem<T>::unpack(vr[i], vf);
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[e] = fmaf(p, vf[e], o[e]);
    }
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) {
      lsum += __shfl_xor(lsum, off, 64);
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[e] += __shfl_xor(o[e], off, 64);
    }
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

  // merge the waves (threads 0..D-1 own one output column each)
  if (tid < D) {
    float wm = neg_inf(), wl = 0.f, wo = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wm = fmaxf(wm, sm_m[w]);
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = sm_m[w] == neg_inf() ? 0.f : fast_exp2(sm_m[w] - wm);
      wl += sm_l[w] * f;
      wo += sm_o[w][tid] * f;
    }
    if (n_split == 1) {
      out[hrow * D + tid] = Elem<T>::from(wl > 0.f ? wo / wl : 0.f);
    } else {
      float* my = part + (hrow * n_split + split) * (D + 2);
      my[2 + tid] = wo;
      if (tid == 0) {
        my[0] = wm;
        my[1] = wl;
      }
    }
  }
}

// One wave per (sequence, head): logsumexp merge of the n_split partials.
template <typename T, int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(T* __restrict__ out,
                                                           const float* __restrict__ part,
                                                           int rows, int n_split) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* ph = part + (size_t)row * n_split * (D + 2);
  float gm = neg_inf();
  for (int w = 0; w < n_split; ++w) gm = fmaxf(gm, ph[w * (D + 2)]);
  float gl = 0.f, go = 0.f;
  for (int w = 0; w < n_split; ++w) {
    const float* pw = ph + w * (D + 2);
    const float f = pw[0] == neg_inf() ? 0.f : fast_exp2(pw[0] - gm);
    gl += pw[1] * f;
    if (lane < D) go += pw[2 + lane] * f;
  }
  if (lane < D) out[(size_t)row * D + lane] = Elem<T>::from(gl > 0.f ? go / gl : 0.f);
}

template <typename T>
int n_split_for(int max_len) {
  return (max_len + span_keys<T>() - 1) / span_keys<T>();
}

template <typename T, int D>
hipError_t launch_decode_d(T* out, const T* q, const T* kc, const T* vc, const int* lens,
                           int n_seq, int H, int max_len, float scale, void* workspace,
                           hipStream_t stream) {
  const int ns = n_split_for<T>(max_len);
  float* part = static_cast<float*>(workspace);
  decode_kernel<T, D><<<dim3(ns, H, n_seq), 64 * kWaves, 0, stream>>>(
      out, q, kc, vc, lens, H, max_len, scale * kLog2e, part, ns);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || ns == 1) return e;
  const int rows = n_seq * H;
  decode_merge_kernel<T, D><<<(rows + 3) / 4, 256, 0, stream>>>(out, part, rows, ns);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_decode_t(T* out, const T* q, const T* kc, const T* vc, const int* lens,
                           int n_seq, int H, int max_len, int D, float scale, void* workspace,
                           hipStream_t stream) {
  if (D == 64)
    return launch_decode_d<T, 64>(out, q, kc, vc, lens, n_seq, H, max_len, scale, workspace,
                                  stream);
  if (D == 32)
    return launch_decode_d<T, 32>(out, q, kc, vc, lens, n_seq, H, max_len, scale, workspace,
                                  stream);
  return hipErrorInvalidValue;
}

}  // namespace

size_t decode_workspace_bytes(int n_seq, int H, int max_len, int D) {
  // fp32 spans are shorter, so the fp32 split count bounds the bf16 one: the size returned
  // serves both element types.
  const int ns = n_split_for<float>(max_len);
  if (ns == 1) return 0;
  return sizeof(float) * (size_t)n_seq * H * ns * (D + 2);
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
