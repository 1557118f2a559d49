// KV-cache decode attention for gfx950: one query token per (sequence, head) against a
// ragged cache. Replaces the per-head GEMV chain of model_forward_cached
// (src/model.cpp:758-790: q K^T, *scale, softmax, P V) with one launch for all sequences and
// heads. Decode is a GEMV: it is bound by HBM, so it uses no MFMA.
//
// Cache layout [n_seq, H, max_len, D] (for n_seq = 1 this is the reference's per-layer
// [H, max_len, d_head] cache, src/model.cpp:659-675); only the first lens[s] rows are read.
//
// Work split. A cache (one sequence and head) is cut into chunks of C = 8*KW keys, one 8-wave
// workgroup per chunk; wave w owns keys [chunk*C + w*KW, chunk*C + (w+1)*KW). Every 16-byte
// load instruction of a wave covers whole key rows (bf16 D=64: 8 lanes x 16 B per row, 8 rows
// per instruction, a contiguous 1 KiB), all K and V loads of a wave are issued before any
// arithmetic, and they carry the non-temporal hint (the cache is streamed once). bf16 scores
// are v_dot2_f32_bf16 on the packed q and K words, so neither side is unpacked; the
// reductions across lanes use DPP and v_permlane16/32_swap (lanes.hpp), not LDS round trips. The 8 waves
// merge (max, sum, o) in LDS with the logsumexp rule. Chunks are small enough that the work
// of a long cache spreads over several CUs: one CU streaming a whole 1024-key cache alone was
// the tail of the launch.
//
// The grid runs over caches fastest, so consecutive workgroups (dealt round-robin to the 8
// XCDs) hold the same chunk index of different caches, and the chunks past a short cache's
// length (which exit at once) do not pile up on one XCD.
//
// A cache that fits one chunk is written directly. A longer one merges inside the same kernel:
// each chunk publishes an fp32 partial (max in log2 units, sum, unnormalised o) and counts
// itself on a per-cache counter; the chunk that arrives last merges all partials, writes the
// output and rearms the counter to zero.
//
// Ordering of that merge. The partials and the counter move only through agent-scope relaxed
// atomic accesses, and the rules that make this correct are those of the AMDGPU memory model
// for gfx942/gfx950 (LLVM AMDGPUUsage, "Memory Model GFX942"): a monotonic agent-scope atomic
// store, load or read-modify-write is a global_store / global_load / global_atomic with sc1 = 1,
// which is coherent across the 8 XCDs on its own (it bypasses the XCD-local L2), and
// s_waitcnt vmcnt(0) after a store waits for the store to complete. The publish sequence
// (sc1 stores, vmcnt(0), sc1 atomic increment; the last arriver reads with sc1 loads) is
// the compiler's agent-scope release / acquire sequence without its L2 writeback and
// invalidate, which only plain (non-sc1) accesses need. A release fence here writes back the
// whole L2, which made the first fence-based version of this kernel 17x slower. Other targets
// compile the standard release / acquire pair (DADGPT_DECODE_SC1_COHERENT below).
#include <mutex>

#include "common.hpp"
#include "kernels.hpp"
#include "lanes.hpp"

#if defined(__gfx942__) || defined(__gfx950__) || !defined(__HIP_DEVICE_COMPILE__)
#define DADGPT_DECODE_SC1_COHERENT 1
#else
#define DADGPT_DECODE_SC1_COHERENT 0
#endif

namespace dadgpt {
namespace {

constexpr int kWaves = 8;         // waves per workgroup (one chunk)
constexpr int kLoadsPerWave = 8;  // 16-byte loads per lane and tensor

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
  // q . k over the 8 bf16 pairs of two 16-byte words: four v_dot2_f32_bf16 on the packed
  // operands (bf16 products are exact in fp32), with no unpacking of either side.
  static __device__ __forceinline__ float dot(const u32x4& q, const u32x4& k) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t qi = q[i], ki = k[i];
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, qi),
                                            __builtin_bit_cast(bf16x2, ki), acc, false);
    }
    return acc;
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
  static __device__ __forceinline__ float dot(const u32x4& q, const u32x4& k) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = fmaf(__uint_as_float(q[i]), __uint_as_float(k[i]), acc);
    return acc;
  }
  static __device__ __forceinline__ float from(float x) { return x; }
};

// Keys per wave: kLoadsPerWave wave-wide loads of 64 x 16 B, each covering whole key rows.
// bf16: 64 keys (D=64) or 128 (D=32); fp32: 32 or 64.
template <typename T, int D>
__host__ __device__ constexpr int keys_per_wave() {
  return kLoadsPerWave * 64 / (D / Elem<T>::kPer16B);
}
template <typename T, int D>
__host__ __device__ constexpr int chunk_keys() {
  return kWaves * keys_per_wave<T, D>();
}

__device__ __forceinline__ int clamp_len(int L, int max_len) {
  return L < 0 ? 0 : (L > max_len ? max_len : L);
}

// Cache rows are read once: non-temporal loads.
__device__ __forceinline__ u32x4 ld_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Agent-scope relaxed accesses: each is coherent across the XCDs by itself.
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workspace of a split decode: one uint32 arrival counter per (sequence, head) from the start
// (the region rounded up to 256 bytes), and the fp32 partials [n_seq*H][n_chunk][D+2] packed
// against the END of the caller's buffer. A buffer sized for the largest shape it serves thus
// never has a later call's partials over any counter of a call of another shape, and the
// counters, rearmed by every call, stay zero between calls.
size_t counter_bytes(int n_seq, int H) {
  return (sizeof(unsigned) * (size_t)n_seq * H + 255) & ~(size_t)255;
}
size_t partial_bytes(int n_seq, int H, int n_chunk, int D) {
  return sizeof(float) * (size_t)n_seq * H * n_chunk * (D + 2);
}

template <typename T, int D>
__global__ __launch_bounds__(64 * kWaves) void decode_kernel(
    T* __restrict__ out, const T* __restrict__ q, const T* __restrict__ kc,
    const T* __restrict__ vc, const int* __restrict__ lens, int H, int max_len,
    float scale_log2, float* __restrict__ part, unsigned* __restrict__ counter, int n_chunk) {
  constexpr int EPL = Elem<T>::kPer16B;       // elements per 16-byte load
  constexpr int KW = keys_per_wave<T, D>();   // keys per wave
  constexpr int C = chunk_keys<T, D>();       // keys per workgroup
  constexpr int LPR = D / EPL;                // lanes per key row
  constexpr int KPL = 64 / LPR;               // key rows per wave-wide load
  constexpr int NLD = kLoadsPerWave;          // loads per wave, per tensor
  __shared__ float sm_o[kWaves][D];
  __shared__ float sm_m[kWaves], sm_l[kWaves];
  __shared__ int sm_last;

  const int seq = blockIdx.x / H, head = blockIdx.x % H, chunk = blockIdx.y;
  const int L = clamp_len(lens[seq], max_len);
  const int nch = (L + C - 1) / C;
  // Chunks past the length do nothing; chunk 0 of an empty cache still writes the zero output.
  if (chunk >= (nch > 1 ? nch : 1)) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane % LPR, grp = lane / LPR;
  const size_t hrow = (size_t)seq * H + head;
  const T* kh = kc + hrow * max_len * D + sub * EPL;
  const T* vh = vc + hrow * max_len * D + sub * EPL;
  const int key0 = chunk * C + wave * KW;

  float mx = neg_inf(), lsum = 0.f;
  float o[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) o[e] = 0.f;

  if (key0 < L) {  // wave-uniform: waves past the length skip their loads
    // q first (it is small and read by every chunk of the cache), kept packed.
    const u32x4 qw = ld_g128u(q + hrow * D + sub * EPL);
    // Rows past the length load row L-1 instead (valid, since key0 < L) and are masked out
    // below: the loads stay unconditional, so the compiler issues all of them back to back.
    u32x4 kr[NLD], vr[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int key = min(key0 + i * KPL + grp, L - 1);
      kr[i] = ld_stream(kh + (size_t)key * D);
    }
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int key = min(key0 + i * KPL + grp, L - 1);
      vr[i] = ld_stream(vh + (size_t)key * D);
    }
    // Keep the scheduler from sinking loads towards their uses: all of them stay in flight.
    __builtin_amdgcn_sched_barrier(0);

    // score of key key0 + i*KPL + grp: every lane of a row group ends with the full dot
    float s[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const float acc = lanes::group_sum<LPR>(Elem<T>::dot(qw, kr[i]));
      const int key = key0 + i * KPL + grp;
      s[i] = key < L ? acc * scale_log2 : neg_inf();
      mx = fmaxf(mx, s[i]);
    }
    mx = lanes::wave_max_of_groups<LPR>(mx);  // uniform within each row group already
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
    // sum over the row groups: lanes with the same column slice (lane % LPR) are partners
    if constexpr (LPR < 8) {
      lsum += __shfl_xor(lsum, LPR, 64);
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[e] += __shfl_xor(o[e], LPR, 64);
    }
    constexpr int K0 = LPR < 8 ? 8 : LPR;
    lsum = lanes::sum_across<K0>(lsum);
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[e] = lanes::sum_across<K0>(o[e]);
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
  if (nch <= 1) {  // the whole cache is this chunk
    if (tid < D) out[hrow * D + tid] = Elem<T>::from(wl > 0.f ? wo / wl : 0.f);
    return;
  }

  // Split cache: publish this chunk's partial; the last chunk to arrive merges all of them.
  float* ph = part + hrow * n_chunk * (D + 2);
  if (tid < D) {
    float* my = ph + chunk * (D + 2);
    st_agent(my + 2 + tid, wo);
    if (tid == 0) {
      st_agent(my, wm);
      st_agent(my + 1, wl);
    }
  }
#if DADGPT_DECODE_SC1_COHERENT
  // This thread's stores are complete at the device coherence point (the asm is also a
  // compiler barrier for them); the barrier then covers the whole workgroup's.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const unsigned before = __hip_atomic_fetch_add(counter + hrow, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
    sm_last = before == (unsigned)(nch - 1);
  }
#else
  __syncthreads();
  if (tid == 0) {
    const unsigned before = __hip_atomic_fetch_add(counter + hrow, 1u, __ATOMIC_ACQ_REL,
                                                   __HIP_MEMORY_SCOPE_AGENT);
    sm_last = before == (unsigned)(nch - 1);
  }
#endif
  __syncthreads();
  if (!sm_last) return;

  if (tid < D) {
    // The partials of kMergeBatch chunks are all loaded before any is used (one memory round
    // trip per batch: this merge ends the kernel for the caches that finish last), and the
    // batches merge online. Every chunk < nch holds a valid key: finite maxima. For
    // nch <= kMergeBatch this is sum_c l_c 2^(m_c - max) in chunk order, as a two-pass merge.
    constexpr int kMergeBatch = 4;
    float gm = neg_inf(), gl = 0.f, go = 0.f;
    for (int c0 = 0; c0 < nch; c0 += kMergeBatch) {
      float mv[kMergeBatch], lv[kMergeBatch], ov[kMergeBatch];
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) {
        const float* pc = ph + min(c0 + j, nch - 1) * (D + 2);  // past nch: unused
        mv[j] = ld_agent(pc);
        lv[j] = ld_agent(pc + 1);
        ov[j] = ld_agent(pc + 2 + tid);
      }
      float bm = gm;
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j)
        if (c0 + j < nch) bm = fmaxf(bm, mv[j]);
      const float fo = fast_exp2(gm - bm);  // 0 before the first batch (gl = go = 0 then)
      gl *= fo;
      go *= fo;
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j)
        if (c0 + j < nch) {
          const float f = fast_exp2(mv[j] - bm);
          gl += lv[j] * f;
          go += ov[j] * f;
        }
      gm = bm;
    }
    out[hrow * D + tid] = Elem<T>::from(go / gl);
  }
  // All nch arrivals of this call are in: rearm the counter for the next call.
  if (tid == 0)
    __hip_atomic_store(counter + hrow, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T, int D>
int n_chunk_for(int max_len) {
  return (max_len + chunk_keys<T, D>() - 1) / chunk_keys<T, D>();
}

template <typename T, int D>
hipError_t launch_decode_d(T* out, const T* q, const T* kc, const T* vc, const int* lens,
                           int n_seq, int H, int max_len, float scale, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  const int nc = n_chunk_for<T, D>(max_len);
  float* part = nullptr;
  unsigned* counter = nullptr;
  if (nc > 1) {
    // the caller checked workspace_bytes >= decode_workspace_bytes(), which bounds both regions
    const size_t at = (workspace_bytes - partial_bytes(n_seq, H, nc, D)) & ~(size_t)15;
    counter = static_cast<unsigned*>(workspace);
    part = reinterpret_cast<float*>(static_cast<char*>(workspace) + at);
  }
  decode_kernel<T, D><<<dim3(n_seq * H, nc), 64 * kWaves, 0, stream>>>(
      out, q, kc, vc, lens, H, max_len, scale * kLog2e, part, counter, nc);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_decode_t(T* out, const T* q, const T* kc, const T* vc, const int* lens,
                           int n_seq, int H, int max_len, int D, float scale, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  if (D == 64)
    return launch_decode_d<T, 64>(out, q, kc, vc, lens, n_seq, H, max_len, scale, workspace,
                                  workspace_bytes, stream);
  if (D == 32)
    return launch_decode_d<T, 32>(out, q, kc, vc, lens, n_seq, H, max_len, scale, workspace,
                                  workspace_bytes, stream);
  return hipErrorInvalidValue;
}

// Scratch of the allocation-free entry point: it stands in for a caller's workspace (same
// layout: counters at the start, partials against the end) and lives as long as the code
// object, one copy per device. In host code `scratch` names a host-side shadow, not device
// memory: only the address hipGetSymbolAddress returns for the current device may reach a
// kernel or a copy.
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

__global__ void zero_words_kernel(unsigned* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

}  // namespace

hipError_t decode_scratch(void** ptr, hipStream_t stream) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = -1;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    // The arrival counters must start at zero (every call leaves them at zero again). A fill
    // kernel, not a memset node, so that a first call made under graph capture replays right.
    zero_words_kernel<<<256, 256, 0, stream>>>(static_cast<unsigned*>(p),
                                               kDecodeScratchBytes / sizeof(unsigned));
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    addr[dev] = p;
  }
  *ptr = addr[dev];
  return hipSuccess;
}

size_t decode_workspace_bytes(int n_seq, int H, int max_len, int D) {
  // fp32 chunks are shorter, so the fp32 chunk count bounds the bf16 one: the size returned
  // serves both element types.
  const int nc = D == 64 ? n_chunk_for<float, 64>(max_len) : n_chunk_for<float, 32>(max_len);
  if (nc == 1) return 0;
  return counter_bytes(n_seq, H) + partial_bytes(n_seq, H, nc, D);
}

hipError_t launch_decode_bf16(bf16* out, const bf16* q, const bf16* k_cache,
                              const bf16* v_cache, const int* lens, int n_seq, int H,
                              int max_len, int D, float scale, void* workspace,
                              size_t workspace_bytes, hipStream_t stream) {
  return launch_decode_t<bf16>(out, q, k_cache, v_cache, lens, n_seq, H, max_len, D, scale,
                               workspace, workspace_bytes, stream);
}

hipError_t launch_decode_f32(float* out, const float* q, const float* k_cache,
                             const float* v_cache, const int* lens, int n_seq, int H,
                             int max_len, int D, float scale, void* workspace,
                             size_t workspace_bytes, hipStream_t stream) {
  return launch_decode_t<float>(out, q, k_cache, v_cache, lens, n_seq, H, max_len, D, scale,
                                workspace, workspace_bytes, stream);
}

}  // namespace dadgpt
