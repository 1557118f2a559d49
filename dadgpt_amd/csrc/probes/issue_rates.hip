// Issue-rate probe for gfx950: how much of the MFMA pipe the attention forward's instruction mix
// can keep busy, independent of memory. Every kernel runs a register-only loop; per iteration:
//
//   mfma     8 independent v_mfma_f32_32x32x16_bf16 (the score and P.V products of one
//            32-key chunk of the forward: 4 + 4)
//   valu     the chunk's softmax work on 16 scores per lane: 16 FMA (scale and running max),
//            16 v_exp_f32, 16 adds (row sum) and 8 bf16 packs
//   mix      both in one wave, with no dependence between them
//   chain    both with the forward's dependences: scores from the first 4 MFMAs feed the
//            exponentials, whose packed bf16 values are the B operand of the last 4
//
// Each kernel is launched with 2, 4 and 8 waves per SIMD (1024 SIMDs on MI355X; the grid is
// sized from the device's CU count) and timed with HIP events over 5 launches; the table gives
// nanoseconds per iteration per SIMD and the MFMA pipe's busy fraction implied by the mfma-only
// time. No global memory is touched except one store per lane at the end.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kIters = 1024;
enum Mode { kMfma, kValu, kMix, kChain };

__device__ __forceinline__ unsigned pack(float a, float b) {
  const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(unsigned, v);
}

template <int MODE>
__global__ __launch_bounds__(256) void probe(float* out, float seed, float c) {
  bf16x8 ka[4], qa[4], va[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ka[i][e] = static_cast<__bf16>(seed * (threadIdx.x + e + i));
      qa[i][e] = static_cast<__bf16>(seed * (e - i));
      va[i][e] = static_cast<__bf16>(seed * (threadIdx.x - e));
    }
  f32x16 acc[4] = {};
  float xs[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) xs[r] = seed * r;
  float l = 0.f;
  const float m = seed;
  for (int it = 0; it < kIters; ++it) {
    f32x16 s = {};
    if constexpr (MODE == kMfma || MODE == kMix) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[i], qa[i], acc[i], 0, 0, 0);
    } else if constexpr (MODE == kChain) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[i], qa[i], s, 0, 0, 0);
    }
    u32x4 w0 = {}, w1 = {};
    if constexpr (MODE != kMfma) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r)
        p[r] = __builtin_amdgcn_exp2f(fmaf(MODE == kChain ? s[r] : xs[r], c, -m));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        w0[e] = pack(p[2 * e], p[2 * e + 1]);
        w1[e] = pack(p[8 + 2 * e], p[9 + 2 * e]);
      }
      float ls = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) ls += p[r];
      l += ls;
      if constexpr (MODE != kChain) {
        // next iteration's inputs: keeps the VALU work live without tying it to the MFMAs
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          xs[r] = p[r];
          asm volatile("" : "+v"(xs[r]));
        }
        asm volatile("" ::"v"(w0), "v"(w1));
      }
    }
    if constexpr (MODE == kMfma || MODE == kMix) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[i], qa[(i + 1) & 3], acc[i], 0, 0, 0);
    } else if constexpr (MODE == kChain) {
      const bf16x8 pb0 = __builtin_bit_cast(bf16x8, w0), pb1 = __builtin_bit_cast(bf16x8, w1);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[0], pb0, acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[1], pb0, acc[1], 0, 0, 0);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[2], pb1, acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[3], pb1, acc[1], 0, 0, 0);
    }
  }
  float r = l;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) r += acc[i][j];
  out[blockIdx.x * 256 + threadIdx.x] = r;
}

bool ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return false;
}

}  // namespace

int main() {
  int dev = 0, cus = 0;
  if (!ok(hipGetDevice(&dev), "hipGetDevice") ||
      !ok(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "CU count"))
    return 1;
  const int simds = 4 * cus;
  float* out = nullptr;
  if (!ok(hipMalloc(&out, sizeof(float) * 256 * (size_t)cus * 8), "hipMalloc")) return 1;
  hipEvent_t e0, e1;
  if (!ok(hipEventCreate(&e0), "event") || !ok(hipEventCreate(&e1), "event")) return 1;
  const char* names[] = {"mfma", "valu", "mix", "chain"};
  std::printf("# ns per iteration per SIMD (%d SIMDs); mfma_busy = mfma-only time / this time\n",
              simds);
  std::printf("%-6s %8s %8s %8s   %s\n", "mode", "2 w/SIMD", "4 w/SIMD", "8 w/SIMD",
              "mfma_busy at 8 w/SIMD");
  double mfma8 = 0;
  for (int mode = 0; mode < 4; ++mode) {
    double t[3];
    for (int k = 0; k < 3; ++k) {
      const int wps = 2 << k, grid = cus * wps;  // 4 waves per workgroup, 4 SIMDs per CU
      float best = 1e30f;
      for (int rep = 0; rep < 6; ++rep) {
        ok(hipEventRecord(e0), "record");
        switch (mode) {
          case kMfma: probe<kMfma><<<grid, 256>>>(out, 0.01f, 0.18f); break;
          case kValu: probe<kValu><<<grid, 256>>>(out, 0.01f, 0.18f); break;
          case kMix: probe<kMix><<<grid, 256>>>(out, 0.01f, 0.18f); break;
          default: probe<kChain><<<grid, 256>>>(out, 0.01f, 0.18f); break;
        }
        if (!ok(hipGetLastError(), "launch")) return 1;
        ok(hipEventRecord(e1), "record");
        if (!ok(hipEventSynchronize(e1), "sync")) return 1;
        float ms = 0;
        ok(hipEventElapsedTime(&ms, e0, e1), "elapsed");
        if (rep > 0 && ms < best) best = ms;  // the first launch warms up
      }
      t[k] = best * 1e6 / ((double)wps * kIters);
    }
    if (mode == kMfma) mfma8 = t[2];
    std::printf("%-6s %8.1f %8.1f %8.1f   %.2f\n", names[mode], t[0], t[1], t[2], mfma8 / t[2]);
    if (mode == kMfma)  // 8 MFMAs of 32x32x16 (32768 flops each) per iteration per SIMD
      std::printf("#   mfma-only rate at 8 w/SIMD: %.0f TFLOP/s over %d SIMDs\n",
                  8.0 * 32768 * simds / (t[2] * 1e-9) / 1e12, simds);
  }
  return hipFree(out) == hipSuccess ? 0 : 1;
}
