// A C++ caller of libdadgpt_gen without PyTorch: the process's HIP runtime is the ROCm
// installation's own (7.2), under the hipBLASLt the library opens. Checks that this pair is
// accepted, that a handle is created, and that a bf16 GEMM (gpu_matmul's replacement,
// cuda/gpu_ops.cu:94-98) matches a CPU product of the same bf16 values. Built with g++ and run
// on a GPU by tests/test_gpu_materialized.py.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "dadgpt/gpu_matmul.h"

static uint16_t to_bf16(float x) {  // round to nearest even (finite inputs)
  uint32_t u;
  std::memcpy(&u, &x, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static float from_bf16(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float x;
  std::memcpy(&x, &u, 4);
  return x;
}

int main() {
  int rt = 0, lt = 0;
  if (dadgpt_blas_stack_versions(&rt, &lt) != 0) {
    std::printf("FAILED versions: %s\n", dadgpt_gen_last_error());
    return 1;
  }
  std::printf("hip runtime %d, hipblaslt %d\n", rt, lt);
  if (rt / 10000000 != 7 || rt / 100000 % 100 != 2 || !dadgpt_blas_stack_supported(rt, lt)) {
    std::printf("FAILED: expected the ROCm 7.2 runtime, accepted\n");
    return 1;
  }
  dadgpt_blas* h = nullptr;
  if (dadgpt_blas_create(&h) != 0) {
    std::printf("FAILED create: %s\n", dadgpt_gen_last_error());
    return 1;
  }
  const int M = 37, K = 96, N = 50;
  std::vector<uint16_t> a(M * K), b(K * N);
  for (int i = 0; i < M * K; ++i) a[i] = to_bf16(std::sin(0.37f * i));
  for (int i = 0; i < K * N; ++i) b[i] = to_bf16(std::cos(0.11f * i));
  uint16_t *da, *db;
  float* dout;
  if (hipMalloc(&da, a.size() * 2) != hipSuccess || hipMalloc(&db, b.size() * 2) != hipSuccess ||
      hipMalloc(&dout, (size_t)M * N * 4) != hipSuccess ||
      hipMemcpy(da, a.data(), a.size() * 2, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(db, b.data(), b.size() * 2, hipMemcpyHostToDevice) != hipSuccess) {
    std::printf("FAILED: device buffers\n");
    return 1;
  }
  if (dadgpt_matmul_bf16(h, dout, da, db, M, K, N, nullptr) != 0) {
    std::printf("FAILED matmul: %s\n", dadgpt_gen_last_error());
    return 1;
  }
  std::vector<float> out((size_t)M * N);
  if (hipMemcpy(out.data(), dout, out.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) {
    std::printf("FAILED: copy back\n");
    return 1;
  }
  double worst = 0.0;
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < N; ++j) {
      double ref = 0.0;
      for (int k = 0; k < K; ++k) ref += (double)from_bf16(a[i * K + k]) * from_bf16(b[k * N + j]);
      worst = std::fmax(worst, std::fabs(ref - out[(size_t)i * N + j]));
    }
  dadgpt_blas_destroy(h);
  (void)hipFree(da);
  (void)hipFree(db);
  (void)hipFree(dout);
  std::printf("max |gpu - cpu| %.3g\n", worst);
  if (!(worst <= 1e-4 * std::sqrt((double)K))) {
    std::printf("FAILED: GEMM differs\n");
    return 1;
  }
  std::printf("OK\n");
  return 0;
}
