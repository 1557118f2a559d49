// The reference's matmul wrappers under their own C++ names (declared in
// <dadgpt/gpu_ops_matmul.hpp>), over the C ABI of <dadgpt/gpu_matmul.h>. Each call launches on
// the null stream and throws std::runtime_error on failure, as CUBLAS_CHECK does
// (cuda/gpu_ops.cuh:19-26).
#include <stdexcept>
#include <string>

#include "dadgpt/gpu_attention.h"
#include "dadgpt/gpu_matmul.h"
#include "dadgpt/gpu_ops_matmul.hpp"

namespace {
void throw_if(int status) {
  if (status != DADGPT_OK)
    throw std::runtime_error(std::string("hipBLASLt error: ") + dadgpt_gen_last_error());
}
}  // namespace

void gpu_set_matmul_precision(MatmulPrecision p) {
  throw_if(dadgpt_set_matmul_precision(p == MatmulPrecision::BF16   ? DADGPT_MATMUL_BF16
                                       : p == MatmulPrecision::TF32 ? DADGPT_MATMUL_TF32
                                                                    : DADGPT_MATMUL_FP32));
}

void gpu_matmul(gpu_blas_handle handle, float* out, const float* a, const float* b, int M, int K,
                int N) {
  throw_if(dadgpt_matmul_f32(handle, out, a, b, M, K, N, 'N', 0.0f, nullptr));
}

void gpu_matmul_transposed_a(gpu_blas_handle handle, float* out, const float* a, const float* b,
                             int M, int K, int N, bool accumulate) {
  throw_if(dadgpt_matmul_f32(handle, out, a, b, M, K, N, 'A', accumulate ? 1.0f : 0.0f, nullptr));
}

void gpu_matmul_transposed_b(gpu_blas_handle handle, float* out, const float* a, const float* b,
                             int M, int K, int N) {
  throw_if(dadgpt_matmul_f32(handle, out, a, b, M, K, N, 'B', 0.0f, nullptr));
}

void gpu_matmul_strided_batched_bt(gpu_blas_handle handle, float* out, const float* a,
                                   const float* b, int M, int K, int N, long long strideA,
                                   long long strideB, long long strideC, int batch_count) {
  throw_if(dadgpt_matmul_f32_strided_batched(handle, out, a, b, M, K, N, 'B', 0.0f, strideA,
                                             strideB, strideC, batch_count, nullptr));
}

void gpu_matmul_strided_batched(gpu_blas_handle handle, float* out, const float* a, const float* b,
                                int M, int K, int N, long long strideA, long long strideB,
                                long long strideC, int batch_count) {
  throw_if(dadgpt_matmul_f32_strided_batched(handle, out, a, b, M, K, N, 'N', 0.0f, strideA,
                                             strideB, strideC, batch_count, nullptr));
}

void gpu_matmul_strided_batched_at(gpu_blas_handle handle, float* out, const float* a,
                                   const float* b, int M, int K, int N, long long strideA,
                                   long long strideB, long long strideC, int batch_count) {
  throw_if(dadgpt_matmul_f32_strided_batched(handle, out, a, b, M, K, N, 'A', 1.0f, strideA,
                                             strideB, strideC, batch_count, nullptr));
}
