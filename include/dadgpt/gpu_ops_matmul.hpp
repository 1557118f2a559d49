// The reference's matmul wrappers under their own names, argument order and C++ signatures
// (cuda/gpu_ops.cuh:40-54 and 84-96), defined in libdadgpt_gen.so over the C ABI of
// <dadgpt/gpu_matmul.h>. The cublasHandle_t parameter becomes gpu_blas_handle, the opaque
// hipBLASLt handle of dadgpt_blas_create. Operands are fp32 device pointers, row-major; the
// multiply precision is process-wide (gpu_set_matmul_precision), as in the reference.
// Launches go on the null stream. Errors throw std::runtime_error with the library's
// message, as CUBLAS_CHECK does (cuda/gpu_ops.cuh:19-26).
#pragma once

#include "dadgpt/gpu_matmul.h"

using gpu_blas_handle = dadgpt_blas*;

// cuda/gpu_ops.cuh:40-44. TF32 multiplies in fp32 on gfx950 (no TF32 format).
enum class MatmulPrecision { FP32, TF32, BF16 };
void gpu_set_matmul_precision(MatmulPrecision p);

// cuda/gpu_ops.cuh:46-48: out[M,N] = a[M,K] b[K,N]
void gpu_matmul(gpu_blas_handle handle, float* out, const float* a, const float* b, int M, int K,
                int N);
// cuda/gpu_ops.cuh:49-51: out = a^T b (a [K,M]), or out += a^T b when accumulate
void gpu_matmul_transposed_a(gpu_blas_handle handle, float* out, const float* a, const float* b,
                             int M, int K, int N, bool accumulate = false);
// cuda/gpu_ops.cuh:52-54: out = a b^T (b [N,K])
void gpu_matmul_transposed_b(gpu_blas_handle handle, float* out, const float* a, const float* b,
                             int M, int K, int N);

// cuda/gpu_ops.cuh:84-88: out[i] = a[i] b[i]^T
void gpu_matmul_strided_batched_bt(gpu_blas_handle handle, float* out, const float* a,
                                   const float* b, int M, int K, int N, long long strideA,
                                   long long strideB, long long strideC, int batch_count);
// cuda/gpu_ops.cuh:89-92: out[i] = a[i] b[i]
void gpu_matmul_strided_batched(gpu_blas_handle handle, float* out, const float* a, const float* b,
                                int M, int K, int N, long long strideA, long long strideB,
                                long long strideC, int batch_count);
// cuda/gpu_ops.cuh:93-96: out[i] += a[i]^T b[i] (accumulates)
void gpu_matmul_strided_batched_at(gpu_blas_handle handle, float* out, const float* a,
                                   const float* b, int M, int K, int N, long long strideA,
                                   long long strideB, long long strideC, int batch_count);
