/*
 * libdadgpt_gen.so — bf16 projection GEMMs on hipBLASLt.
 *
 * Replaces the reference's cuBLAS wrappers gpu_matmul / gpu_matmul_transposed_b
 * (cuda/gpu_ops.cuh:74-96, cuda/gpu_ops.cu:94-112), which the model's projections call
 * (src/model.cpp:372-374 QKV, :427 Wo, :444-451 MLP, :472 and :818 logits). Same row-major
 * convention and argument order (out, a, b, M, K, N); the cublasHandle_t becomes an opaque
 * dadgpt_blas handle. Operands are bf16 (uint16_t bit patterns), accumulation and the output
 * are fp32, as the reference keeps fp32 activations.
 *
 * Status codes are those of <dadgpt/gpu_attention.h> (0 = ok, 1 = invalid argument,
 * 3 = HIP/hipBLASLt error); dadgpt_gen_last_error() describes the last failure on the thread.
 */
#ifndef DADGPT_GPU_MATMUL_H
#define DADGPT_GPU_MATMUL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dadgpt_blas dadgpt_blas;

/* Message of the last failing call of libdadgpt_gen on this thread ("" if none). */
const char* dadgpt_gen_last_error(void);

/* Creates a handle on the current device: a hipBLASLt handle, a 32 MiB workspace and a cache
 * of per-shape algorithm choices (replaces cublasCreate in model_alloc, src/model.cpp:236). */
int dadgpt_blas_create(dadgpt_blas** out);
void dadgpt_blas_destroy(dadgpt_blas* h);

/* Replaces gpu_matmul (cuda/gpu_ops.cu:94-98): row-major out[M,N] = a[M,K] x b[K,N]. */
int dadgpt_matmul_bf16(dadgpt_blas* h, float* out, const uint16_t* a, const uint16_t* b, int M,
                       int K, int N, void* stream);

/* Replaces gpu_matmul_transposed_b (cuda/gpu_ops.cu:108-112): row-major
 * out[M,N] = a[M,K] x b[N,K]^T (the weight-tied logits). */
int dadgpt_matmul_transposed_b_bf16(dadgpt_blas* h, float* out, const uint16_t* a,
                                    const uint16_t* b, int M, int K, int N, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DADGPT_GPU_MATMUL_H */
