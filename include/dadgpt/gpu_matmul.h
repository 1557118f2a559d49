/*
 * libdadgpt_gen.so — projection and attention GEMMs on hipBLASLt.
 *
 * Replaces the reference's cuBLAS matmul layer (cuda/gpu_ops.cuh:40-54,99-112, bodies
 * cuda/gpu_ops.cu:58-141), which the model's projections (src/model.cpp:372-374 QKV, :427 Wo,
 * :444-451 MLP, :472 and :818 logits) and the materialized attention (src/model.cpp:395-420,
 * 575-616) call. Same row-major convention and argument order (out, a, b, M, K, N); the
 * cublasHandle_t becomes an opaque dadgpt_blas handle. The C++ functions with the reference's
 * names and signatures are in <dadgpt/gpu_ops_matmul.hpp>.
 *
 * The hipBLASLt used is the one these sources were compiled against, opened privately by
 * absolute path from the ROCm installation (not whatever libhipblaslt.so.1 the process
 * already holds, e.g. PyTorch's bundled copy); dadgpt_blas_create refuses another version.
 *
 * Status codes are those of <dadgpt/gpu_attention.h> (0 = ok, 1 = invalid argument,
 * 2 = unsupported, 3 = HIP/hipBLASLt error); dadgpt_gen_last_error() describes the last
 * failure on the thread.
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

/* Opens the private hipBLASLt (once per process; later calls return the first result). Every
 * handle creation does this too; calling it early, before anything else in the process loads
 * a hipBLASLt or rocRoller of its own (PyTorch does at import), is what lets both coexist. */
int dadgpt_blas_open(void);

/* Creates a handle on the current device: a hipBLASLt handle, a 32 MiB workspace and a cache
 * of per-shape algorithm choices (replaces cublasCreate in model_alloc, src/model.cpp:236).
 * Refused (DADGPT_ERR_UNSUPPORTED, with both versions in the message) unless the process's
 * HIP runtime and the opened hipBLASLt are a pair dadgpt_blas_stack_supported accepts. */
int dadgpt_blas_create(dadgpt_blas** out);
void dadgpt_blas_destroy(dadgpt_blas* h);

/* hipBLASLt's own version (major*100000 + minor*100 + patch) behind a handle, -1 on error. */
int dadgpt_blas_library_version(dadgpt_blas* h);

/* The process's HIP runtime version (hipRuntimeGetVersion: major*10^7 + minor*10^5 + patch)
 * and the opened hipBLASLt's (-1 for either one that cannot be read, e.g. no device). */
int dadgpt_blas_stack_versions(int* hip_runtime, int* hipblaslt);
/* 1 if (hip_runtime, hipblaslt) is a pair the GPU tests run on: HIP 7.0 (PyTorch's runtime)
 * or 7.2 (the ROCm installation's) with the hipBLASLt version these sources were compiled
 * against; 0 otherwise. */
int dadgpt_blas_stack_supported(int hip_runtime, int hipblaslt);

/* Process-wide multiply precision of the fp32 GEMMs below, as gpu_set_matmul_precision
 * (cuda/gpu_ops.cuh:43-44, cuda/gpu_ops.cu:61-67): storage and accumulation stay fp32.
 * FP32 (default) multiplies in fp32. BF16 rounds the inputs to bfloat16 inside the GEMM
 * (HIPBLAS_COMPUTE_32F_FAST_16BF, as CUBLAS_COMPUTE_32F_FAST_16BF). gfx950 has no TF32 format:
 * TF32 runs as FP32. */
typedef enum dadgpt_matmul_precision {
  DADGPT_MATMUL_FP32 = 0,
  DADGPT_MATMUL_TF32 = 1,
  DADGPT_MATMUL_BF16 = 2
} dadgpt_matmul_precision;
int dadgpt_set_matmul_precision(int precision);
int dadgpt_get_matmul_precision(void);

/* fp32 row-major GEMM, out[M,N] = op(a) op(b) + beta * out (beta 0: out is overwritten):
 *   op 'N': a [M,K], b [K,N]   gpu_matmul                (cuda/gpu_ops.cu:94-98)
 *   op 'A': a [K,M], b [K,N]   gpu_matmul_transposed_a   (:100-106; beta 1 = accumulate)
 *   op 'B': a [M,K], b [N,K]   gpu_matmul_transposed_b   (:108-112) */
int dadgpt_matmul_f32(dadgpt_blas* h, float* out, const float* a, const float* b, int M, int K,
                      int N, int op, float beta, void* stream);

/* Strided-batched form: matrix i of a, b, out starts stride_* elements after matrix i-1.
 *   op 'B', beta 0: gpu_matmul_strided_batched_bt  (cuda/gpu_ops.cu:116-123)
 *   op 'N', beta 0: gpu_matmul_strided_batched     (:125-132)
 *   op 'A', beta 1: gpu_matmul_strided_batched_at  (:134-141) */
int dadgpt_matmul_f32_strided_batched(dadgpt_blas* h, float* out, const float* a,
                                      const float* b, int M, int K, int N, int op, float beta,
                                      long long stride_a, long long stride_b,
                                      long long stride_out, int batch_count, void* stream);

/* bf16 operands, fp32 output (the generation path's projections).
 * Replaces gpu_matmul (cuda/gpu_ops.cu:94-98): row-major out[M,N] = a[M,K] x b[K,N]. */
int dadgpt_matmul_bf16(dadgpt_blas* h, float* out, const uint16_t* a, const uint16_t* b, int M,
                       int K, int N, void* stream);

/* Replaces gpu_matmul_transposed_b (cuda/gpu_ops.cu:108-112): row-major
 * out[M,N] = a[M,K] x b[N,K]^T (the weight-tied logits). */
int dadgpt_matmul_transposed_b_bf16(dadgpt_blas* h, float* out, const uint16_t* a,
                                    const uint16_t* b, int M, int K, int N, void* stream);

/* ---- Materialized attention on these GEMMs (the reference's path for short contexts and
 * dropout, src/model.cpp:395-420 forward, :575-616 backward). fp32 [BH, S, d_head]
 * contiguous q, k, v, out, dout, dq, dk, dv; any d_head. The GEMMs multiply at the
 * process-wide precision (dadgpt_set_matmul_precision); the row kernels are the fused ones
 * of <dadgpt/gpu_attention.h>. */

/* out = softmax(mask(q k^T * scale)) v; probs [BH, S, S] receives the probabilities (kept for
 * the backward, as the reference's attn_probs). */
int dadgpt_attention_materialized_forward(dadgpt_blas* h, float* out, float* probs,
                                          const float* q, const float* k, const float* v, int BH,
                                          int S, int d_head, float scale, void* stream);
/* dq, dk, dv (overwritten) from dout and the forward's probs; dscores [BH, S, S] is scratch. */
int dadgpt_attention_materialized_backward(dadgpt_blas* h, float* dq, float* dk, float* dv,
                                           float* dscores, const float* dout,
                                           const float* probs, const float* q, const float* k,
                                           const float* v, int BH, int S, int d_head,
                                           float scale, void* stream);
/* The same with attention-probability dropout (src/model.cpp:406-416 forward, :594-599
 * backward), the path use_fused_attention picks for every dropout call: the forward writes
 * the probabilities to probs (kept for the backward) and probs * keep / (1 - dropout_p) to
 * dropped [BH, S, S] (a separate buffer, as the reference's attn_dropped), and out =
 * dropped v. The backward regenerates the dropped probabilities from probs and the mask into
 * dscores (no mask is stored: same seed and dropout_p as the forward). The mask is the one of
 * the flash _dropout entry points of <dadgpt/gpu_attention.h>, so both paths drop the same
 * probabilities. */
int dadgpt_attention_materialized_forward_dropout(dadgpt_blas* h, float* out, float* probs,
                                                  float* dropped, const float* q,
                                                  const float* k, const float* v, int BH, int S,
                                                  int d_head, float scale, float dropout_p,
                                                  uint64_t seed, void* stream);
int dadgpt_attention_materialized_backward_dropout(dadgpt_blas* h, float* dq, float* dk,
                                                   float* dv, float* dscores, const float* dout,
                                                   const float* probs, const float* q,
                                                   const float* k, const float* v, int BH, int S,
                                                   int d_head, float scale, float dropout_p,
                                                   uint64_t seed, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DADGPT_GPU_MATMUL_H */
