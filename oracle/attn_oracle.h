/*
 * CPU oracle for the fused causal attention path — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker (or the timed CPU baseline). The product path
 * (dadgpt_amd/) never calls it and fails loudly when its HIP library is missing.
 *
 * The reference has no CPU attention function. Its CPU operators (src/tensor_ops.cpp,
 * src/backward.cpp) are composed here in the op order of the reference's materialized GPU
 * attention (src/model.cpp:396-419 forward, :585-615 backward); the scale and causal-mask
 * steps restate gpu_scale (cuda/gpu_ops.cu:513-518) and gpu_causal_mask /
 * gpu_causal_mask_zero (cuda/gpu_ops.cu:476-503). Each function below cites the reference
 * lines it follows. Layout everywhere: [BH, S, D] row-major, lse [BH, S].
 *
 * Parity pinning (which check pins which function) is listed in oracle/README.md.
 */
#ifndef DADGPT_ATTN_ORACLE_H
#define DADGPT_ATTN_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

/* Causal forward, fp32, reference op order. O [BH,S,D], lse [BH,S] (natural log of the
 * scaled, unmasked score row). Returns 0, or -1 on allocation failure. */
int oracle_attn_fwd_f32(float* O, float* lse, const float* Q, const float* K, const float* V,
                        int BH, int S, int D, float scale);

/* Same, over bh slices [bh0, bh1) only (bounded CPU-baseline samples). */
int oracle_attn_fwd_f32_range(float* O, float* lse, const float* Q, const float* K,
                              const float* V, int bh0, int bh1, int S, int D, float scale);

/* Causal backward, fp32, reference materialized op order. Writes dQ, dK, dV [BH,S,D]
 * (overwrite) and, when delta != NULL, delta [BH,S] = sum_d dO*O. O is only used for delta. */
int oracle_attn_bwd_f32(float* dQ, float* dK, float* dV, float* delta, const float* dO,
                        const float* O, const float* Q, const float* K, const float* V, int BH,
                        int S, int D, float scale);

int oracle_attn_bwd_f32_range(float* dQ, float* dK, float* dV, const float* dO, const float* Q,
                              const float* K, const float* V, int bh0, int bh1, int S, int D,
                              float scale);

/* delta[r] = sum_d dO[r,d] * O[r,d] over rows r in [0, rows). */
void oracle_attn_delta_f32(float* delta, const float* dO, const float* O, long rows, int D);

/* KV-cache decode, fp32, reference op order of model.cpp:765-790, batched over sequences.
 * q [n_seq,H,D]; k_cache, v_cache [n_seq,H,max_len,D]; lens[n_seq] in [1,max_len];
 * out [n_seq,H,D]. */
int oracle_decode_f32(float* out, const float* q, const float* k_cache, const float* v_cache,
                      const int* lens, int n_seq, int H, int max_len, int D, float scale);

/* Double-precision twins (tie-breakers and brute-force checks). */
int oracle_attn_fwd_f64(double* O, double* lse, const double* Q, const double* K,
                        const double* V, int BH, int S, int D, double scale);
int oracle_attn_bwd_f64(double* dQ, double* dK, double* dV, const double* dO, const double* Q,
                        const double* K, const double* V, int BH, int S, int D, double scale);

/* Multi-threaded forward/backward over bh slices (pthreads), for the CPU baseline. */
int oracle_attn_fwd_f32_mt(float* O, float* lse, const float* Q, const float* K, const float* V,
                           int BH, int S, int D, float scale, int n_threads);
int oracle_attn_bwd_f32_mt(float* dQ, float* dK, float* dV, const float* dO, const float* Q,
                           const float* K, const float* V, int BH, int S, int D, float scale,
                           int n_threads);

#ifdef __cplusplus
}
#endif
#endif
