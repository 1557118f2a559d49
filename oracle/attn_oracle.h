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
 * Which check pins which function: tests/test_oracle.py and tests/pins.py (golden vectors from
 * the reference's own operators, closed forms, invariants, finite differences).
 */
#ifndef DADGPT_ATTN_ORACLE_H
#define DADGPT_ATTN_ORACLE_H

#include <stdint.h>

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

/* Attention-probability dropout (the reference: cuda/gpu_ops.cu:712-749, applied at
 * src/model.cpp:406-416 and :594-599). The reference draws its mask from cuRAND, whose
 * stream is not reproduced; this build's mask is Philox4x32-10 as published (Salmon et al.,
 * SC'11): probability (row = bh*S + i, key j) is kept iff u >= ceil(p * 2^16), u = 16-bit
 * half j%2 (low first) of word (j%8)/2 of Philox4x32-10(counter {row lo, row hi, j/8, 0},
 * key {seed lo, seed hi}).
 * Kept probabilities are scaled by 1/(1-p) (fp32), as the reference does. p in [0, 1). */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
uint32_t oracle_dropout_threshold(float p);
int oracle_dropout_keep(uint64_t seed, uint64_t row, int j, uint32_t thr);
/* keep bits [BH, S, S] (1 = kept) */
void oracle_dropout_mask(uint8_t* mask, int BH, int S, uint64_t seed, float p);
/* Forward / backward with dropout, fp32, the materialized op order with dropout
 * (src/model.cpp:396-419 with :406-416, :585-615 with :594-599). lse is that of the undropped
 * scores; delta (when non-NULL) is rowsum(dO * O). Return -3 for p outside [0, 1). */
int oracle_attn_fwd_dropout_f32(float* O, float* lse, const float* Q, const float* K,
                                const float* V, int BH, int S, int D, float scale, float p,
                                uint64_t seed);
/* The forward over bh slices [bh0, bh1) only (rows keep their global index bh*S + i). */
int oracle_attn_fwd_dropout_f32_range(float* O, float* lse, const float* Q, const float* K,
                                      const float* V, int bh0, int bh1, int S, int D,
                                      float scale, float p, uint64_t seed);
int oracle_attn_bwd_dropout_f32(float* dQ, float* dK, float* dV, float* delta, const float* dO,
                                const float* O, const float* Q, const float* K, const float* V,
                                int BH, int S, int D, float scale, float p, uint64_t seed);
/* The backward over slices [bh0, bh1) only (the mask rows keep their global index bh*S + i). */
int oracle_attn_bwd_dropout_f32_range(float* dQ, float* dK, float* dV, const float* dO,
                                      const float* Q, const float* K, const float* V, int bh0,
                                      int bh1, int S, int D, float scale, float p,
                                      uint64_t seed);
int oracle_attn_fwd_dropout_f64(double* O, double* lse, const double* Q, const double* K,
                                const double* V, int BH, int S, int D, double scale, float p,
                                uint64_t seed);
int oracle_attn_bwd_dropout_f64(double* dQ, double* dK, double* dV, const double* dO,
                                const double* Q, const double* K, const double* V, int BH,
                                int S, int D, double scale, float p, uint64_t seed);

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
