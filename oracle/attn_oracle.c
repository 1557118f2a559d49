/*
 * CPU oracle for the fused causal attention path — TEST INFRASTRUCTURE ONLY (see
 * attn_oracle.h). Plain C, single-precision loops with a sequential fp32 k-sum, exactly the
 * arithmetic order of the reference's CPU operators:
 *   matmul               src/tensor_ops.cpp:6-16
 *   matmul_transposed_a  src/tensor_ops.cpp:18-30
 *   softmax              src/tensor_ops.cpp:32-55
 *   matmul_transposed_b  src/tensor_ops.cpp:111-123
 *   softmax_backward     src/backward.cpp:33-50   (accumulates into din)
 * composed in the op order of the materialized GPU attention (src/model.cpp:396-419 and
 * :585-615), with gpu_scale (cuda/gpu_ops.cu:513-518), gpu_causal_mask (-1e9 fill,
 * cuda/gpu_ops.cu:476-485) and gpu_causal_mask_zero (cuda/gpu_ops.cu:495-503) restated as
 * loops. The logsumexp has no CPU counterpart in the reference; it is the closed form of
 * what cuda/attention.cu:68-72 saves: lse_i = m_i + ln sum_{j<=i} exp(s_ij - m_i).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; no fast-math, so expf/logf and the
 * sum order are those of the reference build).
 */
#include "attn_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- the reference's CPU operators, restated (fp32) ---- */

/* out[M,N] = a[M,K] b[N,K]^T  — tensor_ops.cpp:111-123 */
static void mm_bt_f32(float* out, const float* a, const float* b, int M, int K, int N) {
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < N; ++j) {
      float acc = 0.0f;
      for (int t = 0; t < K; ++t) acc += a[(long)i * K + t] * b[(long)j * K + t];
      out[(long)i * N + j] = acc;
    }
}

/* out[M,N] = a[M,K] b[K,N]  — tensor_ops.cpp:6-16 */
static void mm_f32(float* out, const float* a, const float* b, int M, int K, int N) {
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < N; ++j) {
      float acc = 0.0f;
      for (int t = 0; t < K; ++t) acc += a[(long)i * K + t] * b[(long)t * N + j];
      out[(long)i * N + j] = acc;
    }
}

/* out[M,N] = a[K,M]^T b[K,N]  — tensor_ops.cpp:18-30 */
static void mm_at_f32(float* out, const float* a, const float* b, int M, int K, int N) {
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < N; ++j) {
      float acc = 0.0f;
      for (int t = 0; t < K; ++t) acc += a[(long)t * M + i] * b[(long)t * N + j];
      out[(long)i * N + j] = acc;
    }
}

/* Row softmax: max of the row (strict >, first element seeds), exp(x - max), sum, divide —
 * tensor_ops.cpp:32-55 */
static void softmax_rows_f32(float* out, const float* in, int rows, int cols) {
  for (int r = 0; r < rows; ++r) {
    const float* x = in + (long)r * cols;
    float* y = out + (long)r * cols;
    float mx = x[0];
    for (int c = 1; c < cols; ++c)
      if (x[c] > mx) mx = x[c];
    float sum = 0.0f;
    for (int c = 0; c < cols; ++c) {
      y[c] = expf(x[c] - mx);
      sum += y[c];
    }
    for (int c = 0; c < cols; ++c) y[c] /= sum;
  }
}

/* din += out * (dout - sum(dout*out))  — backward.cpp:33-50 */
static void softmax_bwd_rows_f32(const float* dout, const float* out, float* din, int rows,
                                 int cols) {
  for (int r = 0; r < rows; ++r) {
    const float* g = dout + (long)r * cols;
    const float* p = out + (long)r * cols;
    float* d = din + (long)r * cols;
    float dot = 0.0f;
    for (int c = 0; c < cols; ++c) dot += g[c] * p[c];
    for (int c = 0; c < cols; ++c) d[c] += p[c] * (g[c] - dot);
  }
}

/* data *= scale — gpu_scale, gpu_ops.cu:513-518 */
static void scale_f32(float* x, long n, float scale) {
  for (long i = 0; i < n; ++i) x[i] *= scale;
}

/* scores[i][j] = -1e9 for j > i — gpu_causal_mask, gpu_ops.cu:476-485 */
static void causal_fill_f32(float* s, int S) {
  for (int i = 0; i < S; ++i)
    for (int j = i + 1; j < S; ++j) s[(long)i * S + j] = -1e9f;
}

/* grads[i][j] = 0 for j > i — gpu_causal_mask_zero, gpu_ops.cu:495-503 */
static void causal_zero_f32(float* s, int S) {
  for (int i = 0; i < S; ++i)
    for (int j = i + 1; j < S; ++j) s[(long)i * S + j] = 0.0f;
}

/* ---- attention-probability dropout ----
 * The reference drops probabilities with cuRAND (cuda/gpu_ops.cu:712-733: keep iff a uniform
 * r >= rate, kept values times 1/(1-rate) in fp32, the gradient masked and scaled the same
 * way, :736-749). cuRAND's stream is not reproduced here; this build's mask comes from
 * Philox4x32-10 as published (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
 * as 1, 2, 3", SC'11), one block per 8 keys: the keep bit of probability (row = bh*S + i,
 * key j) is 16-bit half j%2 (low half first) of word (j%8)/2 of Philox4x32-10 at counter
 * {row lo, row hi, j/8, 0} under key {seed lo, seed hi}, kept iff that half >= thr with
 * thr = ceil(p * 2^16), i.e. a 16-bit uniform u >= p. */
static uint32_t mulhilo32(uint32_t a, uint32_t b, uint32_t* hi) {
  const uint64_t prod = (uint64_t)a * b;
  *hi = (uint32_t)(prod >> 32);
  return (uint32_t)prod;
}

void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
  uint32_t k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    if (r > 0) { /* key schedule: Weyl increments between rounds */
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    uint32_t hi0, hi1;
    const uint32_t lo0 = mulhilo32(0xD2511F53u, c0, &hi0);
    const uint32_t lo1 = mulhilo32(0xCD9E8D57u, c2, &hi1);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

uint32_t oracle_dropout_threshold(float p) { return (uint32_t)ceil((double)p * 65536.0); }

int oracle_dropout_keep(uint64_t seed, uint64_t row, int j, uint32_t thr) {
  const uint32_t ctr[4] = {(uint32_t)row, (uint32_t)(row >> 32), (uint32_t)j >> 3, 0u};
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t w[4];
  oracle_philox4x32_10(ctr, key, w);
  const uint32_t u = (w[(j & 7) >> 1] >> (16 * (j & 1))) & 0xFFFFu;
  return u >= thr;
}

void oracle_dropout_mask(uint8_t* mask, int BH, int S, uint64_t seed, float p) {
  const uint32_t thr = oracle_dropout_threshold(p);
  for (long row = 0; row < (long)BH * S; ++row)
    for (int j = 0; j < S; ++j)
      mask[row * S + j] = (uint8_t)oracle_dropout_keep(seed, (uint64_t)row, j, thr);
}

/* Dropout of one slice's probabilities (rows bh*S ..): Pd = keep ? P * (1/(1-p)) : 0, the
 * fp32 products of gpu_dropout_forward (cuda/gpu_ops.cu:712-726); keep bits kept in `keep`. */
typedef struct {
  uint64_t seed;
  uint32_t thr;
  float scale; /* 1/(1-p) in fp32, as cuda/gpu_ops.cu:718 */
} drop_t;

static void dropout_slice_f32(float* Pd, uint8_t* keep, const float* P, int S, int bh,
                              const drop_t* dr) {
  for (int i = 0; i < S; ++i)
    for (int j = 0; j < S; ++j) {
      const long n = (long)i * S + j;
      const int k = oracle_dropout_keep(dr->seed, (uint64_t)bh * S + i, j, dr->thr);
      keep[n] = (uint8_t)k;
      Pd[n] = k ? P[n] * dr->scale : 0.0f;
    }
}

/* ---- forward ---- */

/* One (b,h) slice: S = QK^T, *scale, lse (closed form over j<=i), mask, softmax, O = PV.
 * Op order of model.cpp:396-419. P is [S,S] scratch and holds the probabilities on return. */
static void probs_slice_f32(float* lse, const float* Q, const float* K, int S, int D,
                            float scale, float* P) {
  mm_bt_f32(P, Q, K, S, D, S);
  scale_f32(P, (long)S * S, scale);
  if (lse) {
    for (int i = 0; i < S; ++i) {
      const float* row = P + (long)i * S;
      float mx = row[0];
      for (int j = 1; j <= i; ++j)
        if (row[j] > mx) mx = row[j];
      float sum = 0.0f;
      for (int j = 0; j <= i; ++j) sum += expf(row[j] - mx);
      lse[i] = mx + logf(sum);
    }
  }
  causal_fill_f32(P, S);
  softmax_rows_f32(P, P, S, S);
}

static void fwd_slice_f32(float* O, float* lse, const float* Q, const float* K, const float* V,
                          int S, int D, float scale, float* P) {
  probs_slice_f32(lse, Q, K, S, D, scale, P);
  mm_f32(O, P, V, S, S, D);
}

int oracle_attn_fwd_f32_range(float* O, float* lse, const float* Q, const float* K,
                              const float* V, int bh0, int bh1, int S, int D, float scale) {
  float* P = (float*)malloc(sizeof(float) * (size_t)S * S);
  if (!P) return -1;
  for (int bh = bh0; bh < bh1; ++bh) {
    long o = (long)bh * S * D;
    fwd_slice_f32(O + o, lse ? lse + (long)bh * S : NULL, Q + o, K + o, V + o, S, D, scale, P);
  }
  free(P);
  return 0;
}

int oracle_attn_fwd_f32(float* O, float* lse, const float* Q, const float* K, const float* V,
                        int BH, int S, int D, float scale) {
  return oracle_attn_fwd_f32_range(O, lse, Q, K, V, 0, BH, S, D, scale);
}

/* ---- backward ---- */

/* One (b,h) slice in the op order of model.cpp:585-615:
 *   dP = dO V^T; dV = P^T dO; dS = 0; dS += softmax_bwd(dP, P); zero j>i; dS *= scale;
 *   dQ = dS K; dK = dS^T Q.
 * P is recomputed with the forward restatement (the materialized path keeps it from the
 * forward pass, model.cpp:402-407). */
static void bwd_slice_f32(float* dQ, float* dK, float* dV, const float* dO, const float* Q,
                          const float* K, const float* V, int S, int D, float scale, float* P,
                          float* dP, float* dS, float* Otmp) {
  fwd_slice_f32(Otmp, NULL, Q, K, V, S, D, scale, P);
  mm_bt_f32(dP, dO, V, S, D, S);
  mm_at_f32(dV, P, dO, S, S, D);
  memset(dS, 0, sizeof(float) * (size_t)S * S);
  softmax_bwd_rows_f32(dP, P, dS, S, S);
  causal_zero_f32(dS, S);
  scale_f32(dS, (long)S * S, scale);
  mm_f32(dQ, dS, K, S, S, D);
  mm_at_f32(dK, dS, Q, S, S, D);
}

int oracle_attn_bwd_f32_range(float* dQ, float* dK, float* dV, const float* dO, const float* Q,
                              const float* K, const float* V, int bh0, int bh1, int S, int D,
                              float scale) {
  size_t ss = (size_t)S * S;
  float* buf = (float*)malloc(sizeof(float) * (3 * ss + (size_t)S * D));
  if (!buf) return -1;
  for (int bh = bh0; bh < bh1; ++bh) {
    long o = (long)bh * S * D;
    bwd_slice_f32(dQ + o, dK + o, dV + o, dO + o, Q + o, K + o, V + o, S, D, scale, buf,
                  buf + ss, buf + 2 * ss, buf + 3 * ss);
  }
  free(buf);
  return 0;
}

/* delta[r] = sum_d dO*O — the row term of cuda/attention.cu:75-85 */
void oracle_attn_delta_f32(float* delta, const float* dO, const float* O, long rows, int D) {
  for (long r = 0; r < rows; ++r) {
    float acc = 0.0f;
    for (int d = 0; d < D; ++d) acc += dO[r * D + d] * O[r * D + d];
    delta[r] = acc;
  }
}

int oracle_attn_bwd_f32(float* dQ, float* dK, float* dV, float* delta, const float* dO,
                        const float* O, const float* Q, const float* K, const float* V, int BH,
                        int S, int D, float scale) {
  if (delta) oracle_attn_delta_f32(delta, dO, O, (long)BH * S, D);
  return oracle_attn_bwd_f32_range(dQ, dK, dV, dO, Q, K, V, 0, BH, S, D, scale);
}

/* ---- forward and backward with attention-probability dropout ----
 * Op order of the materialized path with dropout (src/model.cpp:396-419 with :406-416;
 * :585-615 with :594-599): forward S = QK^T, *scale, mask, softmax -> P; Pd = dropout(P);
 * O = Pd V. Backward dPd = dO V^T; dV = Pd^T dO; dP = dPd * (keep * 1/(1-p))
 * (gpu_dropout_backward, cuda/gpu_ops.cu:736-741); dS = softmax_bwd(dP, P); zero j>i;
 * *scale; dQ = dS K; dK = dS^T Q. lse is that of the undropped scores. */
static int drop_params(drop_t* dr, float p, uint64_t seed) {
  if (!(p >= 0.0f && p < 1.0f)) return -3;
  dr->seed = seed;
  dr->thr = oracle_dropout_threshold(p);
  dr->scale = 1.0f / (1.0f - p);
  return 0;
}

int oracle_attn_fwd_dropout_f32_range(float* O, float* lse, const float* Q, const float* K,
                                      const float* V, int bh0, int bh1, int S, int D,
                                      float scale, float p, uint64_t seed) {
  drop_t dr;
  if (drop_params(&dr, p, seed)) return -3;
  const size_t ss = (size_t)S * S;
  float* P = (float*)malloc(sizeof(float) * 2 * ss + ss);
  if (!P) return -1;
  float* Pd = P + ss;
  uint8_t* keep = (uint8_t*)(P + 2 * ss);
  for (int bh = bh0; bh < bh1; ++bh) {
    const long o = (long)bh * S * D;
    probs_slice_f32(lse ? lse + (long)bh * S : NULL, Q + o, K + o, S, D, scale, P);
    dropout_slice_f32(Pd, keep, P, S, bh, &dr);
    mm_f32(O + o, Pd, V + o, S, S, D);
  }
  free(P);
  return 0;
}

int oracle_attn_fwd_dropout_f32(float* O, float* lse, const float* Q, const float* K,
                                const float* V, int BH, int S, int D, float scale, float p,
                                uint64_t seed) {
  return oracle_attn_fwd_dropout_f32_range(O, lse, Q, K, V, 0, BH, S, D, scale, p, seed);
}

int oracle_attn_bwd_dropout_f32_range(float* dQ, float* dK, float* dV, const float* dO,
                                      const float* Q, const float* K, const float* V, int bh0,
                                      int bh1, int S, int D, float scale, float p,
                                      uint64_t seed) {
  drop_t dr;
  if (drop_params(&dr, p, seed)) return -3;
  const size_t ss = (size_t)S * S;
  float* P = (float*)malloc(sizeof(float) * 4 * ss + ss);
  if (!P) return -1;
  float *Pd = P + ss, *dP = P + 2 * ss, *dS = P + 3 * ss;
  uint8_t* keep = (uint8_t*)(P + 4 * ss);
  for (int bh = bh0; bh < bh1; ++bh) {
    const long o = (long)bh * S * D;
    probs_slice_f32(NULL, Q + o, K + o, S, D, scale, P);
    dropout_slice_f32(Pd, keep, P, S, bh, &dr);
    mm_bt_f32(dP, dO + o, V + o, S, D, S);
    mm_at_f32(dV + o, Pd, dO + o, S, S, D);
    for (size_t n = 0; n < ss; ++n) dP[n] *= (float)keep[n] * dr.scale;
    memset(dS, 0, sizeof(float) * ss);
    softmax_bwd_rows_f32(dP, P, dS, S, S);
    causal_zero_f32(dS, S);
    scale_f32(dS, (long)ss, scale);
    mm_f32(dQ + o, dS, K + o, S, S, D);
    mm_at_f32(dK + o, dS, Q + o, S, S, D);
  }
  free(P);
  return 0;
}

int oracle_attn_bwd_dropout_f32(float* dQ, float* dK, float* dV, float* delta, const float* dO,
                                const float* O, const float* Q, const float* K, const float* V,
                                int BH, int S, int D, float scale, float p, uint64_t seed) {
  drop_t dr;
  if (drop_params(&dr, p, seed)) return -3;
  if (delta) oracle_attn_delta_f32(delta, dO, O, (long)BH * S, D);
  return oracle_attn_bwd_dropout_f32_range(dQ, dK, dV, dO, Q, K, V, 0, BH, S, D, scale, p,
                                           seed);
}

/* ---- decode ---- */

/* Per sequence s and head h, with L = lens[s] (model.cpp:765-790):
 *   scores = q_h K_h[0:L]^T (matmul_transposed_b, M=1); *scale; softmax over L;
 *   o_h = scores V_h[0:L] (matmul, M=1). */
int oracle_decode_f32(float* out, const float* q, const float* k_cache, const float* v_cache,
                      const int* lens, int n_seq, int H, int max_len, int D, float scale) {
  float* sc = (float*)malloc(sizeof(float) * (size_t)max_len);
  if (!sc) return -1;
  for (int s = 0; s < n_seq; ++s) {
    int L = lens[s];
    if (L < 1 || L > max_len) {
      free(sc);
      return -2;
    }
    for (int h = 0; h < H; ++h) {
      const float* qh = q + ((long)s * H + h) * D;
      const float* kh = k_cache + ((long)s * H + h) * max_len * D;
      const float* vh = v_cache + ((long)s * H + h) * max_len * D;
      mm_bt_f32(sc, qh, kh, 1, D, L);
      scale_f32(sc, L, scale);
      softmax_rows_f32(sc, sc, 1, L);
      mm_f32(out + ((long)s * H + h) * D, sc, vh, 1, L, D);
    }
  }
  free(sc);
  return 0;
}

/* ---- double-precision twins (same loops, double arithmetic, exp/log) ---- */

static void fwd_slice_f64(double* O, double* lse, const double* Q, const double* K,
                          const double* V, int S, int D, double scale, double* P) {
  for (int i = 0; i < S; ++i)
    for (int j = 0; j < S; ++j) {
      double acc = 0.0;
      for (int t = 0; t < D; ++t) acc += Q[(long)i * D + t] * K[(long)j * D + t];
      P[(long)i * S + j] = acc * scale;
    }
  for (int i = 0; i < S; ++i) {
    double* row = P + (long)i * S;
    double mx = row[0];
    for (int j = 1; j <= i; ++j)
      if (row[j] > mx) mx = row[j];
    double sum = 0.0;
    for (int j = 0; j <= i; ++j) sum += exp(row[j] - mx);
    if (lse) lse[i] = mx + log(sum);
    for (int j = 0; j < S; ++j) row[j] = j <= i ? exp(row[j] - mx) / sum : 0.0;
  }
  for (int i = 0; i < S; ++i)
    for (int d = 0; d < D; ++d) {
      double acc = 0.0;
      for (int j = 0; j < S; ++j) acc += P[(long)i * S + j] * V[(long)j * D + d];
      O[(long)i * D + d] = acc;
    }
}

int oracle_attn_fwd_f64(double* O, double* lse, const double* Q, const double* K,
                        const double* V, int BH, int S, int D, double scale) {
  double* P = (double*)malloc(sizeof(double) * (size_t)S * S);
  if (!P) return -1;
  for (int bh = 0; bh < BH; ++bh) {
    long o = (long)bh * S * D;
    fwd_slice_f64(O + o, lse ? lse + (long)bh * S : NULL, Q + o, K + o, V + o, S, D, scale, P);
  }
  free(P);
  return 0;
}

int oracle_attn_bwd_f64(double* dQ, double* dK, double* dV, const double* dO, const double* Q,
                        const double* K, const double* V, int BH, int S, int D, double scale) {
  size_t ss = (size_t)S * S;
  double* P = (double*)malloc(sizeof(double) * (2 * ss + (size_t)S * D));
  if (!P) return -1;
  double* dS = P + ss;
  double* Ot = P + 2 * ss;
  for (int bh = 0; bh < BH; ++bh) {
    long o = (long)bh * S * D;
    const double *q = Q + o, *k = K + o, *v = V + o, *g = dO + o;
    fwd_slice_f64(Ot, NULL, q, k, v, S, D, scale, P);
    for (int i = 0; i < S; ++i) {
      double dot = 0.0;
      for (int j = 0; j < S; ++j) {
        double dp = 0.0;
        for (int t = 0; t < D; ++t) dp += g[(long)i * D + t] * v[(long)j * D + t];
        dS[(long)i * S + j] = dp;
        dot += dp * P[(long)i * S + j];
      }
      for (int j = 0; j < S; ++j)
        dS[(long)i * S + j] = j <= i ? P[(long)i * S + j] * (dS[(long)i * S + j] - dot) * scale
                                     : 0.0;
    }
    for (int j = 0; j < S; ++j)
      for (int d = 0; d < D; ++d) {
        double av = 0.0, ak = 0.0;
        for (int i = 0; i < S; ++i) {
          av += P[(long)i * S + j] * g[(long)i * D + d];
          ak += dS[(long)i * S + j] * q[(long)i * D + d];
        }
        dV[o + (long)j * D + d] = av;
        dK[o + (long)j * D + d] = ak;
      }
    for (int i = 0; i < S; ++i)
      for (int d = 0; d < D; ++d) {
        double aq = 0.0;
        for (int j = 0; j < S; ++j) aq += dS[(long)i * S + j] * k[(long)j * D + d];
        dQ[o + (long)i * D + d] = aq;
      }
  }
  free(P);
  return 0;
}

/* Double-precision twins with dropout (the same keep bits; 1/(1-p) in double): forward
 * O = Pd V with Pd = keep * P / (1-p); backward dV = Pd^T dO, dP = keep * (dO V^T) / (1-p),
 * dS = P (dP - rowsum(P dP)) * scale, dQ = dS K, dK = dS^T Q. */
int oracle_attn_fwd_dropout_f64(double* O, double* lse, const double* Q, const double* K,
                                const double* V, int BH, int S, int D, double scale, float p,
                                uint64_t seed) {
  drop_t dr;
  if (drop_params(&dr, p, seed)) return -3;
  const double inv = 1.0 / (1.0 - (double)p);
  double* P = (double*)malloc(sizeof(double) * ((size_t)S * S + (size_t)S * D));
  if (!P) return -1;
  double* Ot = P + (size_t)S * S;
  for (int bh = 0; bh < BH; ++bh) {
    const long o = (long)bh * S * D;
    fwd_slice_f64(Ot, lse ? lse + (long)bh * S : NULL, Q + o, K + o, V + o, S, D, scale, P);
    for (int i = 0; i < S; ++i)
      for (int d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int j = 0; j <= i; ++j)
          if (oracle_dropout_keep(seed, (uint64_t)bh * S + i, j, dr.thr))
            acc += P[(long)i * S + j] * inv * V[o + (long)j * D + d];
        O[o + (long)i * D + d] = acc;
      }
  }
  free(P);
  return 0;
}

int oracle_attn_bwd_dropout_f64(double* dQ, double* dK, double* dV, const double* dO,
                                const double* Q, const double* K, const double* V, int BH,
                                int S, int D, double scale, float p, uint64_t seed) {
  drop_t dr;
  if (drop_params(&dr, p, seed)) return -3;
  const double inv = 1.0 / (1.0 - (double)p);
  const size_t ss = (size_t)S * S;
  double* P = (double*)malloc(sizeof(double) * (3 * ss + (size_t)S * D));
  if (!P) return -1;
  double *Pd = P + ss, *dS = P + 2 * ss, *Ot = P + 3 * ss;
  for (int bh = 0; bh < BH; ++bh) {
    const long o = (long)bh * S * D;
    const double *q = Q + o, *k = K + o, *v = V + o, *g = dO + o;
    fwd_slice_f64(Ot, NULL, q, k, v, S, D, scale, P);
    for (int i = 0; i < S; ++i) {
      double dot = 0.0;
      for (int j = 0; j < S; ++j) {
        const long n = (long)i * S + j;
        const int kp = j <= i && oracle_dropout_keep(seed, (uint64_t)bh * S + i, j, dr.thr);
        Pd[n] = kp ? P[n] * inv : 0.0;
        double dp = 0.0;
        for (int t = 0; t < D; ++t) dp += g[(long)i * D + t] * v[(long)j * D + t];
        dS[n] = kp ? dp * inv : 0.0; /* dP */
        dot += dS[n] * P[n];
      }
      for (int j = 0; j < S; ++j) {
        const long n = (long)i * S + j;
        dS[n] = j <= i ? P[n] * (dS[n] - dot) * scale : 0.0;
      }
    }
    for (int j = 0; j < S; ++j)
      for (int d = 0; d < D; ++d) {
        double av = 0.0, ak = 0.0;
        for (int i = 0; i < S; ++i) {
          av += Pd[(long)i * S + j] * g[(long)i * D + d];
          ak += dS[(long)i * S + j] * q[(long)i * D + d];
        }
        dV[o + (long)j * D + d] = av;
        dK[o + (long)j * D + d] = ak;
      }
    for (int i = 0; i < S; ++i)
      for (int d = 0; d < D; ++d) {
        double aq = 0.0;
        for (int j = 0; j < S; ++j) aq += dS[(long)i * S + j] * k[(long)j * D + d];
        dQ[o + (long)i * D + d] = aq;
      }
  }
  free(P);
  return 0;
}

/* ---- threaded drivers over independent (b,h) slices ---- */

typedef struct {
  int fwd;
  float *O, *lse, *dQ, *dK, *dV;
  const float *Q, *K, *V, *dO;
  int bh0, bh1, S, D;
  float scale;
  int rc;
} slice_job;

static void* run_job(void* p) {
  slice_job* j = (slice_job*)p;
  if (j->fwd)
    j->rc = oracle_attn_fwd_f32_range(j->O, j->lse, j->Q, j->K, j->V, j->bh0, j->bh1, j->S,
                                      j->D, j->scale);
  else
    j->rc = oracle_attn_bwd_f32_range(j->dQ, j->dK, j->dV, j->dO, j->Q, j->K, j->V, j->bh0,
                                      j->bh1, j->S, j->D, j->scale);
  return NULL;
}

static int run_threads(slice_job base, int BH, int n_threads) {
  if (n_threads < 1) n_threads = 1;
  if (n_threads > BH) n_threads = BH;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * n_threads);
  slice_job* jobs = (slice_job*)malloc(sizeof(slice_job) * n_threads);
  if (!th || !jobs) {
    free(th);
    free(jobs);
    return -1;
  }
  int rc = 0;
  for (int t = 0; t < n_threads; ++t) {
    jobs[t] = base;
    jobs[t].bh0 = (int)((long)BH * t / n_threads);
    jobs[t].bh1 = (int)((long)BH * (t + 1) / n_threads);
    pthread_create(&th[t], NULL, run_job, &jobs[t]);
  }
  for (int t = 0; t < n_threads; ++t) {
    pthread_join(th[t], NULL);
    if (jobs[t].rc) rc = jobs[t].rc;
  }
  free(th);
  free(jobs);
  return rc;
}

int oracle_attn_fwd_f32_mt(float* O, float* lse, const float* Q, const float* K, const float* V,
                           int BH, int S, int D, float scale, int n_threads) {
  slice_job b;
  memset(&b, 0, sizeof(b));
  b.fwd = 1, b.O = O, b.lse = lse, b.Q = Q, b.K = K, b.V = V, b.S = S, b.D = D, b.scale = scale;
  return run_threads(b, BH, n_threads);
}

int oracle_attn_bwd_f32_mt(float* dQ, float* dK, float* dV, const float* dO, const float* Q,
                           const float* K, const float* V, int BH, int S, int D, float scale,
                           int n_threads) {
  slice_job b;
  memset(&b, 0, sizeof(b));
  b.fwd = 0, b.dQ = dQ, b.dK = dK, b.dV = dV, b.dO = dO, b.Q = Q, b.K = K, b.V = V, b.S = S;
  b.D = D, b.scale = scale;
  return run_threads(b, BH, n_threads);
}
