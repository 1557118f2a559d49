// The materialized attention path (src/model.cpp:395-420 forward, :575-616 backward) on the
// strided-batched hipBLASLt GEMMs of blaslt.cpp and the fused row kernels of libdadgpt_attn:
//   forward:  scores = Q K^T (all BH heads in one batched GEMM), probs = softmax(mask(scores *
//             scale)) in one pass, O = P V (one batched GEMM);
//   backward: dP = dO V^T, dV = P^T dO, dS = mask(softmax_backward(dP, P)) * scale in one pass
//             (written over dP), dQ = dS K, dK = dS^T Q.
// With attention dropout (src/model.cpp:406-416, 594-599) the forward multiplies V by the
// dropped probabilities Pd = P * keep / (1 - p) in a separate buffer (P itself is kept for the
// softmax backward), and the backward regenerates Pd from P and the mask (no mask is stored)
// in the score scratch for dV = Pd^T dO, then takes dPd = dO V^T through the dropout and
// softmax backward in one row pass.
// The reference runs the same GEMMs with separate scale / mask / softmax / zero passes; the
// fused row kernels touch each [S, S] row once. dQ, dK, dV are overwritten (the reference
// accumulates dK and dV into gradients it zeroed per micro-batch, src/train.cpp:204; with
// zeroed gradients the results are the same).
#include <hip/hip_runtime.h>

#include <cmath>

#include "dadgpt/gpu_attention.h"
#include "dadgpt/gpu_matmul.h"
#include "gen_internal.hpp"

namespace dadgpt::gen {

namespace {

int attn_status(int st, const char* what) {
  return st ? fail(st, "%s: %s", what, dadgpt_last_error()) : DADGPT_OK;
}

int check(const char* fn, int BH, int S, int d_head, float scale,
          std::initializer_list<const void*> ptrs) {
  for (const void* p : ptrs)
    if (p == nullptr) return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: null pointer argument", fn);
  if (BH < 1 || S < 1 || d_head < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: BH=%d, S=%d, d_head=%d must be positive", fn,
                BH, S, d_head);
  if (!std::isfinite(scale))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: scale must be finite", fn);
  return DADGPT_OK;
}

}  // namespace

int materialized_forward(dadgpt_blas* h, float* out, float* probs, const float* q,
                         const float* k, const float* v, int BH, int S, int dh, float scale,
                         long long stride_q, long long stride_kv, long long stride_o,
                         hipStream_t s) {
  const long long ss = (long long)S * S;
  // scores[i] = Q[i] K[i]^T   (gpu_matmul_strided_batched_bt, src/model.cpp:401-402)
  if (int st = gemm_f32(h, probs, q, k, S, dh, S, 'B', 0.0f, BH, stride_q, stride_kv, ss, s))
    return st;
  if (int st = attn_status(dadgpt_attention_probs(probs, BH, S, scale, s), "attention_probs"))
    return st;
  // O[i] = P[i] V[i]          (gpu_matmul_strided_batched, src/model.cpp:418-419)
  return gemm_f32(h, out, probs, v, S, S, dh, 'N', 0.0f, BH, ss, stride_kv, stride_o, s);
}

int materialized_decode(dadgpt_blas* h, float* out, float* probs, const float* q,
                        const float* kcache, const float* vcache, const int* lens, int n_seq,
                        int H, int max_len, int dh, float scale, hipStream_t s) {
  const int BH = n_seq * H;
  // one query row per (sequence, head): scores [BH, 1, max_len] = q K^T over the whole cache
  if (int st = gemm_f32(h, probs, q, kcache, 1, dh, max_len, 'B', 0.0f, BH, dh,
                        (long long)max_len * dh, max_len, s))
    return st;
  if (int st = attn_status(dadgpt_decode_probs(probs, lens, n_seq, H, max_len, scale, s),
                           "decode_probs"))
    return st;
  // keys past a sequence's length have probability exactly 0
  return gemm_f32(h, out, probs, vcache, 1, max_len, dh, 'N', 0.0f, BH, max_len,
                  (long long)max_len * dh, dh, s);
}

}  // namespace dadgpt::gen

using namespace dadgpt::gen;

extern "C" {

int dadgpt_attention_materialized_forward(dadgpt_blas* h, float* out, float* probs,
                                          const float* q, const float* k, const float* v, int BH,
                                          int S, int d_head, float scale, void* stream) {
  const char* fn = "dadgpt_attention_materialized_forward";
  if (int st = check(fn, BH, S, d_head, scale, {h, out, probs, q, k, v})) return st;
  const long long sq = (long long)S * d_head;
  return materialized_forward(h, out, probs, q, k, v, BH, S, d_head, scale, sq, sq, sq,
                              (hipStream_t)stream);
}

int dadgpt_attention_materialized_forward_dropout(dadgpt_blas* h, float* out, float* probs,
                                                  float* dropped, const float* q,
                                                  const float* k, const float* v, int BH, int S,
                                                  int d_head, float scale, float dropout_p,
                                                  uint64_t seed, void* stream) {
  const char* fn = "dadgpt_attention_materialized_forward_dropout";
  if (int st = check(fn, BH, S, d_head, scale, {h, out, probs, dropped, q, k, v})) return st;
  if (!(dropout_p >= 0.0f && dropout_p < 1.0f))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: dropout_p must be in [0, 1), got %g", fn,
                (double)dropout_p);
  if (dropped == probs)
    return fail(DADGPT_ERR_INVALID_ARGUMENT,
                "%s: dropped must not be probs (the backward needs the undropped probabilities)",
                fn);
  hipStream_t s = (hipStream_t)stream;
  const long long sq = (long long)S * d_head, ss = (long long)S * S;
  // scores = Q K^T, probs = softmax(mask(scores * scale))   (src/model.cpp:401-404)
  if (int st = gemm_f32(h, probs, q, k, S, d_head, S, 'B', 0.0f, BH, sq, sq, ss, s)) return st;
  if (int st = attn_status(dadgpt_attention_probs(probs, BH, S, scale, s), "attention_probs"))
    return st;
  // dropped = dropout(probs)                                (src/model.cpp:406-416)
  if (int st = attn_status(dadgpt_attention_dropout(dropped, probs, BH, S, dropout_p, seed, s),
                           "attention_dropout"))
    return st;
  // O = dropped V                                           (src/model.cpp:418-419)
  return gemm_f32(h, out, dropped, v, S, S, d_head, 'N', 0.0f, BH, ss, sq, sq, s);
}

int dadgpt_attention_materialized_backward_dropout(dadgpt_blas* h, float* dq, float* dk,
                                                   float* dv, float* dscores, const float* dout,
                                                   const float* probs, const float* q,
                                                   const float* k, const float* v, int BH, int S,
                                                   int d_head, float scale, float dropout_p,
                                                   uint64_t seed, void* stream) {
  const char* fn = "dadgpt_attention_materialized_backward_dropout";
  if (int st = check(fn, BH, S, d_head, scale, {h, dq, dk, dv, dscores, dout, probs, q, k, v}))
    return st;
  if (!(dropout_p >= 0.0f && dropout_p < 1.0f))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: dropout_p must be in [0, 1), got %g", fn,
                (double)dropout_p);
  hipStream_t s = (hipStream_t)stream;
  const long long sq = (long long)S * d_head, ss = (long long)S * S;
  // the forward's dropped probabilities, regenerated into the scratch: dV = Pd^T dO
  if (int st = attn_status(dadgpt_attention_dropout(dscores, probs, BH, S, dropout_p, seed, s),
                           "attention_dropout"))
    return st;
  if (int st = gemm_f32(h, dv, dscores, dout, S, S, d_head, 'A', 0.0f, BH, ss, sq, sq, s))
    return st;
  // dPd = dO V^T                (src/model.cpp:585-587)
  if (int st = gemm_f32(h, dscores, dout, v, S, d_head, S, 'B', 0.0f, BH, sq, sq, ss, s))
    return st;
  // dS = mask(softmax_backward(dPd * keep / (1-p), P)) * scale   (src/model.cpp:594-607)
  if (int st = attn_status(dadgpt_attention_probs_backward_dropout(dscores, dscores, probs, BH,
                                                                   S, scale, dropout_p, seed, s),
                           "attention_probs_backward_dropout"))
    return st;
  // dQ = dS K, dK = dS^T Q      (src/model.cpp:610-616)
  if (int st = gemm_f32(h, dq, dscores, k, S, S, d_head, 'N', 0.0f, BH, ss, sq, sq, s)) return st;
  return gemm_f32(h, dk, dscores, q, S, S, d_head, 'A', 0.0f, BH, ss, sq, sq, s);
}

int dadgpt_attention_materialized_backward(dadgpt_blas* h, float* dq, float* dk, float* dv,
                                           float* dscores, const float* dout,
                                           const float* probs, const float* q, const float* k,
                                           const float* v, int BH, int S, int d_head,
                                           float scale, void* stream) {
  const char* fn = "dadgpt_attention_materialized_backward";
  if (int st = check(fn, BH, S, d_head, scale, {h, dq, dk, dv, dscores, dout, probs, q, k, v}))
    return st;
  hipStream_t s = (hipStream_t)stream;
  const long long sq = (long long)S * d_head, ss = (long long)S * S;
  // dP = dO V^T                 (src/model.cpp:585-587)
  if (int st = gemm_f32(h, dscores, dout, v, S, d_head, S, 'B', 0.0f, BH, sq, sq, ss, s))
    return st;
  // dV = P^T dO                 (src/model.cpp:590-592)
  if (int st = gemm_f32(h, dv, probs, dout, S, S, d_head, 'A', 0.0f, BH, ss, sq, sq, s))
    return st;
  // dS = mask(softmax_backward(dP, P)) * scale, over dP   (src/model.cpp:601-607)
  if (int st = attn_status(dadgpt_attention_probs_backward(dscores, dscores, probs, BH, S, scale,
                                                           s),
                           "attention_probs_backward"))
    return st;
  // dQ = dS K                   (src/model.cpp:610-611)
  if (int st = gemm_f32(h, dq, dscores, k, S, S, d_head, 'N', 0.0f, BH, ss, sq, sq, s)) return st;
  // dK = dS^T Q                 (src/model.cpp:614-616)
  return gemm_f32(h, dk, dscores, q, S, S, d_head, 'A', 0.0f, BH, ss, sq, sq, s);
}

}  // extern "C"
