// Thin driver over the reference's OWN CPU operators — TEST INFRASTRUCTURE ONLY.
//
// oracle/Makefile compiles this file together with /root/reference/src/tensor_ops.cpp and
// /root/reference/src/backward.cpp, exactly where they lie, into oracle/_ref/libref_attn.so.
// The reference has no CPU attention function, so this driver calls the reference's
// matmul_transposed_b / softmax / matmul / matmul_transposed_a / softmax_backward in the op
// order of the materialized GPU attention (src/model.cpp:396-419 forward, :585-615 backward;
// decode src/model.cpp:765-790). Only the GPU-side scale and causal-mask steps have no CPU
// counterpart in the reference; they are the three loops below (gpu_scale gpu_ops.cu:513-518,
// gpu_causal_mask gpu_ops.cu:476-485, gpu_causal_mask_zero gpu_ops.cu:495-503).
//
// Used to pin oracle/attn_oracle.c (tests/golden/make_golden.py writes fixtures from it) and,
// when built, as bench.py's CPU baseline ("reference" kind).
#include <cstring>
#include <vector>

#include "backward.hpp"
#include "tensor_ops.hpp"

namespace {

void scale_all(float* x, size_t n, float s) {
  for (size_t i = 0; i < n; ++i) x[i] *= s;
}

void mask_upper(float* x, int S, float value) {
  for (int i = 0; i < S; ++i)
    for (int j = i + 1; j < S; ++j) x[static_cast<size_t>(i) * S + j] = value;
}

void forward_slice(float* O, float* P, const float* Q, const float* K, const float* V, int S,
                   int D, float scale) {
  matmul_transposed_b(P, Q, K, S, D, S);
  scale_all(P, static_cast<size_t>(S) * S, scale);
  mask_upper(P, S, -1e9f);
  softmax(P, P, S, S);
  matmul(O, P, V, S, S, D);
}

}  // namespace

extern "C" {

int ref_attn_fwd_f32(float* O, const float* Q, const float* K, const float* V, int bh0, int bh1,
                     int S, int D, float scale) {
  std::vector<float> P(static_cast<size_t>(S) * S);
  for (int bh = bh0; bh < bh1; ++bh) {
    size_t o = static_cast<size_t>(bh) * S * D;
    forward_slice(O + o, P.data(), Q + o, K + o, V + o, S, D, scale);
  }
  return 0;
}

int ref_attn_bwd_f32(float* dQ, float* dK, float* dV, const float* dO, const float* Q,
                     const float* K, const float* V, int bh0, int bh1, int S, int D,
                     float scale) {
  size_t ss = static_cast<size_t>(S) * S;
  std::vector<float> P(ss), dP(ss), dS(ss), Ot(static_cast<size_t>(S) * D);
  for (int bh = bh0; bh < bh1; ++bh) {
    size_t o = static_cast<size_t>(bh) * S * D;
    forward_slice(Ot.data(), P.data(), Q + o, K + o, V + o, S, D, scale);
    matmul_transposed_b(dP.data(), dO + o, V + o, S, D, S);
    matmul_transposed_a(dV + o, P.data(), dO + o, S, S, D);
    std::memset(dS.data(), 0, ss * sizeof(float));
    softmax_backward(dP.data(), P.data(), dS.data(), S, S);
    mask_upper(dS.data(), S, 0.0f);
    scale_all(dS.data(), ss, scale);
    matmul(dQ + o, dS.data(), K + o, S, S, D);
    matmul_transposed_a(dK + o, dS.data(), Q + o, S, S, D);
  }
  return 0;
}

int ref_decode_f32(float* out, const float* q, const float* k_cache, const float* v_cache,
                   const int* lens, int n_seq, int H, int max_len, int D, float scale) {
  std::vector<float> s(static_cast<size_t>(max_len));
  for (int b = 0; b < n_seq; ++b) {
    int L = lens[b];
    if (L < 1 || L > max_len) return -2;
    for (int h = 0; h < H; ++h) {
      size_t head = static_cast<size_t>(b) * H + h;
      matmul_transposed_b(s.data(), q + head * D, k_cache + head * max_len * D, 1, D, L);
      scale_all(s.data(), static_cast<size_t>(L), scale);
      softmax(s.data(), s.data(), 1, L);
      matmul(out + head * D, s.data(), v_cache + head * max_len * D, 1, L, D);
    }
  }
  return 0;
}

}  // extern "C"
