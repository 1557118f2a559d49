// The reference's attention wrappers and the materialized path's elementwise operators under
// their own C++ names and signatures (cuda/gpu_ops.cuh:57,76,106-122), built on the C ABI. Errors become std::runtime_error with the
// library's message, as CUDA_CHECK does in the reference (cuda/gpu_ops.cuh:10-17).
#include <stdexcept>
#include <string>

#include "dadgpt/attention_impl.hpp"
#include "dadgpt/gpu_attention.h"
#include "dadgpt/gpu_ops_attention.hpp"

namespace {
void throw_if(int status) {
  if (status != DADGPT_OK) throw std::runtime_error(dadgpt_last_error());
}
}  // namespace

bool gpu_flash_attention_supported(int d_head) {
  return dadgpt_flash_attention_supported(d_head) != 0;
}

void gpu_flash_attention_forward(float* out, float* lse, const float* q, const float* k,
                                 const float* v, int BH, int S, int d_head, float scale) {
  throw_if(dadgpt_flash_attention_forward(out, lse, q, k, v, BH, S, d_head, scale));
}

void gpu_flash_attention_backward(float* dq, float* dk, float* dv, float* delta, const float* dout,
                                  const float* out, const float* lse, const float* q,
                                  const float* k, const float* v, int BH, int S, int d_head,
                                  float scale) {
  throw_if(dadgpt_flash_attention_backward(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S,
                                           d_head, scale));
}

void gpu_softmax(float* out, const float* in, int rows, int cols) {
  throw_if(dadgpt_softmax(out, in, rows, cols, nullptr));
}

void gpu_softmax_backward(float* din, const float* dout, const float* out, int rows, int cols) {
  throw_if(dadgpt_softmax_backward(din, dout, out, rows, cols, nullptr));
}

void gpu_causal_mask(float* scores, int num_blocks, int seq_len) {
  throw_if(dadgpt_causal_mask(scores, num_blocks, seq_len, nullptr));
}

void gpu_causal_mask_zero(float* grads, int num_blocks, int seq_len) {
  throw_if(dadgpt_causal_mask_zero(grads, num_blocks, seq_len, nullptr));
}

void gpu_scale(float* data, int size, float scale) {
  throw_if(dadgpt_scale(data, size, scale, nullptr));
}

void gpu_split_heads(float* out, const float* in, int batch_size, int seq_len, int n_heads,
                     int d_head) {
  throw_if(dadgpt_split_heads(out, in, batch_size, seq_len, n_heads, d_head, nullptr));
}

void gpu_merge_heads(float* out, const float* in, int batch_size, int seq_len, int n_heads,
                     int d_head) {
  throw_if(dadgpt_merge_heads(out, in, batch_size, seq_len, n_heads, d_head, nullptr));
}

bool use_fused_attention(AttentionImpl impl, int d_head, int ctx_len, bool attn_dropout) {
  const int c = impl == AttentionImpl::Fused          ? DADGPT_ATTENTION_FUSED
                : impl == AttentionImpl::Materialized ? DADGPT_ATTENTION_MATERIALIZED
                                                      : DADGPT_ATTENTION_AUTO;
  return dadgpt_use_fused_attention(c, d_head, ctx_len, attn_dropout ? 1 : 0) != 0;
}
