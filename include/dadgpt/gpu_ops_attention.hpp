// The reference's fused-attention wrappers under their own names and C++ signatures
// (cuda/gpu_ops.cuh:112-122), defined in libdadgpt_attn.so on top of the C ABI in
// <dadgpt/gpu_attention.h>. A caller compiled against the reference's gpu_ops.cuh (for
// example src/model.cpp:186,392,570) links against these symbols unchanged.
//
// Error behaviour follows the reference: argument and launch errors throw
// std::runtime_error (cuda/gpu_ops.cuh:10-17; unsupported d_head at cuda/attention.cu:238,251).
#pragma once

// cuda/gpu_ops.cuh:115
bool gpu_flash_attention_supported(int d_head);

// cuda/gpu_ops.cuh:116-117
void gpu_flash_attention_forward(float* out, float* lse, const float* q, const float* k,
                                 const float* v, int BH, int S, int d_head, float scale);

// cuda/gpu_ops.cuh:119-122
void gpu_flash_attention_backward(float* dq, float* dk, float* dv, float* delta, const float* dout,
                                  const float* out, const float* lse, const float* q,
                                  const float* k, const float* v, int BH, int S, int d_head,
                                  float scale);

// ---- the materialized path's elementwise operators (null stream, throw on error) ----

// cuda/gpu_ops.cuh:57
void gpu_softmax(float* out, const float* in, int rows, int cols);
// cuda/gpu_ops.cuh:76 (accumulates into din)
void gpu_softmax_backward(float* din, const float* dout, const float* out, int rows, int cols);
// cuda/gpu_ops.cuh:106
void gpu_causal_mask(float* scores, int num_blocks, int seq_len);
// cuda/gpu_ops.cuh:108
void gpu_causal_mask_zero(float* grads, int num_blocks, int seq_len);
// cuda/gpu_ops.cuh:110
void gpu_scale(float* data, int size, float scale);

// cuda/gpu_ops.cuh:98-104: [B*S, H*dh] <-> [B*H, S, dh], fp32, null stream. The attention
// calls of <dadgpt/gpu_attention.h> also read and write the token-major layout in place.
void gpu_split_heads(float* out, const float* in, int batch_size, int seq_len, int n_heads,
                     int d_head);
void gpu_merge_heads(float* out, const float* in, int batch_size, int seq_len, int n_heads,
                     int d_head);

// The predicate of src/model.cpp:183-197 without the Model: the caller passes its
// implementation choice, head size and context length. AttentionImpl is the reference's own
// enum (src/model.hpp:81, `enum class AttentionImpl { Auto, Fused, Materialized };`): it is only
// declared here, so this header can be included before or after the reference's model.hpp.
// Callers without model.hpp include <dadgpt/attention_impl.hpp> for the definition.
enum class AttentionImpl;
bool use_fused_attention(AttentionImpl impl, int d_head, int ctx_len, bool attn_dropout);
