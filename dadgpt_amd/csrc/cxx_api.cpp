// The reference's attention wrappers under their own C++ names and signatures
// (cuda/gpu_ops.cuh:112-122), built on the C ABI. Errors become std::runtime_error with the
// library's message, as CUDA_CHECK does in the reference (cuda/gpu_ops.cuh:10-17).
#include <stdexcept>
#include <string>

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
