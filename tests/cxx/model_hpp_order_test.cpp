// A caller in the reference's layout includes src/model.hpp, which defines
// `enum class AttentionImpl { Auto, Fused, Materialized };` (src/model.hpp:81), together with
// the drop-in header <dadgpt/gpu_ops_attention.hpp> (through cuda/gpu_ops.cuh), in either
// order. The enum below stands for model.hpp's definition; MODEL_HPP_FIRST picks the order.
// The call links against the library's use_fused_attention. Built and run by
// tests/test_capi.py.
#ifdef MODEL_HPP_FIRST
enum class AttentionImpl { Auto, Fused, Materialized };
#include "dadgpt/gpu_ops_attention.hpp"
#else
#include "dadgpt/gpu_ops_attention.hpp"
enum class AttentionImpl { Auto, Fused, Materialized };
#endif
#include <cstdio>

int main() {
  const bool ok = use_fused_attention(AttentionImpl::Fused, 64, 64, false) &&
                  !use_fused_attention(AttentionImpl::Materialized, 64, 4096, false) &&
                  use_fused_attention(AttentionImpl::Auto, 64, 512, false) &&
                  !use_fused_attention(AttentionImpl::Auto, 64, 511, false);
  std::printf(ok ? "OK\n" : "FAILED\n");
  return ok ? 0 : 1;
}
