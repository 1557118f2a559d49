// Links against libdadgpt_attn.so through the reference's own wrapper names and C++
// signatures (cuda/gpu_ops.cuh:57,76,106-122; src/model.hpp:80) and checks their host-side
// behaviour, which needs no GPU: the supported() and fused/materialized predicates, and the
// std::runtime_error thrown for an unsupported d_head (message as cuda/attention.cu:238,251),
// for a null buffer and for bad head split/merge shapes (cuda/gpu_ops.cuh:98-104). Built and
// run by tests/test_capi.py.
#include <cstdio>
#include <stdexcept>
#include <string>

#include "dadgpt/attention_impl.hpp"
#include "dadgpt/gpu_attention.h"
#include "dadgpt/gpu_ops_attention.hpp"

static int failures = 0;
#define EXPECT(cond)                                             \
  do {                                                           \
    if (!(cond)) {                                               \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond); \
      ++failures;                                                \
    }                                                            \
  } while (0)

template <class F>
static std::string thrown(F f) {
  try {
    f();
  } catch (const std::runtime_error& e) {
    return e.what();
  }
  return "<no exception>";
}

int main() {
  EXPECT(gpu_flash_attention_supported(32));
  EXPECT(gpu_flash_attention_supported(64));
  EXPECT(!gpu_flash_attention_supported(48));
  EXPECT(!gpu_flash_attention_supported(128));

  float* p = reinterpret_cast<float*>(0x1000);  // never dereferenced: validation fails first
  std::string m = thrown([&] { gpu_flash_attention_forward(p, p, p, p, p, 4, 64, 48, 0.1f); });
  EXPECT(m == "flash attention: unsupported d_head 48");
  m = thrown([&] {
    gpu_flash_attention_backward(p, p, p, p, p, p, p, p, p, p, 4, 64, 96, 0.1f);
  });
  EXPECT(m == "flash attention: unsupported d_head 96");
  m = thrown([&] { gpu_flash_attention_forward(nullptr, p, p, p, p, 4, 64, 64, 0.1f); });
  EXPECT(m.find("null") != std::string::npos);
  m = thrown([&] { gpu_flash_attention_forward(p, p, p, p, p, 0, 64, 64, 0.1f); });
  EXPECT(m.find("positive") != std::string::npos);

  // the materialized path's operators and the fused/materialized choice (src/model.cpp:183-197)
  m = thrown([&] { gpu_softmax(nullptr, p, 4, 64); });
  EXPECT(m.find("null") != std::string::npos);
  m = thrown([&] { gpu_causal_mask(p, 0, 64); });
  EXPECT(m.find("positive") != std::string::npos);
  m = thrown([&] { gpu_scale(nullptr, 10, 2.0f); });
  EXPECT(m.find("null") != std::string::npos);
  m = thrown([&] { gpu_softmax_backward(p, p, nullptr, 4, 64); });
  EXPECT(m.find("null") != std::string::npos);
  m = thrown([&] { gpu_split_heads(nullptr, p, 2, 16, 4, 64); });
  EXPECT(m.find("null") != std::string::npos);
  m = thrown([&] { gpu_merge_heads(p + 4096, p, 2, 0, 4, 64); });
  EXPECT(m.find("positive") != std::string::npos);
  m = thrown([&] { gpu_split_heads(p + 16, p, 2, 16, 4, 64); });  // overlapping buffers
  EXPECT(m.find("overlap") != std::string::npos);
  EXPECT(use_fused_attention(AttentionImpl::Fused, 64, 64, false));
  EXPECT(!use_fused_attention(AttentionImpl::Fused, 64, 64, true));
  EXPECT(!use_fused_attention(AttentionImpl::Fused, 48, 1024, false));
  EXPECT(!use_fused_attention(AttentionImpl::Materialized, 64, 4096, false));
  EXPECT(use_fused_attention(AttentionImpl::Auto, 32, 512, false));
  EXPECT(!use_fused_attention(AttentionImpl::Auto, 32, 511, false));

  EXPECT(dadgpt_flash_attention_forward(p, p, p, p, p, 4, 64, 48, 0.1f) == DADGPT_ERR_UNSUPPORTED);
  EXPECT(std::string(dadgpt_last_error()) == "flash attention: unsupported d_head 48");
  std::printf(failures ? "FAILED %d\n" : "OK\n", failures);
  return failures ? 1 : 0;
}
