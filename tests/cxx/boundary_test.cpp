// Links against libdadgpt_attn.so through the reference's own wrapper names and C++
// signatures (cuda/gpu_ops.cuh:112-122) and checks their host-side behaviour, which needs no
// GPU: the supported() predicate and the std::runtime_error thrown for an unsupported d_head
// (message as cuda/attention.cu:238,251) and for a null buffer. Built and run by
// tests/test_capi.py.
#include <cstdio>
#include <stdexcept>
#include <string>

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

  EXPECT(dadgpt_flash_attention_forward(p, p, p, p, p, 4, 64, 48, 0.1f) == DADGPT_ERR_UNSUPPORTED);
  EXPECT(std::string(dadgpt_last_error()) == "flash attention: unsupported d_head 48");
  std::printf(failures ? "FAILED %d\n" : "OK\n", failures);
  return failures ? 1 : 0;
}
