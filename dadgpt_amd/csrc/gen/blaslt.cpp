// hipBLASLt GEMMs behind the reference's row-major matmul wrappers (cuda/gpu_ops.cu:58-141).
//
// Which hipBLASLt. The library is not linked: it is opened privately, by absolute path, from
// the ROCm installation whose headers these sources were compiled against
// (DADGPT_HIPBLASLT_SO), with RTLD_LOCAL | RTLD_DEEPBIND, and every entry point is taken from
// that handle. A process can hold another libhipblaslt.so.1: PyTorch's ROCm wheel bundles an
// older hipBLASLt (and rocRoller) under the same sonames, loaded by `import torch`. Linking by
// soname bound this library's calls to that copy, whose structures and kernel set are not the
// ones compiled here. Opened privately, the ROCm copy shares the process's HIP runtime (its
// libamdhip64.so.7 dependency resolves to the one already loaded) and stays out of the global
// symbol scope, so PyTorch keeps binding to its own. Its rocRoller dependency resolves by
// soname too, so it must be opened before PyTorch loads its rocRoller: the Python package
// does that at import (dadgpt_blas_open); opened later, dlopen fails and every handle creation
// reports why. dadgpt_blas_create also refuses a copy whose reported version differs from the
// headers', and a HIP runtime that no GPU test has run this hipBLASLt on (stack_supported).
//
// Row-major to column-major: a row-major X[R,C] is the column-major X^T (C rows, R cols,
// leading dimension C), so the row-major product out = op(a) op(b) is the column-major
// out^T = op(b)^T op(a)^T: hipBLASLt's first operand is `b`, its second `a`, as stored.
//
// One plan (descriptors, layouts, algorithm) per distinct problem, reused. The 32 MiB
// workspace is allocated once per handle, and only candidates whose workspace fits it are
// kept. The first beta = 0 call of a problem (outside stream capture) times up to 16
// heuristic candidates on its own operands and keeps the fastest (for the skinny decode shapes
// the heuristic's first choice was up to several times slower).
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt-version.h>
#include <hipblaslt/hipblaslt.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "dadgpt/gpu_attention.h"
#include "dadgpt/gpu_matmul.h"
#include "gen_internal.hpp"

#ifndef DADGPT_HIPBLASLT_SO
#define DADGPT_HIPBLASLT_SO "/opt/rocm/lib/libhipblaslt.so.1"
#endif

namespace dadgpt::gen {
namespace {

// The entry points used, with the header's own types.
struct LtApi {
  decltype(&hipblasLtCreate) create;
  decltype(&hipblasLtDestroy) destroy;
  decltype(&hipblasLtGetVersion) get_version;
  decltype(&hipblasLtMatmulDescCreate) desc_create;
  decltype(&hipblasLtMatmulDescDestroy) desc_destroy;
  decltype(&hipblasLtMatmulDescSetAttribute) desc_set;
  decltype(&hipblasLtMatrixLayoutCreate) layout_create;
  decltype(&hipblasLtMatrixLayoutDestroy) layout_destroy;
  decltype(&hipblasLtMatrixLayoutSetAttribute) layout_set;
  decltype(&hipblasLtMatmulPreferenceCreate) pref_create;
  decltype(&hipblasLtMatmulPreferenceDestroy) pref_destroy;
  decltype(&hipblasLtMatmulPreferenceSetAttribute) pref_set;
  decltype(&hipblasLtMatmulAlgoGetHeuristic) heuristic;
  decltype(&hipblasLtMatmul) matmul;
};

std::string g_api_error;

const LtApi* api() {
  static LtApi a{};
  static const LtApi* loaded = nullptr;
  static std::once_flag once;
  std::call_once(once, [] {
    void* so = dlopen(DADGPT_HIPBLASLT_SO, RTLD_NOW | RTLD_LOCAL | RTLD_DEEPBIND);
    if (!so) {
      const char* e = dlerror();
      g_api_error = std::string("cannot open " DADGPT_HIPBLASLT_SO
                                " (a process that loaded another hipBLASLt/rocRoller first, "
                                "such as PyTorch's, must load this library before it: in Python, "
                                "import dadgpt_amd before torch): ") +
                    std::string(e ? e : "?").substr(0, 160);
      return;
    }
    bool ok = true;
    auto sym = [&](auto& fn, const char* name) {
      fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(so, name));
      if (!fn) {
        ok = false;
        g_api_error = std::string(DADGPT_HIPBLASLT_SO " has no symbol ") + name;
      }
    };
    sym(a.create, "hipblasLtCreate");
    sym(a.destroy, "hipblasLtDestroy");
    sym(a.get_version, "hipblasLtGetVersion");
    sym(a.desc_create, "hipblasLtMatmulDescCreate");
    sym(a.desc_destroy, "hipblasLtMatmulDescDestroy");
    sym(a.desc_set, "hipblasLtMatmulDescSetAttribute");
    sym(a.layout_create, "hipblasLtMatrixLayoutCreate");
    sym(a.layout_destroy, "hipblasLtMatrixLayoutDestroy");
    sym(a.layout_set, "hipblasLtMatrixLayoutSetAttribute");
    sym(a.pref_create, "hipblasLtMatmulPreferenceCreate");
    sym(a.pref_destroy, "hipblasLtMatmulPreferenceDestroy");
    sym(a.pref_set, "hipblasLtMatmulPreferenceSetAttribute");
    sym(a.heuristic, "hipblasLtMatmulAlgoGetHeuristic");
    sym(a.matmul, "hipblasLtMatmul");
    if (ok) loaded = &a;  // the handle stays open until the process ends
  });
  return loaded;
}

constexpr int kCompiledVersion =
    HIPBLASLT_VERSION_MAJOR * 100000 + HIPBLASLT_VERSION_MINOR * 100 + HIPBLASLT_VERSION_PATCH;
// HIP runtimes (major, minor) that the GPU tests run this hipBLASLt on: PyTorch's ROCm 7.0
// runtime (the Python test suite, which loads PyTorch's libamdhip64 first) and the 7.2 runtime
// of the ROCm installation whose hipBLASLt this is (tests/cxx/blas_stack_test.cpp, a C++ caller
// without PyTorch). The hipBLASLt must be the version the headers declare.
constexpr int kTestedRuntimes[][2] = {{7, 0}, {7, 2}};

bool stack_supported(int hip_runtime, int hipblaslt) {
  if (hipblaslt != kCompiledVersion) return false;
  const int major = hip_runtime / 10000000, minor = hip_runtime / 100000 % 100;
  for (const auto& t : kTestedRuntimes)
    if (t[0] == major && t[1] == minor) return true;
  return false;
}

constexpr size_t kWorkspaceBytes = 32u << 20;
constexpr int kCandidates = 16;

// Process-wide multiply precision, as the reference's g_compute_type (cuda/gpu_ops.cu:61-67).
std::atomic<int> g_precision{DADGPT_MATMUL_FP32};

}  // namespace
}  // namespace dadgpt::gen

// One GEMM problem: row-major out[M,N] (fp32) = op(a) op(b) (+ beta out), `count` matrices
// `s*` elements apart. op: 'N' (a [M,K], b [K,N]), 'A' (a [K,M] transposed), 'B' (b [N,K]
// transposed).
struct GemmKey {
  int M, N, K;
  char op;
  hipDataType in;
  hipblasComputeType_t compute;
  int count;
  long long sa, sb, sc;
  auto tie() const { return std::tie(M, N, K, op, in, compute, count, sa, sb, sc); }
  bool operator<(const GemmKey& o) const { return tie() < o.tie(); }
};

struct dadgpt_blas {
  hipblasLtHandle_t lt = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, ld = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    std::vector<hipblasLtMatmulAlgo_t> candidates;
    bool tuned = false;
  };
  std::map<GemmKey, Plan> plans;
  std::mutex mu;  // plans are built and tuned under it
};

namespace dadgpt::gen {
namespace {

int lt_fail(hipblasStatus_t s, const char* what) {
  return fail(DADGPT_ERR_HIP, "%s: hipBLASLt status %d", what, (int)s);
}

void destroy_plan(const LtApi* L, dadgpt_blas::Plan& p) {
  if (p.la) L->layout_destroy(p.la);
  if (p.lb) L->layout_destroy(p.lb);
  if (p.ld) L->layout_destroy(p.ld);
  if (p.desc) L->desc_destroy(p.desc);
}

hipblasStatus_t batch_layout(const LtApi* L, hipblasLtMatrixLayout_t l, int count,
                             long long stride) {
  if (count == 1) return HIPBLAS_STATUS_SUCCESS;
  const int32_t c = count;
  const int64_t s = stride;
  hipblasStatus_t st = L->layout_set(l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &c, sizeof(c));
  if (st != HIPBLAS_STATUS_SUCCESS) return st;
  return L->layout_set(l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &s, sizeof(s));
}

// Builds (or finds) the plan of one problem.
int plan_for(dadgpt_blas* h, const GemmKey& k, dadgpt_blas::Plan** out) {
  auto it = h->plans.find(k);
  if (it != h->plans.end()) {
    *out = &it->second;
    return DADGPT_OK;
  }
  const LtApi* L = api();
  dadgpt_blas::Plan p;
  auto bail = [&](int st) {
    destroy_plan(L, p);
    return st;
  };
  hipblasStatus_t s;
  if ((s = L->desc_create(&p.desc, k.compute, HIP_R_32F)) != HIPBLAS_STATUS_SUCCESS)
    return lt_fail(s, "hipblasLtMatmulDescCreate");
  // column-major: first operand b (transposed for 'B'), second operand a (transposed for 'A')
  const hipblasOperation_t op1 = k.op == 'B' ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  const hipblasOperation_t op2 = k.op == 'A' ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  if ((s = L->desc_set(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op1, sizeof(op1))) !=
          HIPBLAS_STATUS_SUCCESS ||
      (s = L->desc_set(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op2, sizeof(op2))) !=
          HIPBLAS_STATUS_SUCCESS)
    return bail(lt_fail(s, "hipblasLtMatmulDescSetAttribute"));
  // b as stored: [K,N] row-major = (N x K, ld N); transposed [N,K] = (K x N, ld K)
  s = k.op == 'B' ? L->layout_create(&p.la, k.in, k.K, k.N, k.K)
                  : L->layout_create(&p.la, k.in, k.N, k.K, k.N);
  if (s != HIPBLAS_STATUS_SUCCESS) return bail(lt_fail(s, "hipblasLtMatrixLayoutCreate(b)"));
  // a as stored: [M,K] row-major = (K x M, ld K); transposed [K,M] = (M x K, ld M)
  s = k.op == 'A' ? L->layout_create(&p.lb, k.in, k.M, k.K, k.M)
                  : L->layout_create(&p.lb, k.in, k.K, k.M, k.K);
  if (s != HIPBLAS_STATUS_SUCCESS) return bail(lt_fail(s, "hipblasLtMatrixLayoutCreate(a)"));
  if ((s = L->layout_create(&p.ld, HIP_R_32F, k.N, k.M, k.N)) != HIPBLAS_STATUS_SUCCESS)
    return bail(lt_fail(s, "hipblasLtMatrixLayoutCreate(out)"));
  if ((s = batch_layout(L, p.la, k.count, k.sb)) != HIPBLAS_STATUS_SUCCESS ||
      (s = batch_layout(L, p.lb, k.count, k.sa)) != HIPBLAS_STATUS_SUCCESS ||
      (s = batch_layout(L, p.ld, k.count, k.sc)) != HIPBLAS_STATUS_SUCCESS)
    return bail(lt_fail(s, "hipblasLtMatrixLayoutSetAttribute(batch)"));

  hipblasLtMatmulPreference_t pref = nullptr;
  if ((s = L->pref_create(&pref)) != HIPBLAS_STATUS_SUCCESS)
    return bail(lt_fail(s, "hipblasLtMatmulPreferenceCreate"));
  const uint64_t ws = h->workspace_bytes;
  s = L->pref_set(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
  hipblasLtMatmulHeuristicResult_t res[kCandidates];
  int n = 0;
  if (s == HIPBLAS_STATUS_SUCCESS)
    s = L->heuristic(h->lt, p.desc, p.la, p.lb, p.ld, p.ld, pref, kCandidates, res, &n);
  L->pref_destroy(pref);
  if (s != HIPBLAS_STATUS_SUCCESS) return bail(lt_fail(s, "hipblasLtMatmulAlgoGetHeuristic"));
  for (int i = 0; i < n && i < kCandidates; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= h->workspace_bytes)
      p.candidates.push_back(res[i].algo);
  if (p.candidates.empty())
    return bail(fail(DADGPT_ERR_UNSUPPORTED,
                     "hipBLASLt has no algorithm within a %zu-byte workspace for M=%d N=%d "
                     "K=%d op %c batch %d",
                     h->workspace_bytes, k.M, k.N, k.K, k.op, k.count));
  p.algo = p.candidates[0];
  *out = &(h->plans[k] = p);
  return DADGPT_OK;
}

hipblasStatus_t run(dadgpt_blas* h, dadgpt_blas::Plan* p, const hipblasLtMatmulAlgo_t& algo,
                    float* out, const void* a, const void* b, float beta, hipStream_t stream) {
  const float alpha = 1.0f;
  return api()->matmul(h->lt, p->desc, &alpha, b, p->la, a, p->lb, &beta, out, p->ld, out,
                       p->ld, &algo, h->workspace, h->workspace_bytes, stream);
}

// Times each candidate of a fresh plan on the call's operands (only for beta = 0: the output
// is rewritten by the call that follows), two rounds of three calls, and keeps the first
// candidate, in the heuristic's order, within kTieSlack of the fastest. Candidates differ in
// summation order, so the plan decides the product's bits; near-ties going to the earlier
// candidate make processes on different boxes with the same libraries pick the same plan
// unless the candidates' times differ by more than the slack. Skipped under stream capture.
constexpr float kTieSlack = 1.10f;
void tune(dadgpt_blas* h, dadgpt_blas::Plan* p, float* out, const void* a, const void* b,
          hipStream_t stream) {
  p->tuned = true;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (p->candidates.size() < 2 || hipStreamIsCapturing(stream, &cap) != hipSuccess ||
      cap != hipStreamCaptureStatusNone)
    return;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return;
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return;
  }
  const size_t n = p->candidates.size();
  std::vector<float> t(n, 1e30f);
  for (int round = 0; round < 2; ++round)
    for (size_t i = 0; i < n; ++i) {
      const auto& algo = p->candidates[i];
      if (run(h, p, algo, out, a, b, 0.0f, stream) != HIPBLAS_STATUS_SUCCESS) continue;
      bool ok = hipEventRecord(e0, stream) == hipSuccess;
      for (int r = 0; r < 3 && ok; ++r) ok = run(h, p, algo, out, a, b, 0.0f, stream) == 0;
      ok = ok && hipEventRecord(e1, stream) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
      float ms = 0.f;
      if (ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess && ms < t[i]) t[i] = ms;
    }
  float best = 1e30f;
  for (float x : t) best = x < best ? x : best;
  for (size_t i = 0; i < n; ++i)
    if (t[i] < 1e30f && t[i] <= best * kTieSlack) {
      p->algo = p->candidates[i];
      break;
    }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
}

int matmul(dadgpt_blas* h, GemmKey k, float* out, const void* a, const void* b, float beta,
           void* stream, const char* fn) {
  if (!h || !out || !a || !b) return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: null argument", fn);
  if (k.M < 1 || k.K < 1 || k.N < 1 || k.count < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: M=%d K=%d N=%d batch=%d must be positive", fn,
                k.M, k.K, k.N, k.count);
  if (k.count > 1 && (k.sa < 0 || k.sb < 0 || k.sc < 0))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: negative batch stride", fn);
  if (!std::isfinite(beta)) return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: beta not finite", fn);
  if (k.count == 1) k.sa = k.sb = k.sc = 0;
  std::lock_guard<std::mutex> lock(h->mu);
  dadgpt_blas::Plan* p = nullptr;
  if (int st = plan_for(h, k, &p)) return st;
  if (!p->tuned && beta == 0.0f) tune(h, p, out, a, b, (hipStream_t)stream);
  const hipblasStatus_t s = run(h, p, p->algo, out, a, b, beta, (hipStream_t)stream);
  if (s != HIPBLAS_STATUS_SUCCESS) return lt_fail(s, fn);
  return DADGPT_OK;
}

hipblasComputeType_t f32_compute() {
  // gfx950 has no TF32 format: TF32 requests run as full fp32, the more precise choice.
  return g_precision.load() == DADGPT_MATMUL_BF16 ? HIPBLAS_COMPUTE_32F_FAST_16BF
                                                   : HIPBLAS_COMPUTE_32F;
}

bool valid_op(int op) { return op == 'N' || op == 'A' || op == 'B'; }

// hipBLASLt ends the process when a handle is created with no device visible, so every
// handle creation checks for one first.
bool have_device() {
  int n = 0;
  return hipGetDeviceCount(&n) == hipSuccess && n > 0;
}

}  // namespace

int gemm(dadgpt_blas* h, float* out, const bf16* a, const bf16* b, int M, int K, int N,
         bool trans_b, hipStream_t stream) {
  GemmKey k{M, N, K, trans_b ? 'B' : 'N', HIP_R_16BF, HIPBLAS_COMPUTE_32F, 1, 0, 0, 0};
  return matmul(h, k, out, a, b, 0.0f, stream, "gemm");
}

int gemm_f32(dadgpt_blas* h, float* out, const float* a, const float* b, int M, int K, int N,
             char op, float beta, int count, long long sa, long long sb, long long sc,
             hipStream_t stream) {
  GemmKey k{M, N, K, op, HIP_R_32F, f32_compute(), count, sa, sb, sc};
  return matmul(h, k, out, a, b, beta, stream, "gemm_f32");
}

}  // namespace dadgpt::gen

using namespace dadgpt::gen;

extern "C" {

int dadgpt_blas_open(void) {
  if (!api()) return fail(DADGPT_ERR_UNSUPPORTED, "dadgpt_blas_open: %s", g_api_error.c_str());
  return DADGPT_OK;
}

int dadgpt_blas_create(dadgpt_blas** out) {
  if (!out) return fail(DADGPT_ERR_INVALID_ARGUMENT, "dadgpt_blas_create: null argument");
  const LtApi* L = api();
  if (!L) return fail(DADGPT_ERR_UNSUPPORTED, "dadgpt_blas_create: %s", g_api_error.c_str());
  if (!have_device()) return fail(DADGPT_ERR_HIP, "dadgpt_blas_create: no HIP device visible");
  auto* h = new dadgpt_blas();
  hipblasStatus_t s = L->create(&h->lt);
  if (s != HIPBLAS_STATUS_SUCCESS) {
    delete h;
    return lt_fail(s, "hipblasLtCreate");
  }
  int version = 0;
  if (L->get_version(h->lt, &version) != HIPBLAS_STATUS_SUCCESS || version != kCompiledVersion) {
    L->destroy(h->lt);
    delete h;
    return fail(DADGPT_ERR_UNSUPPORTED,
                "dadgpt_blas_create: " DADGPT_HIPBLASLT_SO " reports version %d, these sources "
                "were compiled against %d",
                version, kCompiledVersion);
  }
  int runtime = 0;
  if (hipRuntimeGetVersion(&runtime) != hipSuccess || !stack_supported(runtime, version)) {
    L->destroy(h->lt);
    delete h;
    return fail(DADGPT_ERR_UNSUPPORTED,
                "dadgpt_blas_create: HIP runtime %d.%d.%d with hipBLASLt %d is not a combination "
                "the GPU tests cover (HIP 7.0 or 7.2 with hipBLASLt %d)",
                runtime / 10000000, runtime / 100000 % 100, runtime % 100000, version,
                kCompiledVersion);
  }
  if (hipMalloc(&h->workspace, kWorkspaceBytes) != hipSuccess) {
    L->destroy(h->lt);
    delete h;
    return fail(DADGPT_ERR_HIP, "dadgpt_blas_create: hipMalloc of the workspace failed");
  }
  h->workspace_bytes = kWorkspaceBytes;
  *out = h;
  return DADGPT_OK;
}

void dadgpt_blas_destroy(dadgpt_blas* h) {
  if (!h) return;
  const LtApi* L = api();
  for (auto& [key, p] : h->plans) destroy_plan(L, p);
  (void)hipFree(h->workspace);
  L->destroy(h->lt);
  delete h;
}

int dadgpt_blas_stack_versions(int* hip_runtime, int* hipblaslt) {
  if (!hip_runtime || !hipblaslt)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "dadgpt_blas_stack_versions: null argument");
  *hip_runtime = -1;
  *hipblaslt = -1;
  if (hipRuntimeGetVersion(hip_runtime) != hipSuccess) *hip_runtime = -1;
  const LtApi* L = api();
  if (!L) return fail(DADGPT_ERR_UNSUPPORTED, "dadgpt_blas_stack_versions: %s", g_api_error.c_str());
  hipblasLtHandle_t lt = nullptr;
  if (have_device() && L->create(&lt) == HIPBLAS_STATUS_SUCCESS) {
    if (L->get_version(lt, hipblaslt) != HIPBLAS_STATUS_SUCCESS) *hipblaslt = -1;
    L->destroy(lt);
  }
  return DADGPT_OK;
}

int dadgpt_blas_stack_supported(int hip_runtime, int hipblaslt) {
  return stack_supported(hip_runtime, hipblaslt) ? 1 : 0;
}

int dadgpt_blas_library_version(dadgpt_blas* h) {
  int v = 0;
  if (!h || api()->get_version(h->lt, &v) != HIPBLAS_STATUS_SUCCESS) return -1;
  return v;
}

int dadgpt_set_matmul_precision(int precision) {
  if (precision != DADGPT_MATMUL_FP32 && precision != DADGPT_MATMUL_TF32 &&
      precision != DADGPT_MATMUL_BF16)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "dadgpt_set_matmul_precision: unknown value %d",
                precision);
  g_precision.store(precision);
  return DADGPT_OK;
}

int dadgpt_get_matmul_precision(void) { return g_precision.load(); }

int dadgpt_matmul_bf16(dadgpt_blas* h, float* out, const uint16_t* a, const uint16_t* b, int M,
                       int K, int N, void* stream) {
  GemmKey k{M, N, K, 'N', HIP_R_16BF, HIPBLAS_COMPUTE_32F, 1, 0, 0, 0};
  return matmul(h, k, out, a, b, 0.0f, stream, "dadgpt_matmul_bf16");
}

int dadgpt_matmul_transposed_b_bf16(dadgpt_blas* h, float* out, const uint16_t* a,
                                    const uint16_t* b, int M, int K, int N, void* stream) {
  GemmKey k{M, N, K, 'B', HIP_R_16BF, HIPBLAS_COMPUTE_32F, 1, 0, 0, 0};
  return matmul(h, k, out, a, b, 0.0f, stream, "dadgpt_matmul_transposed_b_bf16");
}

int dadgpt_matmul_f32(dadgpt_blas* h, float* out, const float* a, const float* b, int M, int K,
                      int N, int op, float beta, void* stream) {
  if (!valid_op(op))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "dadgpt_matmul_f32: op %d not 'N', 'A' or 'B'", op);
  GemmKey k{M, N, K, (char)op, HIP_R_32F, f32_compute(), 1, 0, 0, 0};
  return matmul(h, k, out, a, b, beta, stream, "dadgpt_matmul_f32");
}

int dadgpt_matmul_f32_strided_batched(dadgpt_blas* h, float* out, const float* a,
                                      const float* b, int M, int K, int N, int op, float beta,
                                      long long stride_a, long long stride_b,
                                      long long stride_out, int batch_count, void* stream) {
  if (!valid_op(op))
    return fail(DADGPT_ERR_INVALID_ARGUMENT,
                "dadgpt_matmul_f32_strided_batched: op %d not 'N', 'A' or 'B'", op);
  GemmKey k{M, N, K, (char)op, HIP_R_32F, f32_compute(), batch_count,
            stride_a, stride_b, stride_out};
  return matmul(h, k, out, a, b, beta, stream, "dadgpt_matmul_f32_strided_batched");
}

}  // extern "C"
