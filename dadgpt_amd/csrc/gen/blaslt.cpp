// hipBLASLt bf16 GEMMs behind the reference's row-major matmul wrappers
// (cuda/gpu_ops.cu:94-112). hipBLASLt is column-major: a row-major X[R,C] is the column-major
// matrix X^T (C rows, R cols, leading dimension C), so
//   out[M,N] = a[M,K] b[K,N]    is  out^T[N,M] = b^T[N,K] a^T[K,M]    (both operands as stored)
//   out[M,N] = a[M,K] b[N,K]^T  is  out^T[N,M] = (b^T)^T[N,K] a^T[K,M] (first operand transposed)
// One plan (descriptors, layouts, an algorithm) is built per distinct shape and reused; the
// 32 MiB workspace is allocated once per handle. The first call of a shape (outside stream
// capture) times up to 16 of the heuristic's candidates on the call's own operands and keeps
// the fastest: for the skinny decode shapes (M = batch) the heuristic's first choice was up to
// several times slower than the best candidate.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdio>
#include <map>
#include <tuple>
#include <vector>

#include "dadgpt/gpu_attention.h"
#include "dadgpt/gpu_matmul.h"
#include "gen_internal.hpp"

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
  std::map<std::tuple<int, int, int, int>, Plan> plans;  // (M, N, K, transposed_b)
};

namespace dadgpt::gen {

namespace {

constexpr size_t kWorkspaceBytes = 32u << 20;
constexpr int kCandidates = 16;

int lt_fail(hipblasStatus_t s, const char* what) {
  return fail(DADGPT_ERR_HIP, "%s: hipBLASLt status %d", what, (int)s);
}

// Builds (or finds) the plan of one shape.
int plan_for(dadgpt_blas* h, int M, int N, int K, bool trans_b, dadgpt_blas::Plan** out) {
  const auto key = std::make_tuple(M, N, K, trans_b ? 1 : 0);
  auto it = h->plans.find(key);
  if (it != h->plans.end()) {
    *out = &it->second;
    return DADGPT_OK;
  }
  dadgpt_blas::Plan p;
  hipblasStatus_t s;
  if ((s = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F)) !=
      HIPBLAS_STATUS_SUCCESS)
    return lt_fail(s, "hipblasLtMatmulDescCreate");
  const hipblasOperation_t op_a = trans_b ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  const hipblasOperation_t op_b = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_a, sizeof(op_a));
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_b, sizeof(op_b));
  // first operand: the weight as stored (N x K, ld N) or, transposed, (K x N, ld K)
  if (trans_b)
    s = hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, K, N, K);
  else
    s = hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, N, K, N);
  if (s != HIPBLAS_STATUS_SUCCESS) return lt_fail(s, "hipblasLtMatrixLayoutCreate(A)");
  if ((s = hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, K, M, K)) != HIPBLAS_STATUS_SUCCESS)
    return lt_fail(s, "hipblasLtMatrixLayoutCreate(B)");
  if ((s = hipblasLtMatrixLayoutCreate(&p.ld, HIP_R_32F, N, M, N)) != HIPBLAS_STATUS_SUCCESS)
    return lt_fail(s, "hipblasLtMatrixLayoutCreate(D)");

  hipblasLtMatmulPreference_t pref = nullptr;
  if ((s = hipblasLtMatmulPreferenceCreate(&pref)) != HIPBLAS_STATUS_SUCCESS)
    return lt_fail(s, "hipblasLtMatmulPreferenceCreate");
  const uint64_t ws = h->workspace_bytes;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                        sizeof(ws));
  hipblasLtMatmulHeuristicResult_t res[kCandidates];
  int n = 0;
  s = hipblasLtMatmulAlgoGetHeuristic(h->lt, p.desc, p.la, p.lb, p.ld, p.ld, pref, kCandidates,
                                      res, &n);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (s != HIPBLAS_STATUS_SUCCESS || n < 1)
    return fail(DADGPT_ERR_HIP, "hipBLASLt has no algorithm for M=%d N=%d K=%d%s (status %d)",
                M, N, K, trans_b ? " (b transposed)" : "", (int)s);
  p.algo = res[0].algo;
  for (int i = 0; i < n; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS) p.candidates.push_back(res[i].algo);
  *out = &(h->plans[key] = p);
  return DADGPT_OK;
}

// Times each candidate of a fresh plan on the call's operands (the output is rewritten by the
// call that follows) and keeps the fastest. Skipped while the stream is being captured.
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
  const float alpha = 1.0f, beta = 0.0f;
  float best = 1e30f;
  for (const auto& algo : p->candidates) {
    auto run = [&] {
      return hipblasLtMatmul(h->lt, p->desc, &alpha, b, p->la, a, p->lb, &beta, out, p->ld, out,
                             p->ld, &algo, h->workspace, h->workspace_bytes, stream);
    };
    if (run() != HIPBLAS_STATUS_SUCCESS) continue;
    bool ok = hipEventRecord(e0, stream) == hipSuccess;
    for (int r = 0; r < 3 && ok; ++r) ok = run() == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipEventRecord(e1, stream) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
    float ms = 0.f;
    if (ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess && ms < best) {
      best = ms;
      p->algo = algo;
    }
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
}

int matmul(dadgpt_blas* h, float* out, const uint16_t* a, const uint16_t* b, int M, int K, int N,
           bool trans_b, void* stream, const char* fn) {
  if (!h || !out || !a || !b) return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: null argument", fn);
  if (M < 1 || K < 1 || N < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: M=%d K=%d N=%d must be positive", fn, M, K, N);
  dadgpt_blas::Plan* p = nullptr;
  if (int st = plan_for(h, M, N, K, trans_b, &p)) return st;
  if (!p->tuned) tune(h, p, out, a, b, (hipStream_t)stream);
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t s =
      hipblasLtMatmul(h->lt, p->desc, &alpha, b, p->la, a, p->lb, &beta, out, p->ld, out, p->ld,
                      &p->algo, h->workspace, h->workspace_bytes, (hipStream_t)stream);
  if (s != HIPBLAS_STATUS_SUCCESS) return lt_fail(s, fn);
  return DADGPT_OK;
}

}  // namespace

int gemm(dadgpt_blas* h, float* out, const bf16* a, const bf16* b, int M, int K, int N,
         bool trans_b, hipStream_t stream) {
  return matmul(h, out, reinterpret_cast<const uint16_t*>(a),
                reinterpret_cast<const uint16_t*>(b), M, K, N, trans_b, stream, "gemm");
}

}  // namespace dadgpt::gen

using namespace dadgpt::gen;

extern "C" {

int dadgpt_blas_create(dadgpt_blas** out) {
  if (!out) return fail(DADGPT_ERR_INVALID_ARGUMENT, "dadgpt_blas_create: null argument");
  auto* h = new dadgpt_blas();
  hipblasStatus_t s = hipblasLtCreate(&h->lt);
  if (s != HIPBLAS_STATUS_SUCCESS) {
    delete h;
    return lt_fail(s, "hipblasLtCreate");
  }
  if (hipMalloc(&h->workspace, kWorkspaceBytes) != hipSuccess) {
    hipblasLtDestroy(h->lt);
    delete h;
    return fail(DADGPT_ERR_HIP, "dadgpt_blas_create: hipMalloc of the workspace failed");
  }
  h->workspace_bytes = kWorkspaceBytes;
  *out = h;
  return DADGPT_OK;
}

void dadgpt_blas_destroy(dadgpt_blas* h) {
  if (!h) return;
  for (auto& [key, p] : h->plans) {
    hipblasLtMatrixLayoutDestroy(p.la);
    hipblasLtMatrixLayoutDestroy(p.lb);
    hipblasLtMatrixLayoutDestroy(p.ld);
    hipblasLtMatmulDescDestroy(p.desc);
  }
  (void)hipFree(h->workspace);
  hipblasLtDestroy(h->lt);
  delete h;
}

int dadgpt_matmul_bf16(dadgpt_blas* h, float* out, const uint16_t* a, const uint16_t* b, int M,
                       int K, int N, void* stream) {
  return matmul(h, out, a, b, M, K, N, false, stream, "dadgpt_matmul_bf16");
}

int dadgpt_matmul_transposed_b_bf16(dadgpt_blas* h, float* out, const uint16_t* a,
                                    const uint16_t* b, int M, int K, int N, void* stream) {
  return matmul(h, out, a, b, M, K, N, true, stream, "dadgpt_matmul_transposed_b_bf16");
}

}  // extern "C"
