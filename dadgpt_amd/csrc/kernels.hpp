// Launch functions of the attention kernels (host side of each .hip file). Arguments are
// validated by capi.cpp before any of these is called; every function returns the
// hipGetLastError() status of its own launches.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dadgpt {

typedef __bf16 bf16;

// Causal flash forward, bf16 in/out, fp32 logsumexp (natural log). [BH,S,D], D in {32,64}.
hipError_t launch_fwd_bf16(bf16* out, float* lse, const bf16* q, const bf16* k, const bf16* v,
                           int BH, int S, int D, float scale, hipStream_t stream);

// Causal flash backward, bf16 in/out. delta [BH,S] fp32 is written (scratch, as the
// reference's). dq/dk/dv are overwritten. `phases` selects the kernels launched, in order:
// bit 0 delta, bit 1 dQ, bit 2 dK/dV (kBwdAll for the whole backward).
constexpr int kBwdDelta = 1, kBwdDq = 2, kBwdDkdv = 4, kBwdAll = 7;
hipError_t launch_bwd_bf16(bf16* dq, bf16* dk, bf16* dv, float* delta, const bf16* dout,
                           const bf16* out, const float* lse, const bf16* q, const bf16* k,
                           const bf16* v, int BH, int S, int D, float scale, hipStream_t stream,
                           int phases = kBwdAll);

// fp32 flash forward/backward (the reference's own precision).
hipError_t launch_fwd_f32(float* out, float* lse, const float* q, const float* k,
                          const float* v, int BH, int S, int D, float scale, hipStream_t stream);
hipError_t launch_bwd_f32(float* dq, float* dk, float* dv, float* delta, const float* dout,
                          const float* out, const float* lse, const float* q, const float* k,
                          const float* v, int BH, int S, int D, float scale,
                          hipStream_t stream);

// Decode over ragged KV caches [n_seq,H,max_len,D]. A cache longer than one workgroup chunk
// (512 keys bf16, 256 fp32 at D=64) is split into chunks merged inside the kernel through the
// workspace: arrival counters at its start, fp32 partials packed against its end (its full
// size, workspace_bytes, places them). decode_workspace_bytes is 0 when no split is needed.
size_t decode_workspace_bytes(int n_seq, int H, int max_len, int D);
hipError_t launch_decode_bf16(bf16* out, const bf16* q, const bf16* k_cache,
                              const bf16* v_cache, const int* lens, int n_seq, int H,
                              int max_len, int D, float scale, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);
hipError_t launch_decode_f32(float* out, const float* q, const float* k_cache,
                             const float* v_cache, const int* lens, int n_seq, int H,
                             int max_len, int D, float scale, void* workspace,
                             size_t workspace_bytes, hipStream_t stream);

}  // namespace dadgpt
