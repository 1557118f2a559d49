// Launch functions of the attention kernels (host side of each .hip file). Arguments are
// validated by capi.cpp before any of these is called; every function returns the
// hipGetLastError() status of its own launches.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dadgpt {

typedef __bf16 bf16;

// Where the rows of one (b, h) slice of a bf16 attention tensor lie: row s of slice
// bh = b * n_heads + h starts at element b * batch + h * head + s * row, and its D elements
// are contiguous. A contiguous [BH, S, D] tensor is {S * D, 0, D} with n_heads = 1; the
// token-major [B * S, H * D] layout of the projections is {S * H * D, D, H * D}. The host
// keeps every stride a multiple of 8 elements (16 bytes) and row below 2^24.
struct HeadStrides {
  long long batch, head;
  int row;
};
enum AttnTensor { kTQ, kTK, kTV, kTO, kTDO, kTDQ, kTDK, kTDV, kAttnTensors };
struct AttnLayout {
  int n_heads;
  HeadStrides t[kAttnTensors];
};

inline AttnLayout contiguous_layout(int S, int D) {
  AttnLayout L{};
  L.n_heads = 1;
  for (auto& t : L.t) t = HeadStrides{(long long)S * D, 0, D};
  return L;
}

// Whether `L` places every tensor as contiguous [BH, S, D] (the kernels then use their
// compile-time contiguous addressing). Unit-stride heads count: b * H * S * D + h * S * D is
// the same element as bh * S * D.
inline bool is_contiguous(const AttnLayout& L, int S, int D) {
  const long long slice = (long long)S * D;
  for (const auto& t : L.t)
    if (t.row != D || t.head != slice || t.batch != slice * L.n_heads) {
      if (L.n_heads == 1 && t.row == D && t.batch == slice) continue;  // head unused
      return false;
    }
  return true;
}

// Attention-probability dropout of a call: rate p in [0, 1) and the generator's seed (the
// mask definition is in dropout.hpp). The host checks p; dropout runs on the contiguous
// layout only.
struct Dropout {
  float p;
  uint64_t seed;
};

// Causal flash forward, bf16 in/out, fp32 logsumexp (natural log) [BH, S]. q, k, v, out as
// `layout` places them (tensors kTQ, kTK, kTV, kTO), D in {32,64}. With `drop`, the
// probabilities multiplying V are dropped (the logsumexp is that of the undropped scores).
hipError_t launch_fwd_bf16(bf16* out, float* lse, const bf16* q, const bf16* k, const bf16* v,
                           int BH, int S, int D, float scale, const AttnLayout& layout,
                           hipStream_t stream, const Dropout* drop = nullptr);

// Causal flash backward, bf16 in/out. delta [BH,S] fp32 is written (scratch, as the
// reference's). dq/dk/dv are overwritten. `phases` selects the kernels launched, in order:
// bit 1 dQ (which also computes and writes delta), bit 2 dK/dV (reads delta); kBwdAll is the
// whole backward. Bit 0 launches the standalone delta kernel (a separate pass, equal up to
// fp32 summation order; not part of kBwdAll).
constexpr int kBwdDelta = 1, kBwdDq = 2, kBwdDkdv = 4, kBwdAll = kBwdDq | kBwdDkdv;
hipError_t launch_bwd_bf16(bf16* dq, bf16* dk, bf16* dv, float* delta, const bf16* dout,
                           const bf16* out, const float* lse, const bf16* q, const bf16* k,
                           const bf16* v, int BH, int S, int D, float scale,
                           const AttnLayout& layout, hipStream_t stream, int phases = kBwdAll,
                           const Dropout* drop = nullptr);

// fp32 flash forward/backward (the reference's own precision), optionally with dropout.
hipError_t launch_fwd_f32(float* out, float* lse, const float* q, const float* k,
                          const float* v, int BH, int S, int D, float scale, hipStream_t stream,
                          const Dropout* drop = nullptr);
hipError_t launch_bwd_f32(float* dq, float* dk, float* dv, float* delta, const float* dout,
                          const float* out, const float* lse, const float* q, const float* k,
                          const float* v, int BH, int S, int D, float scale,
                          hipStream_t stream, const Dropout* drop = nullptr);

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

// Row kernels of the materialized attention path (materialized.hip), fp32 [rows, cols]:
// the reference's softmax (out may be in), softmax backward (din += p (dout - rowsum(dout p))),
// causal fill of n_blocks S x S blocks (value above the diagonal) and scale; and the fused
// chains: attention_probs turns raw scores [BH, S, S] into probabilities in place (x scale,
// causal mask, softmax), attention_probs_backward writes d(scores) from d(probs) and probs
// (softmax backward, causal zero, x scale; ds may be dp), decode_probs turns decode scores
// [n_seq * H, max_len] into probabilities over each sequence's first lens[seq] keys.
hipError_t launch_softmax_rows(float* out, const float* in, long long rows, int cols,
                               hipStream_t stream);
hipError_t launch_softmax_backward_rows(float* din, const float* dout, const float* p,
                                        long long rows, int cols, hipStream_t stream);
hipError_t launch_causal_fill(float* m, int n_blocks, int S, float value, hipStream_t stream);
hipError_t launch_scale(float* x, long long n, float scale, hipStream_t stream);
hipError_t launch_attention_probs(float* p, int BH, int S, float scale, hipStream_t stream);
hipError_t launch_attention_probs_backward(float* ds, const float* dp, const float* p, int BH,
                                           int S, float scale, hipStream_t stream);
hipError_t launch_decode_probs(float* p, const int* lens, int n_seq, int H, int max_len,
                               float scale, hipStream_t stream);
// Attention-probability dropout of the materialized path, with the flash kernels' mask
// (dropout.hpp): out [BH, S, S] = p * keep / (1 - drop.p) (out may be p); and the backward row
// pass ds = causal_zero(softmax_backward(dpd * keep / (1 - drop.p), p)) * scale (ds may be dpd).
hipError_t launch_attention_dropout(float* out, const float* p, int BH, int S,
                                   const Dropout& drop, hipStream_t stream);
hipError_t launch_attention_probs_backward_dropout(float* ds, const float* dpd, const float* p,
                                                   int BH, int S, float scale,
                                                   const Dropout& drop, hipStream_t stream);
// The reference's head split [B*S, H*dh] -> [B*H, S, dh] and merge (its inverse), fp32
// (materialized.hip). out and in do not overlap; B*S < 2^31 rows.
hipError_t launch_split_heads(float* out, const float* in, int B, int S, int H, int dh,
                              hipStream_t stream);
hipError_t launch_merge_heads(float* out, const float* in, int B, int S, int H, int dh,
                              hipStream_t stream);

// Device scratch that stands in for the decode workspace in the allocation-free entry point:
// kDecodeScratchBytes per device, held until the process ends. decode_scratch returns the
// current device's address, looked up (and zero-filled by a kernel on `stream`) on the first
// call on that device.
constexpr size_t kDecodeScratchBytes = size_t(4) << 20;
hipError_t decode_scratch(void** ptr, hipStream_t stream);

}  // namespace dadgpt
