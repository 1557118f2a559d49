// extern "C" entry points of libdadgpt_attn.so (declared in include/dadgpt/gpu_attention.h).
// Every argument check runs on the host before any HIP call, so each error path can be
// exercised on a machine without a GPU; a failing call records a thread-local message and
// returns a status instead of throwing across the C boundary.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>

#include "dadgpt/gpu_attention.h"
#include "kernels.hpp"

namespace {

thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int ok() {
  g_last_error[0] = '\0';
  return DADGPT_OK;
}

int from_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(DADGPT_ERR_HIP, "%s: HIP error %d (%s)", what, static_cast<int>(e),
              hipGetErrorString(e));
}

bool supported(int d_head) { return d_head == 32 || d_head == 64; }

// Tensors are read with 16-byte vector loads: every buffer must be non-null and 16-byte
// aligned (any contiguous [BH,S,D] tensor from a device allocator is).
int check_ptrs(const char* fn, std::initializer_list<const void*> ptrs) {
  int i = 0;
  for (const void* p : ptrs) {
    if (p == nullptr)
      return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: pointer argument %d is null", fn, i);
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: pointer argument %d is not 16-byte aligned",
                  fn, i);
    ++i;
  }
  return DADGPT_OK;
}

// Launch limits. Row and stride arithmetic in the kernels is 32-bit (row counts up to 2^24);
// every attention grid is (BH, ceil(S / tile)) with tiles of at least 64 rows and
// grid.y <= 65535; a dispatch counts its work-items along x in 32 bits (BH workgroups of at
// most 256 lanes; 8 lanes per row in the delta kernel).
constexpr long kMaxRows = 1L << 24;
constexpr long kMaxSeq = 65535L * 64;

int check_attn(const char* fn, int BH, int S, int d_head, float scale,
               std::initializer_list<const void*> ptrs) {
  if (int st = check_ptrs(fn, ptrs)) return st;
  if (BH < 1 || S < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: BH=%d and S=%d must be positive", fn, BH, S);
  if (S > kMaxSeq)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: S=%d exceeds %ld", fn, S, kMaxSeq);
  if (BH >= kMaxRows || (long long)BH * S > (1LL << 29))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: BH=%d x S=%d too large", fn, BH, S);
  if (!supported(d_head))
    return fail(DADGPT_ERR_UNSUPPORTED, "flash attention: unsupported d_head %d", d_head);
  if (!std::isfinite(scale))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: scale must be finite", fn);
  return DADGPT_OK;
}

// Decode shape: grid (n_seq * H, chunks) of 512-lane workgroups, so n_seq * H * 512 < 2^32
// work-items and at most 65535 chunks of the shortest chunk (256 keys, fp32 at d_head 64).
int check_decode_shape(const char* fn, int n_seq, int H, int max_len, int d_head, float scale,
                       std::initializer_list<const void*> ptrs) {
  if (int st = check_ptrs(fn, ptrs)) return st;
  if (n_seq < 1 || H < 1 || max_len < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT,
                "%s: n_seq=%d, n_heads=%d, max_len=%d must be positive", fn, n_seq, H, max_len);
  if ((long long)n_seq * H >= (1LL << 23) || max_len > 65535L * 256)
    return fail(DADGPT_ERR_INVALID_ARGUMENT,
                "%s: n_seq=%d x n_heads=%d or max_len=%d exceeds the launch limits", fn, n_seq,
                H, max_len);
  if (!supported(d_head))
    return fail(DADGPT_ERR_UNSUPPORTED, "decode attention: unsupported d_head %d", d_head);
  if (!std::isfinite(scale))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: scale must be finite", fn);
  return DADGPT_OK;
}

int check_decode(const char* fn, int n_seq, int H, int max_len, int d_head, float scale,
                 const void* ws, size_t ws_bytes, std::initializer_list<const void*> ptrs) {
  if (int st = check_decode_shape(fn, n_seq, H, max_len, d_head, scale, ptrs)) return st;
  const size_t need = dadgpt::decode_workspace_bytes(n_seq, H, max_len, d_head);
  if (need > 0 && (ws == nullptr || ws_bytes < need))
    return fail(DADGPT_ERR_WORKSPACE, "%s: workspace of %zu bytes given, %zu needed", fn,
                ws == nullptr ? 0 : ws_bytes, need);
  return DADGPT_OK;
}

// Row kernels of the materialized path: fp32 [rows, cols] matrices, 4-byte aligned, one wave
// per row (rows / 4 workgroups of 256 lanes: rows * 64 work-items < 2^32).
int check_rows(const char* fn, long long rows, long long cols,
               std::initializer_list<const void*> ptrs) {
  int i = 0;
  for (const void* p : ptrs) {
    if (p == nullptr)
      return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: pointer argument %d is null", fn, i);
    if (reinterpret_cast<uintptr_t>(p) % 4 != 0)
      return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: pointer argument %d is not 4-byte aligned",
                  fn, i);
    ++i;
  }
  if (rows < 1 || cols < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: rows=%lld and cols=%lld must be positive", fn,
                rows, cols);
  if (rows >= (1LL << 26) || cols > kMaxRows)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: rows=%lld x cols=%lld exceeds the launch limits",
                fn, rows, cols);
  return DADGPT_OK;
}

// n_blocks square S x S blocks ([BH, S, S] scores).
int check_blocks(const char* fn, int n_blocks, int S, const void* p) {
  if (n_blocks < 1 || S < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: n_blocks=%d and S=%d must be positive", fn,
                n_blocks, S);
  return check_rows(fn, (long long)n_blocks * S, S, {p});
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

int check_dropout(const char* fn, float p) {
  if (!(p >= 0.0f && p < 1.0f))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: dropout_p must be in [0, 1), got %g", fn,
                (double)p);
  return DADGPT_OK;
}

// Strides of the strided/token-major calls: non-negative multiples of 8 elements (the kernels
// move 16-byte pieces), rows at least d_head apart and at most 2^24 (64 rows of a tile stay
// within a 32-bit byte offset). Converts them to the kernels' layout.
int check_strides(const char* fn, int B, int H, int S, int d_head,
                  const dadgpt_head_strides* strides, int count, dadgpt::AttnLayout* L) {
  static const char* names[] = {"q", "k", "v", "out", "dout", "dq", "dk", "dv"};
  if (strides == nullptr)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: strides is null", fn);
  if (B < 1 || H < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: B=%d and H=%d must be positive", fn, B, H);
  if ((long long)B * H > kMaxRows)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: B=%d x H=%d too large", fn, B, H);
  *L = dadgpt::contiguous_layout(S, d_head);
  L->n_heads = H;
  for (int i = 0; i < count; ++i) {
    const dadgpt_head_strides& t = strides[i];
    if (t.batch < 0 || t.head < 0 || t.row < d_head || t.row > kMaxRows || t.batch % 8 != 0 ||
        t.head % 8 != 0 || t.row % 8 != 0)
      return fail(DADGPT_ERR_INVALID_ARGUMENT,
                  "%s: strides of %s {batch %lld, head %lld, row %lld}: each must be a "
                  "non-negative multiple of 8, with d_head (%d) <= row <= 2^24",
                  fn, names[i], (long long)t.batch, (long long)t.head, (long long)t.row,
                  d_head);
    L->t[i] = dadgpt::HeadStrides{t.batch, t.head, (int)t.row};
  }
  return DADGPT_OK;
}

// Token-major rows hold all H heads side by side: every leading dimension is at least H*d_head.
int check_ld(const char* fn, int H, int d_head, std::initializer_list<int64_t> lds) {
  for (int64_t ld : lds)
    if (ld < (int64_t)H * d_head || ld > kMaxRows)
      return fail(DADGPT_ERR_INVALID_ARGUMENT,
                  "%s: leading dimension %lld outside [n_heads x d_head = %lld, 2^24]", fn,
                  (long long)ld, (long long)H * d_head);
  return DADGPT_OK;
}

// Token-major strides: row b*S + s holds the H heads side by side, rows ld elements apart.
dadgpt_head_strides tokens(int64_t ld, int S, int d_head) {
  return dadgpt_head_strides{ld * S, d_head, ld};
}

static_assert(DADGPT_DECODE_NOALLOC_SCRATCH_BYTES == dadgpt::kDecodeScratchBytes,
              "the header's scratch limit must be the kernels' own");

using dadgpt::bf16;
const bf16* B(const uint16_t* p) { return reinterpret_cast<const bf16*>(p); }
bf16* B(uint16_t* p) { return reinterpret_cast<bf16*>(p); }

// Shared checks of the head split and merge: positive sizes; one workgroup of at most 256
// lanes per token row (rows below 2^24, so the work-items fit 32 bits) and rows of fewer than
// 2^31 elements (32-bit column indices); non-null buffers that do not overlap.
int check_heads(const char* fn, float* out, const float* in, int B, int S, int H, int dh) {
  if (!out || !in) return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: null buffer", fn);
  if (B < 1 || S < 1 || H < 1 || dh < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT,
                "%s: batch_size=%d, seq_len=%d, n_heads=%d, d_head=%d must be positive", fn, B,
                S, H, dh);
  const long long rows = (long long)B * S, D = (long long)H * dh;
  if (rows >= kMaxRows || D > INT32_MAX)
    return fail(DADGPT_ERR_INVALID_ARGUMENT,
                "%s: %lld token rows of %lld elements exceed the launch limits", fn, rows, D);
  const uintptr_t o = reinterpret_cast<uintptr_t>(out), i = reinterpret_cast<uintptr_t>(in);
  const uintptr_t bytes = (uintptr_t)(rows * D) * sizeof(float);
  if (o < i + bytes && i < o + bytes)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: out and in overlap", fn);
  return DADGPT_OK;
}

}  // namespace

extern "C" {

const char* dadgpt_last_error(void) { return g_last_error; }

const char* dadgpt_status_string(int status) {
  switch (status) {
    case DADGPT_OK: return "ok";
    case DADGPT_ERR_INVALID_ARGUMENT: return "invalid argument";
    case DADGPT_ERR_UNSUPPORTED: return "unsupported";
    case DADGPT_ERR_HIP: return "hip error";
    case DADGPT_ERR_WORKSPACE: return "workspace";
    default: return "unknown status";
  }
}

const char* dadgpt_version(void) { return "dadgpt-mi355x attention 0.1 (gfx950)"; }

int dadgpt_flash_attention_supported(int d_head) { return supported(d_head) ? 1 : 0; }

int dadgpt_flash_attention_forward_async(float* out, float* lse, const float* q, const float* k,
                                         const float* v, int BH, int S, int d_head,
                                         float scale, void* stream) {
  const char* fn = "dadgpt_flash_attention_forward";
  if (int st = check_attn(fn, BH, S, d_head, scale, {out, lse, q, k, v})) return st;
  return from_hip(dadgpt::launch_fwd_f32(out, lse, q, k, v, BH, S, d_head, scale,
                                         as_stream(stream)),
                  fn);
}

int dadgpt_flash_attention_forward(float* out, float* lse, const float* q, const float* k,
                                   const float* v, int BH, int S, int d_head, float scale) {
  return dadgpt_flash_attention_forward_async(out, lse, q, k, v, BH, S, d_head, scale, nullptr);
}

int dadgpt_flash_attention_backward_async(float* dq, float* dk, float* dv, float* delta,
                                          const float* dout, const float* out,
                                          const float* lse, const float* q, const float* k,
                                          const float* v, int BH, int S, int d_head,
                                          float scale, void* stream) {
  const char* fn = "dadgpt_flash_attention_backward";
  if (int st = check_attn(fn, BH, S, d_head, scale, {dq, dk, dv, delta, dout, out, lse, q, k, v}))
    return st;
  return from_hip(dadgpt::launch_bwd_f32(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S,
                                         d_head, scale, as_stream(stream)),
                  fn);
}

int dadgpt_flash_attention_backward(float* dq, float* dk, float* dv, float* delta,
                                    const float* dout, const float* out, const float* lse,
                                    const float* q, const float* k, const float* v, int BH,
                                    int S, int d_head, float scale) {
  return dadgpt_flash_attention_backward_async(dq, dk, dv, delta, dout, out, lse, q, k, v, BH,
                                               S, d_head, scale, nullptr);
}

int dadgpt_flash_attention_forward_bf16(uint16_t* out, float* lse, const uint16_t* q,
                                        const uint16_t* k, const uint16_t* v, int BH, int S,
                                        int d_head, float scale, void* stream) {
  const char* fn = "dadgpt_flash_attention_forward_bf16";
  if (int st = check_attn(fn, BH, S, d_head, scale, {out, lse, q, k, v})) return st;
  return from_hip(dadgpt::launch_fwd_bf16(B(out), lse, B(q), B(k), B(v), BH, S, d_head, scale,
                                          dadgpt::contiguous_layout(S, d_head),
                                          as_stream(stream)),
                  fn);
}

int dadgpt_flash_attention_backward_bf16(uint16_t* dq, uint16_t* dk, uint16_t* dv,
                                         float* delta, const uint16_t* dout,
                                         const uint16_t* out, const float* lse,
                                         const uint16_t* q, const uint16_t* k,
                                         const uint16_t* v, int BH, int S, int d_head,
                                         float scale, void* stream) {
  const char* fn = "dadgpt_flash_attention_backward_bf16";
  if (int st = check_attn(fn, BH, S, d_head, scale, {dq, dk, dv, delta, dout, out, lse, q, k, v}))
    return st;
  return from_hip(dadgpt::launch_bwd_bf16(B(dq), B(dk), B(dv), delta, B(dout), B(out), lse,
                                          B(q), B(k), B(v), BH, S, d_head, scale,
                                          dadgpt::contiguous_layout(S, d_head),
                                          as_stream(stream)),
                  fn);
}

int dadgpt_flash_attention_forward_bf16_dropout(uint16_t* out, float* lse, const uint16_t* q,
                                                const uint16_t* k, const uint16_t* v, int BH,
                                                int S, int d_head, float scale,
                                                float dropout_p, uint64_t seed, void* stream) {
  const char* fn = "dadgpt_flash_attention_forward_bf16_dropout";
  if (int st = check_attn(fn, BH, S, d_head, scale, {out, lse, q, k, v})) return st;
  if (int st = check_dropout(fn, dropout_p)) return st;
  const dadgpt::Dropout drop{dropout_p, seed};
  return from_hip(dadgpt::launch_fwd_bf16(B(out), lse, B(q), B(k), B(v), BH, S, d_head, scale,
                                          dadgpt::contiguous_layout(S, d_head),
                                          as_stream(stream), &drop),
                  fn);
}

int dadgpt_flash_attention_backward_bf16_dropout(uint16_t* dq, uint16_t* dk, uint16_t* dv,
                                                 float* delta, const uint16_t* dout,
                                                 const uint16_t* out, const float* lse,
                                                 const uint16_t* q, const uint16_t* k,
                                                 const uint16_t* v, int BH, int S, int d_head,
                                                 float scale, float dropout_p, uint64_t seed,
                                                 void* stream) {
  const char* fn = "dadgpt_flash_attention_backward_bf16_dropout";
  if (int st = check_attn(fn, BH, S, d_head, scale, {dq, dk, dv, delta, dout, out, lse, q, k, v}))
    return st;
  if (int st = check_dropout(fn, dropout_p)) return st;
  const dadgpt::Dropout drop{dropout_p, seed};
  return from_hip(dadgpt::launch_bwd_bf16(B(dq), B(dk), B(dv), delta, B(dout), B(out), lse,
                                          B(q), B(k), B(v), BH, S, d_head, scale,
                                          dadgpt::contiguous_layout(S, d_head),
                                          as_stream(stream), dadgpt::kBwdAll, &drop),
                  fn);
}

int dadgpt_flash_attention_forward_dropout(float* out, float* lse, const float* q,
                                           const float* k, const float* v, int BH, int S,
                                           int d_head, float scale, float dropout_p,
                                           uint64_t seed, void* stream) {
  const char* fn = "dadgpt_flash_attention_forward_dropout";
  if (int st = check_attn(fn, BH, S, d_head, scale, {out, lse, q, k, v})) return st;
  if (int st = check_dropout(fn, dropout_p)) return st;
  const dadgpt::Dropout drop{dropout_p, seed};
  return from_hip(dadgpt::launch_fwd_f32(out, lse, q, k, v, BH, S, d_head, scale,
                                         as_stream(stream), &drop),
                  fn);
}

int dadgpt_flash_attention_backward_dropout(float* dq, float* dk, float* dv, float* delta,
                                            const float* dout, const float* out,
                                            const float* lse, const float* q, const float* k,
                                            const float* v, int BH, int S, int d_head,
                                            float scale, float dropout_p, uint64_t seed,
                                            void* stream) {
  const char* fn = "dadgpt_flash_attention_backward_dropout";
  if (int st = check_attn(fn, BH, S, d_head, scale, {dq, dk, dv, delta, dout, out, lse, q, k, v}))
    return st;
  if (int st = check_dropout(fn, dropout_p)) return st;
  const dadgpt::Dropout drop{dropout_p, seed};
  return from_hip(dadgpt::launch_bwd_f32(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S,
                                         d_head, scale, as_stream(stream), &drop),
                  fn);
}

int dadgpt_flash_attention_backward_bf16_phase(int phase, uint16_t* dq, uint16_t* dk,
                                               uint16_t* dv, float* delta, const uint16_t* dout,
                                               const uint16_t* out, const float* lse,
                                               const uint16_t* q, const uint16_t* k,
                                               const uint16_t* v, int BH, int S, int d_head,
                                               float scale, void* stream) {
  const char* fn = "dadgpt_flash_attention_backward_bf16_phase";
  if (phase < 0 || phase > 2)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: phase %d not in {0,1,2}", fn, phase);
  if (int st = check_attn(fn, BH, S, d_head, scale, {dq, dk, dv, delta, dout, out, lse, q, k, v}))
    return st;
  return from_hip(dadgpt::launch_bwd_bf16(B(dq), B(dk), B(dv), delta, B(dout), B(out), lse,
                                          B(q), B(k), B(v), BH, S, d_head, scale,
                                          dadgpt::contiguous_layout(S, d_head),
                                          as_stream(stream), 1 << phase),
                  fn);
}

int dadgpt_flash_attention_forward_bf16_strided(uint16_t* out, float* lse, const uint16_t* q,
                                                const uint16_t* k, const uint16_t* v, int batch,
                                                int H, int S, int d_head, float scale,
                                                const dadgpt_head_strides* strides,
                                                void* stream) {
  const char* fn = "dadgpt_flash_attention_forward_bf16_strided";
  dadgpt::AttnLayout L;
  if (int st = check_strides(fn, batch, H, S, d_head, strides, 4, &L)) return st;
  if (int st = check_attn(fn, batch * H, S, d_head, scale, {out, lse, q, k, v})) return st;
  return from_hip(dadgpt::launch_fwd_bf16(B(out), lse, B(q), B(k), B(v), batch * H, S, d_head,
                                          scale, L, as_stream(stream)),
                  fn);
}

int dadgpt_flash_attention_backward_bf16_strided(uint16_t* dq, uint16_t* dk, uint16_t* dv,
                                                 float* delta, const uint16_t* dout,
                                                 const uint16_t* out, const float* lse,
                                                 const uint16_t* q, const uint16_t* k,
                                                 const uint16_t* v, int batch, int H, int S,
                                                 int d_head, float scale,
                                                 const dadgpt_head_strides* strides,
                                                 void* stream) {
  const char* fn = "dadgpt_flash_attention_backward_bf16_strided";
  dadgpt::AttnLayout L;
  if (int st = check_strides(fn, batch, H, S, d_head, strides, 8, &L)) return st;
  if (int st = check_attn(fn, batch * H, S, d_head, scale,
                          {dq, dk, dv, delta, dout, out, lse, q, k, v}))
    return st;
  return from_hip(dadgpt::launch_bwd_bf16(B(dq), B(dk), B(dv), delta, B(dout), B(out), lse,
                                          B(q), B(k), B(v), batch * H, S, d_head, scale, L,
                                          as_stream(stream)),
                  fn);
}

int dadgpt_flash_attention_forward_bf16_tokens(uint16_t* out, int64_t ld_out, float* lse,
                                               const uint16_t* q, const uint16_t* k,
                                               const uint16_t* v, int64_t ld_qkv, int batch,
                                               int H, int S, int d_head, float scale,
                                               void* stream) {
  const char* fn = "dadgpt_flash_attention_forward_bf16_tokens";
  if (int st = check_ld(fn, H, d_head, {ld_qkv, ld_out})) return st;
  const dadgpt_head_strides in = tokens(ld_qkv, S, d_head), o = tokens(ld_out, S, d_head);
  const dadgpt_head_strides st[4] = {in, in, in, o};
  return dadgpt_flash_attention_forward_bf16_strided(out, lse, q, k, v, batch, H, S, d_head,
                                                     scale, st, stream);
}

int dadgpt_flash_attention_backward_bf16_tokens(uint16_t* dq, uint16_t* dk, uint16_t* dv,
                                                int64_t ld_dqkv, float* delta,
                                                const uint16_t* dout, const uint16_t* out,
                                                int64_t ld_out, const float* lse,
                                                const uint16_t* q, const uint16_t* k,
                                                const uint16_t* v, int64_t ld_qkv, int batch,
                                                int H, int S, int d_head, float scale,
                                                void* stream) {
  const char* fn = "dadgpt_flash_attention_backward_bf16_tokens";
  if (int st = check_ld(fn, H, d_head, {ld_qkv, ld_out, ld_dqkv})) return st;
  const dadgpt_head_strides in = tokens(ld_qkv, S, d_head), o = tokens(ld_out, S, d_head),
                            g = tokens(ld_dqkv, S, d_head);
  const dadgpt_head_strides st[8] = {in, in, in, o, o, g, g, g};
  return dadgpt_flash_attention_backward_bf16_strided(dq, dk, dv, delta, dout, out, lse, q, k, v,
                                                      batch, H, S, d_head, scale, st, stream);
}

size_t dadgpt_decode_workspace_bytes(int n_seq, int n_heads, int max_len, int d_head) {
  if (n_seq < 1 || n_heads < 1 || max_len < 1 || !supported(d_head)) return 0;
  return dadgpt::decode_workspace_bytes(n_seq, n_heads, max_len, d_head);
}

int dadgpt_decode_attention_bf16(uint16_t* out, const uint16_t* q, const uint16_t* k_cache,
                                 const uint16_t* v_cache, const int32_t* lens, int n_seq,
                                 int n_heads, int max_len, int d_head, float scale,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "dadgpt_decode_attention_bf16";
  if (int st = check_decode(fn, n_seq, n_heads, max_len, d_head, scale, workspace,
                            workspace_bytes, {out, q, k_cache, v_cache, lens}))
    return st;
  return from_hip(dadgpt::launch_decode_bf16(B(out), B(q), B(k_cache), B(v_cache), lens, n_seq,
                                             n_heads, max_len, d_head, scale, workspace,
                                             workspace_bytes, as_stream(stream)),
                  fn);
}

int dadgpt_decode_attention_bf16_noalloc(uint16_t* out, const uint16_t* q,
                                         const uint16_t* k_cache, const uint16_t* v_cache,
                                         const int32_t* lens, int n_seq, int n_heads,
                                         int max_len, int d_head, float scale, void* stream) {
  const char* fn = "dadgpt_decode_attention_bf16_noalloc";
  if (int st = check_decode_shape(fn, n_seq, n_heads, max_len, d_head, scale,
                                  {out, q, k_cache, v_cache, lens}))
    return st;
  const size_t need = dadgpt::decode_workspace_bytes(n_seq, n_heads, max_len, d_head);
  if (need > dadgpt::kDecodeScratchBytes)
    return fail(DADGPT_ERR_WORKSPACE,
                "%s: this shape needs %zu bytes of scratch, above the fixed %zu", fn, need,
                dadgpt::kDecodeScratchBytes);
  void* scratch = nullptr;
  if (hipError_t e = dadgpt::decode_scratch(&scratch, as_stream(stream)); e != hipSuccess)
    return from_hip(e, fn);
  return from_hip(dadgpt::launch_decode_bf16(B(out), B(q), B(k_cache), B(v_cache), lens, n_seq,
                                             n_heads, max_len, d_head, scale, scratch,
                                             dadgpt::kDecodeScratchBytes, as_stream(stream)),
                  fn);
}

// ---- materialized attention path ----

int dadgpt_softmax(float* out, const float* in, int rows, int cols, void* stream) {
  const char* fn = "dadgpt_softmax";
  if (int st = check_rows(fn, rows, cols, {out, in})) return st;
  return from_hip(dadgpt::launch_softmax_rows(out, in, rows, cols, as_stream(stream)), fn);
}

int dadgpt_softmax_backward(float* din, const float* dout, const float* out, int rows, int cols,
                            void* stream) {
  const char* fn = "dadgpt_softmax_backward";
  if (int st = check_rows(fn, rows, cols, {din, dout, out})) return st;
  return from_hip(
      dadgpt::launch_softmax_backward_rows(din, dout, out, rows, cols, as_stream(stream)), fn);
}

int dadgpt_causal_mask(float* scores, int n_blocks, int S, void* stream) {
  const char* fn = "dadgpt_causal_mask";
  if (int st = check_blocks(fn, n_blocks, S, scores)) return st;
  return from_hip(dadgpt::launch_causal_fill(scores, n_blocks, S, -1e9f, as_stream(stream)), fn);
}

int dadgpt_causal_mask_zero(float* grads, int n_blocks, int S, void* stream) {
  const char* fn = "dadgpt_causal_mask_zero";
  if (int st = check_blocks(fn, n_blocks, S, grads)) return st;
  return from_hip(dadgpt::launch_causal_fill(grads, n_blocks, S, 0.0f, as_stream(stream)), fn);
}

int dadgpt_split_heads(float* out, const float* in, int batch_size, int seq_len, int n_heads,
                       int d_head, void* stream) {
  const char* fn = "dadgpt_split_heads";
  if (int st = check_heads(fn, out, in, batch_size, seq_len, n_heads, d_head)) return st;
  return from_hip(dadgpt::launch_split_heads(out, in, batch_size, seq_len, n_heads, d_head,
                                             as_stream(stream)),
                  fn);
}

int dadgpt_merge_heads(float* out, const float* in, int batch_size, int seq_len, int n_heads,
                       int d_head, void* stream) {
  const char* fn = "dadgpt_merge_heads";
  if (int st = check_heads(fn, out, in, batch_size, seq_len, n_heads, d_head)) return st;
  return from_hip(dadgpt::launch_merge_heads(out, in, batch_size, seq_len, n_heads, d_head,
                                             as_stream(stream)),
                  fn);
}

int dadgpt_scale(float* data, int64_t count, float scale, void* stream) {
  const char* fn = "dadgpt_scale";
  if (data == nullptr) return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: data is null", fn);
  if (count < 0) return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: count %lld < 0", fn,
                             (long long)count);
  if (count == 0) return ok();
  return from_hip(dadgpt::launch_scale(data, count, scale, as_stream(stream)), fn);
}

int dadgpt_attention_probs(float* probs, int BH, int S, float scale, void* stream) {
  const char* fn = "dadgpt_attention_probs";
  if (int st = check_blocks(fn, BH, S, probs)) return st;
  if (!std::isfinite(scale))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: scale must be finite", fn);
  return from_hip(dadgpt::launch_attention_probs(probs, BH, S, scale, as_stream(stream)), fn);
}

int dadgpt_attention_probs_backward(float* dscores, const float* dprobs, const float* probs,
                                    int BH, int S, float scale, void* stream) {
  const char* fn = "dadgpt_attention_probs_backward";
  if (int st = check_blocks(fn, BH, S, dscores)) return st;
  if (int st = check_blocks(fn, BH, S, dprobs)) return st;
  if (int st = check_blocks(fn, BH, S, probs)) return st;
  if (!std::isfinite(scale))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: scale must be finite", fn);
  return from_hip(dadgpt::launch_attention_probs_backward(dscores, dprobs, probs, BH, S, scale,
                                                          as_stream(stream)),
                  fn);
}

int dadgpt_attention_dropout(float* dropped, const float* probs, int BH, int S, float dropout_p,
                             uint64_t seed, void* stream) {
  const char* fn = "dadgpt_attention_dropout";
  if (int st = check_blocks(fn, BH, S, dropped)) return st;
  if (int st = check_blocks(fn, BH, S, probs)) return st;
  if (int st = check_dropout(fn, dropout_p)) return st;
  const dadgpt::Dropout drop{dropout_p, seed};
  return from_hip(dadgpt::launch_attention_dropout(dropped, probs, BH, S, drop, as_stream(stream)),
                  fn);
}

int dadgpt_attention_probs_backward_dropout(float* dscores, const float* dprobs,
                                            const float* probs, int BH, int S, float scale,
                                            float dropout_p, uint64_t seed, void* stream) {
  const char* fn = "dadgpt_attention_probs_backward_dropout";
  if (int st = check_blocks(fn, BH, S, dscores)) return st;
  if (int st = check_blocks(fn, BH, S, dprobs)) return st;
  if (int st = check_blocks(fn, BH, S, probs)) return st;
  if (!std::isfinite(scale))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: scale must be finite", fn);
  if (int st = check_dropout(fn, dropout_p)) return st;
  const dadgpt::Dropout drop{dropout_p, seed};
  return from_hip(dadgpt::launch_attention_probs_backward_dropout(dscores, dprobs, probs, BH, S,
                                                                  scale, drop,
                                                                  as_stream(stream)),
                  fn);
}

int dadgpt_decode_probs(float* probs, const int32_t* lens, int n_seq, int n_heads, int max_len,
                        float scale, void* stream) {
  const char* fn = "dadgpt_decode_probs";
  if (probs == nullptr || lens == nullptr)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: null pointer argument", fn);
  if (n_seq < 1 || n_heads < 1 || max_len < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT,
                "%s: n_seq=%d, n_heads=%d, max_len=%d must be positive", fn, n_seq, n_heads,
                max_len);
  if (int st = check_rows(fn, (long long)n_seq * n_heads, max_len, {probs})) return st;
  if (!std::isfinite(scale))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: scale must be finite", fn);
  return from_hip(dadgpt::launch_decode_probs(probs, lens, n_seq, n_heads, max_len, scale,
                                              as_stream(stream)),
                  fn);
}

int dadgpt_use_fused_attention(int impl, int d_head, int ctx_len, int attn_dropout) {
  // src/model.cpp:185-197: dropout or an unsupported head size forces the materialized path;
  // otherwise the selected implementation, and Auto picks fused from a context of 512 up.
  if (attn_dropout || !supported(d_head)) return 0;
  if (impl == DADGPT_ATTENTION_FUSED) return 1;
  if (impl == DADGPT_ATTENTION_MATERIALIZED) return 0;
  return ctx_len >= 512 ? 1 : 0;
}

int dadgpt_decode_attention_f32(float* out, const float* q, const float* k_cache,
                                const float* v_cache, const int32_t* lens, int n_seq,
                                int n_heads, int max_len, int d_head, float scale,
                                void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "dadgpt_decode_attention_f32";
  if (int st = check_decode(fn, n_seq, n_heads, max_len, d_head, scale, workspace,
                            workspace_bytes, {out, q, k_cache, v_cache, lens}))
    return st;
  return from_hip(dadgpt::launch_decode_f32(out, q, k_cache, v_cache, lens, n_seq, n_heads,
                                            max_len, d_head, scale, workspace, workspace_bytes,
                                            as_stream(stream)),
                  fn);
}

}  // extern "C"
