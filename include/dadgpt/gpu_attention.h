/*
 * libdadgpt_attn.so — C ABI of the MI355X (gfx950) fused causal attention path.
 *
 * Drop-in for the attention launch wrappers of the reference (Jimdrews/DadGPT,
 * cuda/gpu_ops.cuh:112-122, defined in cuda/attention.cu:232-252) plus the KV-cache decode
 * that the reference composes inline in src/model.cpp:758-790. The C++-linkage functions
 * with the reference's exact names and signatures are declared in
 * <dadgpt/gpu_ops_attention.hpp> and defined in the same library.
 *
 * Conventions (shared by every entry point):
 *  - All tensor pointers are device pointers owned by the caller, 16-byte aligned (checked);
 *    the library allocates nothing in these calls. Layout [BH, S, d_head] contiguous, heads
 *    already split (cuda/attention.cu:6), except for the _strided and _tokens calls; lse
 *    and delta are [BH, S] fp32; lse is the natural-log logsumexp of the scaled scores
 *    (cuda/attention.cu:71).
 *  - bf16 tensors are passed as uint16_t* holding IEEE bfloat16 bit patterns.
 *  - Outputs are overwritten, never accumulated (cuda/gpu_ops.cuh:118).
 *  - Arguments are validated on the host before any HIP call; a failing call returns a
 *    nonzero dadgpt_status and dadgpt_last_error() describes it (thread-local). Launch errors
 *    (hipGetLastError) map to DADGPT_ERR_HIP; asynchronous faults surface at the caller's
 *    next synchronisation, as in the reference (cuda/gpu_ops.cuh:10-17).
 *  - Functions without a stream argument launch on the null (legacy default) stream, as the
 *    reference does (cuda/attention.cu:211,220-226). `stream` arguments take a hipStream_t;
 *    NULL means the null stream.
 */
#ifndef DADGPT_GPU_ATTENTION_H
#define DADGPT_GPU_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum dadgpt_status {
  DADGPT_OK = 0,
  DADGPT_ERR_INVALID_ARGUMENT = 1, /* null pointer, non-positive size, bad scale */
  DADGPT_ERR_UNSUPPORTED = 2,      /* d_head outside the supported set */
  DADGPT_ERR_HIP = 3,              /* a HIP launch reported an error */
  DADGPT_ERR_WORKSPACE = 4         /* decode workspace missing or too small */
} dadgpt_status;

/* Message of the last failing call on this thread ("" if none). */
const char* dadgpt_last_error(void);
/* Static name of a status code. */
const char* dadgpt_status_string(int status);
/* Library version string. */
const char* dadgpt_version(void);

/* Replaces bool gpu_flash_attention_supported(int d_head) — cuda/gpu_ops.cuh:115,
 * cuda/attention.cu:232. Returns 1 for d_head in {32, 64}, else 0. */
int dadgpt_flash_attention_supported(int d_head);

/* Replaces gpu_flash_attention_forward — cuda/gpu_ops.cuh:116-117, cuda/attention.cu:234-239.
 * fp32 q,k,v -> out [BH,S,d_head], lse [BH,S]. Null stream. */
int dadgpt_flash_attention_forward(float* out, float* lse, const float* q, const float* k,
                                   const float* v, int BH, int S, int d_head, float scale);

/* Replaces gpu_flash_attention_backward — cuda/gpu_ops.cuh:119-122,
 * cuda/attention.cu:241-252. Writes dq, dk, dv; delta [BH,S] is caller scratch
 * (src/model.cpp:250). Null stream. */
int dadgpt_flash_attention_backward(float* dq, float* dk, float* dv, float* delta,
                                    const float* dout, const float* out, const float* lse,
                                    const float* q, const float* k, const float* v, int BH,
                                    int S, int d_head, float scale);

/* Stream-ordered variants of the two fp32 calls above (no reference counterpart: the
 * reference has no stream argument). */
int dadgpt_flash_attention_forward_async(float* out, float* lse, const float* q,
                                         const float* k, const float* v, int BH, int S,
                                         int d_head, float scale, void* stream);
int dadgpt_flash_attention_backward_async(float* dq, float* dk, float* dv, float* delta,
                                          const float* dout, const float* out,
                                          const float* lse, const float* q, const float* k,
                                          const float* v, int BH, int S, int d_head,
                                          float scale, void* stream);

/* bf16 sibling of gpu_flash_attention_forward (no reference counterpart: the reference's
 * attention is fp32-only, cuda/attention.cu:1). bf16 q,k,v,out; fp32 lse. MFMA, fp32
 * accumulation. */
int dadgpt_flash_attention_forward_bf16(uint16_t* out, float* lse, const uint16_t* q,
                                        const uint16_t* k, const uint16_t* v, int BH, int S,
                                        int d_head, float scale, void* stream);

/* bf16 sibling of gpu_flash_attention_backward (no reference counterpart). bf16
 * dout/out/q/k/v in, bf16 dq/dk/dv out (overwritten); fp32 lse in; delta [BH,S] fp32
 * scratch, written. */
int dadgpt_flash_attention_backward_bf16(uint16_t* dq, uint16_t* dk, uint16_t* dv,
                                         float* delta, const uint16_t* dout,
                                         const uint16_t* out, const float* lse,
                                         const uint16_t* q, const uint16_t* k,
                                         const uint16_t* v, int BH, int S, int d_head,
                                         float scale, void* stream);

/* ---- Attention-probability dropout (replaces the reference's materialized path with
 * dropout: gpu_dropout_forward on P before P V, src/model.cpp:406-416, and
 * gpu_dropout_backward on dP, :594-599; kernels cuda/gpu_ops.cu:712-749). Fused into the
 * flash kernels: the keep bits are regenerated in the backward, no mask is stored. Kept
 * probabilities are scaled by 1/(1-p) (fp32), as the reference does; lse stays that of the
 * undropped scores. The mask is not cuRAND's: probability (row = bh*S + i, key j) is kept
 * iff u >= ceil(p * 2^16), u = 16-bit half j%2 (low first) of word (j%8)/2 of Philox4x32-10
 * (Salmon et al., SC'11) at counter {row lo, row hi, j/8, 0} under key {seed lo, seed hi}.
 * The backward must get the
 * forward's (dropout_p, seed). dropout_p in [0, 1); contiguous [BH, S, d_head] layout. */
int dadgpt_flash_attention_forward_bf16_dropout(uint16_t* out, float* lse, const uint16_t* q,
                                                const uint16_t* k, const uint16_t* v, int BH,
                                                int S, int d_head, float scale,
                                                float dropout_p, uint64_t seed, void* stream);
int dadgpt_flash_attention_backward_bf16_dropout(uint16_t* dq, uint16_t* dk, uint16_t* dv,
                                                 float* delta, const uint16_t* dout,
                                                 const uint16_t* out, const float* lse,
                                                 const uint16_t* q, const uint16_t* k,
                                                 const uint16_t* v, int BH, int S, int d_head,
                                                 float scale, float dropout_p, uint64_t seed,
                                                 void* stream);

/* fp32 siblings (the reference's own precision; the reference's dropout path is fp32). */
int dadgpt_flash_attention_forward_dropout(float* out, float* lse, const float* q,
                                           const float* k, const float* v, int BH, int S,
                                           int d_head, float scale, float dropout_p,
                                           uint64_t seed, void* stream);
int dadgpt_flash_attention_backward_dropout(float* dq, float* dk, float* dv, float* delta,
                                            const float* dout, const float* out,
                                            const float* lse, const float* q, const float* k,
                                            const float* v, int BH, int S, int d_head,
                                            float scale, float dropout_p, uint64_t seed,
                                            void* stream);

/* One kernel of dadgpt_flash_attention_backward_bf16, for per-kernel timing and profiling
 * (no reference counterpart). phase 1: dq, and delta = rowsum(dout * out) of the same rows;
 * 2: dk, dv (reads delta). Running phases 1, 2 in order equals the full backward. phase 0
 * computes delta alone in a separate pass (equal to phase 1's up to fp32 summation order). */
int dadgpt_flash_attention_backward_bf16_phase(int phase, uint16_t* dq, uint16_t* dk,
                                               uint16_t* dv, float* delta,
                                               const uint16_t* dout, const uint16_t* out,
                                               const float* lse, const uint16_t* q,
                                               const uint16_t* k, const uint16_t* v, int BH,
                                               int S, int d_head, float scale, void* stream);

/* ---- Attention over strided layouts (no reference counterpart). The reference splits the
 * projections' token-major [B*S, H*d_head] rows into [B*H, S, d_head] before the fused kernel
 * and merges the outputs and gradients back (gpu_split_heads / gpu_merge_heads,
 * cuda/gpu_ops.cu:426-474, called at src/model.cpp:384-387,423-424 in the forward and
 * :564-565,619-624 in the backward). These entry points read and write the tensors where they
 * lie, so those six permutation passes disappear. Same arithmetic, lse/delta layout
 * ([B*H, S] fp32, natural log) and overwrite semantics as the contiguous bf16 calls. */

/* Placement of one bf16 tensor viewed as [B, H, S, d_head]: row s of head h of batch b
 * starts at element b*batch + h*head + s*row of its pointer; the d_head elements of a row are
 * contiguous. Every stride is in elements, non-negative and a multiple of 8 (16 bytes);
 * row >= d_head and row <= 2^24. Contiguous [B*H, S, d_head] is {H*S*d_head, S*d_head,
 * d_head}; token-major [B*S, H*d_head] is {S*H*d_head, d_head, H*d_head}. */
typedef struct dadgpt_head_strides {
  int64_t batch, head, row;
} dadgpt_head_strides;

/* Index of each tensor in the strides arrays below. */
enum {
  DADGPT_T_Q = 0, DADGPT_T_K, DADGPT_T_V, DADGPT_T_OUT, /* forward: strides[4] */
  DADGPT_T_DOUT, DADGPT_T_DQ, DADGPT_T_DK, DADGPT_T_DV  /* backward: strides[8] */
};

/* Forward with q, k, v, out placed by strides[DADGPT_T_Q .. DADGPT_T_OUT]; lse [B*H, S].
 * Outputs must not overlap each other or the inputs. */
int dadgpt_flash_attention_forward_bf16_strided(uint16_t* out, float* lse, const uint16_t* q,
                                                const uint16_t* k, const uint16_t* v, int B,
                                                int H, int S, int d_head, float scale,
                                                const dadgpt_head_strides* strides,
                                                void* stream);

/* Backward with every tensor placed by strides[0 .. 7] (order above); delta [B*H, S] fp32
 * scratch, written. dq, dk, dv may share one buffer (e.g. the gradient of a fused QKV
 * projection output) as long as their rows do not overlap. */
int dadgpt_flash_attention_backward_bf16_strided(uint16_t* dq, uint16_t* dk, uint16_t* dv,
                                                 float* delta, const uint16_t* dout,
                                                 const uint16_t* out, const float* lse,
                                                 const uint16_t* q, const uint16_t* k,
                                                 const uint16_t* v, int B, int H, int S,
                                                 int d_head, float scale,
                                                 const dadgpt_head_strides* strides,
                                                 void* stream);

/* Token-major forms: row t = b*S + s of every tensor holds the H heads' d_head values side by
 * side, as the QKV projection produces them and the Wo projection consumes them. ld_qkv is
 * the row pitch (elements) of q, k and v: H*d_head for three separate [B*S, H*d_head]
 * tensors (the reference's la.q/la.k/la.v), 3*H*d_head for one fused [B*S, 3*H*d_head]
 * projection output with k = q + H*d_head and v = q + 2*H*d_head. ld_out is the pitch of out
 * and dout, ld_dqkv that of dq, dk, dv. Replace split_heads -> flash forward -> merge_heads
 * (src/model.cpp:384-392,423-424) and split_heads -> flash backward -> 3x merge_heads
 * (src/model.cpp:564-576,619-624). */
int dadgpt_flash_attention_forward_bf16_tokens(uint16_t* out, int64_t ld_out, float* lse,
                                               const uint16_t* q, const uint16_t* k,
                                               const uint16_t* v, int64_t ld_qkv, int B, int H,
                                               int S, int d_head, float scale, void* stream);
int dadgpt_flash_attention_backward_bf16_tokens(uint16_t* dq, uint16_t* dk, uint16_t* dv,
                                                int64_t ld_dqkv, float* delta,
                                                const uint16_t* dout, const uint16_t* out,
                                                int64_t ld_out, const float* lse,
                                                const uint16_t* q, const uint16_t* k,
                                                const uint16_t* v, int64_t ld_qkv, int B, int H,
                                                int S, int d_head, float scale, void* stream);

/* Bytes of decode workspace for a cache shape, valid for both element types. It is 0 when
 * max_len fits one workgroup chunk (256 keys fp32 and 512 bf16 at d_head 64; 512 and 1024 at
 * d_head 32): then no workspace is needed and NULL may be passed. Longer caches are split
 * into chunks merged inside the same kernel by the last chunk of each cache, through the
 * workspace: per-(sequence, head) arrival counters at its start, fp32 partials packed against
 * its end. Contract: size it for the largest (n_seq, n_heads, max_len, d_head) it will serve,
 * ZERO-FILL it once (hipMemset at allocation), and pass its full size as workspace_bytes on
 * every call; each call leaves the counters at zero again, so calls of any shape up to the
 * sizing one can share it. Calls that share a workspace must not overlap in time. */
size_t dadgpt_decode_workspace_bytes(int n_seq, int n_heads, int max_len, int d_head);

/* KV-cache decode attention (replaces the per-head composition in src/model.cpp:758-790:
 * q K^T, *scale, softmax over the cache length, P V; no reference signature exists).
 *  q [n_seq, n_heads, d_head]; k_cache, v_cache [n_seq, n_heads, max_len, d_head];
 *  lens: DEVICE int32 [n_seq], valid cache rows per sequence (clamped to [0, max_len];
 *  a length of 0 yields a zero output row); out [n_seq, n_heads, d_head]. */
int dadgpt_decode_attention_bf16(uint16_t* out, const uint16_t* q, const uint16_t* k_cache,
                                 const uint16_t* v_cache, const int32_t* lens, int n_seq,
                                 int n_heads, int max_len, int d_head, float scale,
                                 void* workspace, size_t workspace_bytes, void* stream);
/* Allocation-free form of dadgpt_decode_attention_bf16. It has no counterpart in the
 * reference: it is for callers that cannot allocate or pass a workspace (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc). Same arguments minus the workspace,
 * same kernels, bit-identical results. The split-cache partials and arrival counters live in
 * a fixed scratch region of DADGPT_DECODE_NOALLOC_SCRATCH_BYTES per device inside the library,
 * held until the process ends; a shape whose dadgpt_decode_workspace_bytes() exceeds it is
 * refused with DADGPT_ERR_WORKSPACE before any HIP call (for example n_seq * n_heads = 384 at
 * d_head 64 serves max_len up to about 10,000). The first call on a device looks the region
 * up and zero-fills it with a kernel on `stream`; every call leaves its counters at zero.
 * Every call on one device shares the region: calls that overlap in time on one device (two
 * streams, two threads) race and must be serialised by the caller. */
#define DADGPT_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)
int dadgpt_decode_attention_bf16_noalloc(uint16_t* out, const uint16_t* q,
                                         const uint16_t* k_cache, const uint16_t* v_cache,
                                         const int32_t* lens, int n_seq, int n_heads,
                                         int max_len, int d_head, float scale, void* stream);

int dadgpt_decode_attention_f32(float* out, const float* q, const float* k_cache,
                                const float* v_cache, const int32_t* lens, int n_seq,
                                int n_heads, int max_len, int d_head, float scale,
                                void* workspace, size_t workspace_bytes, void* stream);

/* ---- Materialized attention (the reference's second attention path, src/model.cpp:395-420
 * forward and :575-616 backward, with the [BH, S, S] probabilities in memory). Its batched
 * GEMMs are in <dadgpt/gpu_matmul.h> (libdadgpt_gen.so), which also composes the whole path
 * (dadgpt_attention_materialized_forward/backward). Here are its elementwise operators, fp32
 * row-major, each one launch on `stream`:
 *  - the reference's own, same semantics (the reference-named C++ forms are in
 *    <dadgpt/gpu_ops_attention.hpp>);
 *  - one-pass fusions of the chains the reference runs between its GEMMs. */

/* gpu_softmax (cuda/gpu_ops.cuh:57, cuda/gpu_ops.cu:147-199): row softmax, out may be in. */
int dadgpt_softmax(float* out, const float* in, int rows, int cols, void* stream);
/* gpu_softmax_backward (cuda/gpu_ops.cuh:76, cuda/gpu_ops.cu:542-569): ACCUMULATES
 * din += out * (dout - rowsum(dout * out)). */
int dadgpt_softmax_backward(float* din, const float* dout, const float* out, int rows, int cols,
                            void* stream);
/* gpu_causal_mask (cuda/gpu_ops.cuh:106, cuda/gpu_ops.cu:476-493): scores[b][i][j] = -1e9 for
 * j > i in each of n_blocks S x S blocks. */
int dadgpt_causal_mask(float* scores, int n_blocks, int S, void* stream);
/* gpu_causal_mask_zero (cuda/gpu_ops.cuh:108, cuda/gpu_ops.cu:495-511): 0 for j > i. */
int dadgpt_causal_mask_zero(float* grads, int n_blocks, int S, void* stream);
/* gpu_scale (cuda/gpu_ops.cuh:110, cuda/gpu_ops.cu:513-525): data[i] *= scale. */
int dadgpt_scale(float* data, int64_t count, float scale, void* stream);
/* gpu_split_heads (cuda/gpu_ops.cuh:99-100, cuda/gpu_ops.cu:426-446): fp32
 * in [batch_size * seq_len, n_heads * d_head] -> out [batch_size * n_heads, seq_len, d_head],
 * out[(b*H + h)*S*dh + s*dh + x] = in[(b*S + s)*H*dh + h*dh + x]. out and in must not overlap.
 * The attention entry points above read and write the token-major layout in place
 * (_strided, _tokens), so the product path needs no split pass. */
int dadgpt_split_heads(float* out, const float* in, int batch_size, int seq_len, int n_heads,
                       int d_head, void* stream);
/* gpu_merge_heads (cuda/gpu_ops.cuh:102-103, cuda/gpu_ops.cu:448-474): the inverse,
 * [batch_size * n_heads, seq_len, d_head] -> [batch_size * seq_len, n_heads * d_head]. */
int dadgpt_merge_heads(float* out, const float* in, int batch_size, int seq_len, int n_heads,
                       int d_head, void* stream);

/* scores [BH, S, S] -> probabilities in place: x scale, -1e9 above the diagonal, row softmax
 * (gpu_scale + gpu_causal_mask + gpu_softmax, src/model.cpp:407-409, in one pass). */
int dadgpt_attention_probs(float* probs, int BH, int S, float scale, void* stream);
/* d(scores) [BH, S, S] from d(probs) and probs: softmax backward, 0 above the diagonal,
 * x scale (gpu_zero + gpu_softmax_backward + gpu_causal_mask_zero + gpu_scale,
 * src/model.cpp:601-607, in one pass). dscores may be dprobs. */
int dadgpt_attention_probs_backward(float* dscores, const float* dprobs, const float* probs,
                                    int BH, int S, float scale, void* stream);
/* Attention-probability dropout of the materialized path (src/model.cpp:406-416; the
 * reference's gpu_dropout_forward, cuda/gpu_ops.cu:712-733): dropped [BH, S, S] =
 * probs * keep / (1 - dropout_p), with the keep mask of the flash _dropout entry points
 * (probability (bh, i, j) is row bh*S + i, key j of that mask; no mask is stored).
 * dropped may be probs. dropout_p in [0, 1). */
int dadgpt_attention_dropout(float* dropped, const float* probs, int BH, int S, float dropout_p,
                             uint64_t seed, void* stream);
/* dadgpt_attention_probs_backward with dropout (src/model.cpp:594-607): d(dropped probs) is
 * first multiplied by keep / (1 - dropout_p) (gpu_dropout_backward, cuda/gpu_ops.cu:736-749),
 * then taken through the softmax backward against the undropped probs. */
int dadgpt_attention_probs_backward_dropout(float* dscores, const float* dprobs,
                                            const float* probs, int BH, int S, float scale,
                                            float dropout_p, uint64_t seed, void* stream);
/* Decode scores [n_seq * n_heads, max_len] -> probabilities in place over each sequence's
 * first lens[seq] keys (DEVICE int32 lens; x scale, keys at or past the length -1e9, row
 * softmax; an empty cache gives a zero row): the gpu_scale + gpu_softmax step of the
 * reference's decode (src/model.cpp:776-780) for a batch of ragged caches. */
int dadgpt_decode_probs(float* probs, const int32_t* lens, int n_seq, int n_heads, int max_len,
                        float scale, void* stream);

/* The reference's choice between the two paths (AttentionImpl, src/model.hpp:80;
 * use_fused_attention, src/model.cpp:183-197): 1 = fused flash kernels, 0 = materialized.
 * Attention dropout or an unsupported d_head forces materialized; Fused and Materialized
 * force their path; Auto takes fused from ctx_len 512 up. The reference takes the
 * materialized path for dropout because its fused kernel has none; here the flash kernels
 * carry dropout too (the _dropout entry points), so a caller may keep them, but this predicate
 * answers exactly as the reference's does. */
typedef enum dadgpt_attention_impl {
  DADGPT_ATTENTION_AUTO = 0,
  DADGPT_ATTENTION_FUSED = 1,
  DADGPT_ATTENTION_MATERIALIZED = 2
} dadgpt_attention_impl;
int dadgpt_use_fused_attention(int impl, int d_head, int ctx_len, int attn_dropout);

#ifdef __cplusplus
}
#endif

#endif /* DADGPT_GPU_ATTENTION_H */
