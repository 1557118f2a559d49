/*
 * libdadgpt_gen.so — batched GPT-2 generation on the MI355X attention path.
 *
 * Replaces, for a batch of ragged prompts, the reference's generation stack:
 *   generate_tokens / sample_token (greedy)   src/generate.cpp:16-37, 94-139
 *   model_prefill                             src/model.cpp:827-851
 *   model_forward_cached                      src/model.cpp:687-825
 *   KVCache, kv_cache_alloc                   src/model.hpp:140-152, src/model.cpp:659-685
 * The reference decodes one sequence at a time with 2*H cache memcpys and 2*H cuBLAS GEMVs per
 * layer and token. Here the prompts of a batch prefill together (one flash-attention launch per
 * layer over the padded batch, the KV append fused into the QKV split), and every decode step
 * runs one ragged decode-attention launch per layer for the whole batch. Prefill projections
 * are bf16 hipBLASLt GEMMs (<dadgpt/gpu_matmul.h>); decode projections for batches of up to 16
 * run on skinny MFMA kernels over pre-transposed weights with the residual add + LayerNorm
 * and bias + GELU fused into their prologues. The residual stream, LayerNorm statistics and
 * logits are fp32. Attention runs in bf16 (default), in fp32 on the fused kernels, or in fp32
 * on the materialized path (attn_mode below) with everything else identical.
 *
 * Status codes are those of <dadgpt/gpu_attention.h>; dadgpt_gen_last_error() describes the
 * last failure on the calling thread.
 */
#ifndef DADGPT_GPT2_GENERATE_H
#define DADGPT_GPT2_GENERATE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The reference's ModelConfig (src/model.hpp:10-20) without batch_size.
 * GPT-2 124M: d_model 768, n_layers 12, n_heads 12, d_ff 3072, ctx_len 1024, vocab 50257. */
typedef struct dadgpt_gpt2_config {
  int d_model, n_layers, n_heads, d_ff, ctx_len, vocab_size;
} dadgpt_gpt2_config;

typedef struct dadgpt_gpt2 dadgpt_gpt2;

typedef struct dadgpt_gpt2_timing {
  float prefill_ms;      /* the batched prefill, through the first greedy pick */
  float decode_ms;       /* all decode steps */
  float decode_attn_ms;  /* the decode-attention launches inside those steps (measured with
                            graphs off only: -1 with graphs on) */
  int decode_steps;
} dadgpt_gpt2_timing;

/* Parameter count (bf16 elements) of the reference's parameter arena, in its order
 * (src/model.cpp:17-56): tok_emb [V,d], pos_emb [ctx,d], then per layer ln1_w, ln1_b,
 * Wq [d,d], bq, Wk, bk, Wv, bv, Wo, bo, ln2_w, ln2_b, fc1_w [d,d_ff], fc1_b, fc2_w [d_ff,d],
 * fc2_b; then lnf_w, lnf_b. Weights are row-major [in, out]. 0 for an invalid config. */
size_t dadgpt_gpt2_param_count(const dadgpt_gpt2_config* config);

/* The reference's initialisation (src/model.cpp:121-166) into a device arena of
 * dadgpt_gpt2_param_count elements: weights N(0, 0.02); Wo and fc2_w N(0, 0.02/sqrt(2L));
 * biases 0; LayerNorm weights 1. The normals come from a counter-based splitmix64 +
 * Box-Muller stream of `seed` (one sub-stream per tensor), rounded to bf16. */
int dadgpt_gpt2_init_params(uint16_t* params, const dadgpt_gpt2_config* config, uint64_t seed,
                            void* stream);

/* Attention of a model (everything else is the same in every mode):
 *  BF16: the bf16 flash prefill and bf16 decode kernels over bf16 KV caches (the default);
 *  FP32: the fp32 flash prefill (the reference's fused path, use_fused_attention true,
 *        src/model.cpp:390-393) and the fp32 decode kernel over fp32 caches;
 *  FP32_MATERIALIZED: the reference's materialized path (src/model.cpp:395-420; decode as
 *        src/model.cpp:765-790: q K^T, x scale, softmax over the cache length, P V) on fp32
 *        hipBLASLt GEMMs, over fp32 caches. The GPU's own fp32 reference for the others. */
enum {
  DADGPT_GPT2_ATTN_BF16 = 0,
  DADGPT_GPT2_ATTN_FP32 = 1,
  DADGPT_GPT2_ATTN_FP32_MATERIALIZED = 2
};
/* OR-ed into attn_mode with either fp32 attention: the projections run in fp32 too (fp32
 * LayerNorm/GELU/attention outputs feed fp32 hipBLASLt GEMMs over fp32 widenings of the
 * weights), i.e. the reference's default precision end to end (MatmulPrecision::FP32,
 * cuda/gpu_ops.cu:61). The decode step then uses the same GEMMs instead of the skinny bf16
 * kernels. */
#define DADGPT_GPT2_FP32_PROJECTIONS 0x100

/* A model over a caller-owned device parameter arena (kept by pointer: it must outlive the
 * model). Allocates the fused QKV weights, transposed copies of the projection weights, the
 * KV caches [max_batch, H, ctx_len, d_head] per layer, activations for max_batch x ctx_len
 * rows, a hipBLASLt handle, and in FP32_MATERIALIZED mode a [max_batch * H, ctx, ctx] fp32
 * probability buffer. d_head must be 32 or 64. attn_mode is one of the values above. */
int dadgpt_gpt2_create(const dadgpt_gpt2_config* config, const uint16_t* params, int max_batch,
                       int attn_mode, dadgpt_gpt2** out);  /* attn_mode: see above */
void dadgpt_gpt2_destroy(dadgpt_gpt2* model);

/* Decode steps after the first replay one captured HIP graph per batch size (default on);
 * off, every step is launched kernel by kernel (and timing brackets each attention launch).
 * The replayed step reads all per-step state (tokens, positions, cache lengths) from device
 * memory, so it is the same work as the eager step. Only steps made of this library's own
 * kernels are captured: up to 16 sequences on the skinny projections, with flash decode
 * attention. Steps that call hipBLASLt (more batch rows, other shapes, fp32 projections,
 * materialized attention) always run eagerly, since the library may record memory-set nodes
 * into a capture that are not safe to replay. */
int dadgpt_gpt2_set_graphs(dadgpt_gpt2* model, int enable);

/* Greedy generation for n <= max_batch prompts (host arrays):
 *   prompts [n, prompt_stride] int32 token ids, row b holding prompt_lens[b] >= 1 tokens;
 *   every prompt_lens[b] + new_tokens <= ctx_len (the reference stops at the context, and
 *   truncating a long prompt, src/generate.cpp:100-110, is the caller's choice).
 * Outputs (host): tokens [n, new_tokens]; margins [n, new_tokens] or NULL (top-1 minus
 * top-2 logit of each pick); logits [new_tokens, n, vocab] or NULL (every step's logits: for
 * tests, it synchronises per step); timing or NULL.
 * Token t of row b is the first maximum of the logits after the prompt and tokens 0..t-1
 * (std::max_element, src/generate.cpp:34-37). No stop token: exactly new_tokens per row (for
 * the reference's stop token and prompt truncation, dadgpt_gpt2_generate_tokens below). */
int dadgpt_gpt2_generate(dadgpt_gpt2* model, const int32_t* prompts, const int32_t* prompt_lens,
                         int n, int prompt_stride, int new_tokens, int32_t* tokens,
                         float* margins, float* logits, dadgpt_gpt2_timing* timing);

/* The prompt truncation of generate_tokens (src/generate.cpp:97-110), on the host: with
 * eff = min(max_len, ctx_len), a prompt of len >= eff tokens (len > 1) becomes its first token
 * followed by its last max(eff - 2, 0) tokens; any other prompt is copied unchanged. Writes
 * out (room for len tokens) and *out_len (>= 1); DADGPT_ERR_INVALID_ARGUMENT for null
 * buffers, len < 1 or ctx_len < 1. */
int dadgpt_gpt2_truncate_prompt(const int32_t* prompt, int len, int max_len, int ctx_len,
                                int32_t* out, int32_t* out_len);

/* generate_tokens (src/generate.cpp:94-139) with greedy sampling, for n <= max_batch prompts at
 * once. Per row, as the reference does for its one sequence:
 *   - max_len is capped at ctx_len, and the prompt is truncated as
 *     dadgpt_gpt2_truncate_prompt does;
 *   - greedy picks are appended until the row holds max_len tokens or picks its stop token
 *     (stop_tokens[b]; -1, or stop_tokens NULL, for none), which is kept as its last token.
 * Rows are independent: a row that stops emits nothing more while the others continue, and
 * its tokens are those it gets in a batch of its own. A row whose (truncated) prompt already
 * holds max_len tokens is returned as it is.
 * Outputs (host): out [n, out_stride] with out_stride >= max(min(max_len, ctx_len), 1), row b
 * holding the truncated prompt followed by the picks; out_lens[b] its length. */
int dadgpt_gpt2_generate_tokens(dadgpt_gpt2* model, const int32_t* prompts,
                                const int32_t* prompt_lens, int n, int prompt_stride,
                                int max_len, const int32_t* stop_tokens, int32_t* out,
                                int out_stride, int32_t* out_lens);

#ifdef __cplusplus
}
#endif

#endif /* DADGPT_GPT2_GENERATE_H */
