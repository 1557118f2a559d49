// Batched GPT-2 prefill and greedy decode over the MI355X attention path (the generation stack
// of src/generate.cpp:94-139 and src/model.cpp:659-851, re-planned for a batch of ragged
// prompts). Per layer and step the work is: LayerNorm -> fused QKV GEMM (hipBLASLt) -> QKV
// split with the KV-cache append -> attention (flash forward over the padded batch for the
// prefill; one ragged decode launch for all sequences per decode step) -> Wo GEMM -> bias +
// residual -> LayerNorm -> fc1 GEMM -> bias + GELU -> fc2 GEMM -> bias + residual. Every
// launch is stream-ordered on the model's stream; the host synchronises once per call (or per
// step when the caller asks for every step's logits).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

#include "dadgpt/gpt2_generate.h"
#include "dadgpt/gpu_attention.h"
#include "dadgpt/gpu_matmul.h"
#include "gen_internal.hpp"

namespace dadgpt::gen {

namespace {
thread_local std::string g_last_error;
}

int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return DADGPT_OK;
  return fail(DADGPT_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

namespace {

// Offsets of the reference's parameter arena (src/model.cpp:17-56).
struct Offsets {
  size_t tok_emb = 0, pos_emb = 0;
  struct Layer {
    size_t ln1_w, ln1_b, Wq, bq, Wk, bk, Wv, bv, Wo, bo, ln2_w, ln2_b, fc1_w, fc1_b, fc2_w,
        fc2_b;
  };
  std::vector<Layer> layers;
  size_t lnf_w = 0, lnf_b = 0, total = 0;
};

Offsets offsets_of(const dadgpt_gpt2_config& c) {
  Offsets o;
  size_t at = 0;
  auto take = [&](size_t n) {
    const size_t here = at;
    at += n;
    return here;
  };
  const size_t d = c.d_model, dd = d * d, dff = (size_t)c.d_ff;
  o.tok_emb = take((size_t)c.vocab_size * d);
  o.pos_emb = take((size_t)c.ctx_len * d);
  o.layers.resize(c.n_layers);
  for (auto& L : o.layers) {
    L.ln1_w = take(d);
    L.ln1_b = take(d);
    L.Wq = take(dd);
    L.bq = take(d);
    L.Wk = take(dd);
    L.bk = take(d);
    L.Wv = take(dd);
    L.bv = take(d);
    L.Wo = take(dd);
    L.bo = take(d);
    L.ln2_w = take(d);
    L.ln2_b = take(d);
    L.fc1_w = take(d * dff);
    L.fc1_b = take(dff);
    L.fc2_w = take(dff * d);
    L.fc2_b = take(d);
  }
  o.lnf_w = take(d);
  o.lnf_b = take(d);
  o.total = at;
  return o;
}

bool config_ok(const dadgpt_gpt2_config* c) {
  if (!c || c->d_model < 1 || c->n_layers < 1 || c->n_heads < 1 || c->d_ff < 1 ||
      c->ctx_len < 1 || c->vocab_size < 2)
    return false;
  if (c->d_model % c->n_heads) return false;
  const int dh = c->d_model / c->n_heads;
  return dh == 32 || dh == 64;
}

uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

}  // namespace

}  // namespace dadgpt::gen

using namespace dadgpt::gen;
using dadgpt::gen::bf16;

struct dadgpt_gpt2 {
  dadgpt_gpt2_config c{};
  Offsets off;
  const bf16* params = nullptr;
  int max_batch = 0;
  bool fp32 = false;          // fp32 Q/K/V, caches and attention (modes 1 and 2)
  bool materialized = false;  // mode 2: the materialized path (GEMMs + row softmax)
  bool proj32 = false;        // fp32 projections (fp32 activations and weights; fp32 attention)
  int dh = 0;
  size_t esz = 2;  // bytes per attention element (Q/K/V, caches, attention output)
  dadgpt_blas* blas = nullptr;
  hipStream_t stream = nullptr;
  std::vector<void*> allocs;

  std::vector<bf16*> wqkv;   // per layer [d, 3d]
  std::vector<float*> bqkv;  // per layer [3d]
  // decode steps of at most 16 sequences: transposed weights for the skinny projections
  bool skinny = false;
  std::vector<bf16*> wqkv_t, wo_t, w1_t, w2_t;  // [3d, d], [d, d], [d_ff, d], [d, d_ff]
  std::vector<void*> kc, vc;  // per layer [max_batch, H, ctx, dh]
  // fp32 projections: fp32 copies of the projection weights (exact widenings of the arena)
  std::vector<float*> wqkv32, wo32, w1_32, w2_32;
  float* emb32 = nullptr;

  float *x = nullptr, *qkv = nullptr, *y = nullptr, *f = nullptr, *xl = nullptr;
  float *logits = nullptr, *lse = nullptr, *pick = nullptr;
  float* probs = nullptr;  // materialized mode: [max_batch * H, ctx, ctx] probabilities
  bf16 *h = nullptr, *a = nullptr, *g = nullptr;  // projection inputs (bf16 projections)
  float *h32 = nullptr, *a32 = nullptr, *g32 = nullptr;  // the same with fp32 projections
  void *qh = nullptr, *kh = nullptr, *vh = nullptr, *ao = nullptr;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  int *tok_in = nullptr, *pos0 = nullptr, *nvalid = nullptr, *ones = nullptr, *lens = nullptr;
  // prefill rows packed without padding: padded position b*S + s of each packed row, and the
  // packed row of each prompt's last token
  int *rowmap = nullptr, *lastrow = nullptr;
  int *cur_tok = nullptr, *cur_pos = nullptr, *cache_len = nullptr;
  // where each row stops (RowStop): stop token, length limit, stopped flag; the stopped-row
  // count and its pinned host copies (two slots, read one check late)
  int *stop_tok = nullptr, *limit = nullptr, *done = nullptr, *ndone = nullptr;
  int* h_ndone = nullptr;
  hipEvent_t ndone_ev[2] = {nullptr, nullptr};
  int* out_tok = nullptr;       // [ctx_len, max_batch]: every step any call can take
  float* out_margin = nullptr;
  std::vector<hipEvent_t> events;
  bool use_graphs = true;
  std::map<int, hipGraphExec_t> graphs;  // captured decode step per batch size

  const bf16* P(size_t offset) const { return params + offset; }
  RowStop row_stop() const { return RowStop{stop_tok, limit, done, ndone}; }

  int alloc(void** p, size_t bytes, const char* what) {
    if (hipMalloc(p, bytes < 16 ? 16 : bytes) != hipSuccess)
      return fail(DADGPT_ERR_HIP, "dadgpt_gpt2_create: hipMalloc of %zu bytes (%s) failed", bytes,
                  what);
    allocs.push_back(*p);
    return DADGPT_OK;
  }
  template <typename T>
  int alloc_n(T** p, size_t count, const char* what) {
    return alloc(reinterpret_cast<void**>(p), count * sizeof(T), what);
  }
};

namespace {

// Prefill attention over n padded prompts of S rows. fp32: split heads [n*H, S, dh] in
// m->qh/kh/vh -> m->ao (merged into the packed rows afterwards). bf16: Q heads from m->qh, K
// and V read in place from the layer's cache (rows 0..S-1 of [max_batch, H, ctx, dh]), and
// the output written token-major into m->ao (padded rows), gathered into the packed rows of
// the Wo GEMM's input afterwards: no split K/V copies.
int attention_prefill(dadgpt_gpt2* m, int layer, int n, int S, float scale) {
  const int H = m->c.n_heads, dh = m->dh;
  if (m->materialized) {
    const long long sl = (long long)S * dh;
    return materialized_forward(m->blas, (float*)m->ao, m->probs, (const float*)m->qh,
                                (const float*)m->kh, (const float*)m->vh, n * H, S, dh, scale,
                                sl, sl, sl, m->stream);
  }
  if (m->fp32)
    return dadgpt_flash_attention_forward_async((float*)m->ao, m->lse, (const float*)m->qh,
                                                (const float*)m->kh, (const float*)m->vh, n * H,
                                                S, dh, scale, m->stream);
  const int64_t ctx = m->c.ctx_len, d = (int64_t)H * dh;
  const dadgpt_head_strides heads{d * S, (int64_t)S * dh, dh}, cache{d * ctx, ctx * dh, dh},
      tokens{d * S, dh, d};
  const dadgpt_head_strides st[4] = {heads, cache, cache, tokens};
  return dadgpt_flash_attention_forward_bf16_strided(
      (uint16_t*)m->ao, m->lse, (const uint16_t*)m->qh, (const uint16_t*)m->kc[layer],
      (const uint16_t*)m->vc[layer], n, H, S, dh, scale, st, m->stream);
}

int attention_decode(dadgpt_gpt2* m, int layer, int n, float scale) {
  const int H = m->c.n_heads, L = m->c.ctx_len;
  if (m->materialized)
    return materialized_decode(m->blas, (float*)m->ao, m->probs, (const float*)m->qh,
                               (const float*)m->kc[layer], (const float*)m->vc[layer],
                               m->cache_len, n, H, L, m->dh, scale, m->stream);
  if (m->fp32)
    return dadgpt_decode_attention_f32((float*)m->ao, (const float*)m->qh,
                                       (const float*)m->kc[layer], (const float*)m->vc[layer],
                                       m->cache_len, n, H, L, m->dh, scale, m->ws, m->ws_bytes,
                                       m->stream);
  return dadgpt_decode_attention_bf16((uint16_t*)m->ao, (const uint16_t*)m->qh,
                                      (const uint16_t*)m->kc[layer],
                                      (const uint16_t*)m->vc[layer], m->cache_len, n, H, L,
                                      m->dh, scale, m->ws, m->ws_bytes, m->stream);
}

// The attention error of the C ABI is recorded by libdadgpt_attn; carry it over (the
// materialized path records its own, in this library).
int attn_fail(const dadgpt_gpt2* m, int st, const char* what) {
  if (m->materialized) return st;
  return fail(st, "%s: %s", what, dadgpt_last_error());
}

#define TRY(expr)                          \
  do {                                     \
    if (int st_ = (expr)) return st_;      \
  } while (0)
#define TRY_HIP(expr, what) TRY(check_hip((expr), (what)))

// A projection out[M,N] (fp32) = in[M,K] W[K,N] (or W[N,K]^T): bf16 operands, or with fp32
// projections the fp32 activations and weights (the reference's default fp32 matmuls).
int proj(dadgpt_gpt2* m, float* out, const void* in, const bf16* w, const float* w32, int M,
         int K, int N, bool trans_b) {
  if (m->proj32)
    return gemm_f32(m->blas, out, static_cast<const float*>(in), w32, M, K, N,
                    trans_b ? 'B' : 'N', 0.0f, 1, 0, 0, 0, m->stream);
  return gemm(m->blas, out, static_cast<const bf16*>(in), w, M, K, N, trans_b, m->stream);
}
const void* in_h(const dadgpt_gpt2* m) { return m->proj32 ? (const void*)m->h32 : m->h; }
const void* in_g(const dadgpt_gpt2* m) { return m->proj32 ? (const void*)m->g32 : m->g; }

// x += y + bias (when y), then LayerNorm(x) * w + b (when w) into the projection input h.
int layernorm_h(dadgpt_gpt2* m, float* x, const float* y, const bf16* bias, const bf16* w,
                const bf16* b, int rows) {
  const int d = m->c.d_model;
  const hipError_t e =
      m->proj32 ? residual_layernorm<float>(x, y, bias, m->h32, w, b, rows, d, m->stream)
                : residual_layernorm<bf16>(x, y, bias, m->h, w, b, rows, d, m->stream);
  return check_hip(e, "residual_layernorm");
}

// One transformer block over `rows` rows. prefill: the prompts' positions packed without
// padding (m->rowmap gives each row's place b*S + s in the padded [n, S] batch the attention
// runs on; K/V appended for s < len); otherwise one token per sequence at cur_pos (rows = n,
// S = 1). attn_ev: optional pair of events around the attention launch.
int block(dadgpt_gpt2* m, int l, int n, int S, int rows, bool prefill, hipEvent_t* attn_ev) {
  const auto& c = m->c;
  const auto& L = m->off.layers[l];
  const int d = c.d_model, H = c.n_heads, dh = m->dh;
  const float scale = 1.0f / std::sqrt(static_cast<float>(dh));  // src/model.cpp:389
  hipStream_t s = m->stream;

  // h holds LayerNorm 1 of x (written by whichever kernel last updated x)
  TRY(proj(m, m->qkv, in_h(m), m->wqkv[l], m->proj32 ? m->wqkv32[l] : nullptr, rows, d, 3 * d,
           false));
  const void* attn_in = m->proj32 ? (const void*)m->a32 : m->a;
  if (prefill) {
    if (m->fp32)
      TRY_HIP(qkv_split<float>((float*)m->qh, (float*)m->kh, (float*)m->vh, (float*)m->kc[l],
                               (float*)m->vc[l], m->qkv, m->bqkv[l], m->pos0, m->nvalid,
                               m->rowmap, rows, S, H, dh, c.ctx_len, s),
              "qkv_split");
    else  // Q heads and the cache append only
      TRY_HIP(qkv_split<bf16>((bf16*)m->qh, nullptr, nullptr, (bf16*)m->kc[l], (bf16*)m->vc[l],
                              m->qkv, m->bqkv[l], m->pos0, m->nvalid, m->rowmap, rows, S, H,
                              dh, c.ctx_len, s),
              "qkv_split");
    if (int st = attention_prefill(m, l, n, S, scale))
      return attn_fail(m, st, "prefill attention");
    if (m->proj32)
      TRY_HIP((merge_heads<float, float>(m->a32, (const float*)m->ao, m->rowmap, rows, S, H, dh,
                                         s)),
              "merge_heads");
    else if (m->fp32)
      TRY_HIP((merge_heads<float, bf16>(m->a, (const float*)m->ao, m->rowmap, rows, S, H, dh, s)),
              "merge_heads");
    else
      TRY_HIP(gather_rows<bf16>(m->a, (const bf16*)m->ao, m->rowmap, rows, d, s),
              "gather_rows(attention)");
  } else {
    if (m->fp32)
      TRY_HIP(qkv_split<float>((float*)m->qh, nullptr, nullptr, (float*)m->kc[l],
                               (float*)m->vc[l], m->qkv, m->bqkv[l], m->cur_pos, m->ones,
                               nullptr, n, 1, H, dh, c.ctx_len, s),
              "qkv_split");
    else
      TRY_HIP(qkv_split<bf16>((bf16*)m->qh, nullptr, nullptr, (bf16*)m->kc[l], (bf16*)m->vc[l],
                              m->qkv, m->bqkv[l], m->cur_pos, m->ones, nullptr, n, 1, H, dh,
                              c.ctx_len, s),
              "qkv_split");
    if (attn_ev) TRY_HIP(hipEventRecord(attn_ev[0], s), "hipEventRecord");
    if (int st = attention_decode(m, l, n, scale)) return attn_fail(m, st, "decode attention");
    if (attn_ev) TRY_HIP(hipEventRecord(attn_ev[1], s), "hipEventRecord");
    // decode output [n, H, dh] is already the [n, d] row layout
    if (m->proj32)
      attn_in = m->ao;
    else if (m->fp32)
      TRY_HIP(to_bf16(m->a, (const float*)m->ao, (size_t)n * d, s), "to_bf16");
    else
      attn_in = m->ao;
  }
  TRY(proj(m, m->y, attn_in, m->P(L.Wo), m->proj32 ? m->wo32[l] : nullptr, rows, d, d, false));
  TRY(layernorm_h(m, m->x, m->y, m->P(L.bo), m->P(L.ln2_w), m->P(L.ln2_b), rows));
  TRY(proj(m, m->f, in_h(m), m->P(L.fc1_w), m->proj32 ? m->w1_32[l] : nullptr, rows, d, c.d_ff,
           false));
  TRY_HIP(m->proj32 ? bias_gelu<float>(m->g32, m->f, m->P(L.fc1_b), rows, c.d_ff, s)
                    : bias_gelu<bf16>(m->g, m->f, m->P(L.fc1_b), rows, c.d_ff, s),
          "bias_gelu");
  TRY(proj(m, m->y, in_g(m), m->P(L.fc2_w), m->proj32 ? m->w2_32[l] : nullptr, rows, c.d_ff, d,
           false));
  // the residual add, fused with the next LayerNorm: layer l+1's LayerNorm 1, or after the
  // last layer the final LayerNorm (decode; the prefill normalises only the gathered rows)
  const bf16 *nw = nullptr, *nb = nullptr;
  if (l + 1 < c.n_layers) {
    nw = m->P(m->off.layers[l + 1].ln1_w);
    nb = m->P(m->off.layers[l + 1].ln1_b);
  } else if (!prefill) {
    nw = m->P(m->off.lnf_w);
    nb = m->P(m->off.lnf_b);
  }
  TRY(layernorm_h(m, m->x, m->y, m->P(L.fc2_b), nw, nb, rows));
  return DADGPT_OK;
}

// LayerNorm 1 of layer 0 over freshly embedded rows.
int first_layernorm(dadgpt_gpt2* m, int rows) {
  const auto& L0 = m->off.layers[0];
  return layernorm_h(m, m->x, nullptr, nullptr, m->P(L0.ln1_w), m->P(L0.ln1_b), rows);
}

// Weight-tied logits of the n final-LayerNorm rows in m->h, greedy pick (stored at the step
// the device state implies), and the embedding of each picked token at its position into
// x[0, n), the next decode step's input.
int head(dadgpt_gpt2* m, int n) {
  const auto& c = m->c;
  hipStream_t s = m->stream;
  TRY(proj(m, m->logits, in_h(m), m->P(m->off.tok_emb), m->emb32, n, c.d_model, c.vocab_size,
           true));
  TRY_HIP(argmax_advance(m->out_tok, m->out_margin, m->cur_tok, m->cur_pos, m->cache_len,
                         m->lens, m->row_stop(), m->logits, m->pick, n, c.vocab_size, m->x,
                         m->P(m->off.tok_emb), m->P(m->off.pos_emb), c.d_model, c.ctx_len, s),
          "argmax_advance");
  return DADGPT_OK;
}

// One decode step for n sequences: the blocks over x (each sequence's last token embedded at
// its position by the previous head), then the head. Everything it reads and advances is
// device state, so a captured copy replays for every step.
int decode_step_skinny(dadgpt_gpt2* m, int n, hipEvent_t* attn_ev);

int decode_step(dadgpt_gpt2* m, int n, hipEvent_t* attn_ev) {
  if (m->skinny && n <= 16) return decode_step_skinny(m, n, attn_ev);
  const auto& c = m->c;
  TRY(first_layernorm(m, n));
  for (int l = 0; l < c.n_layers; ++l)
    TRY(block(m, l, n, 1, n, false, attn_ev ? attn_ev + 2 * l : nullptr));
  return head(m, n);
}

// The decode step on the skinny projections (n <= 16 sequences). Per layer 5 dependent
// launches, each projection doing the elementwise work around it (see skinny.hip):
// QKV (LayerNorm 1 of x in its prologue; bias, q out, K/V appended to the caches) -> decode
// attention -> Wo (bias + residual add into x) -> fc1 (LayerNorm 2 of x; bias + GELU into g)
// -> fc2 (bias + residual add into x). x is the fp32 residual stream.
int decode_step_skinny(dadgpt_gpt2* m, int n, hipEvent_t* attn_ev) {
  const auto& c = m->c;
  const int d = c.d_model, H = c.n_heads, dh = m->dh;
  const float scale = 1.0f / std::sqrt(static_cast<float>(dh));  // src/model.cpp:389
  hipStream_t s = m->stream;
  for (int l = 0; l < c.n_layers; ++l) {
    const auto& L = m->off.layers[l];
    SkinnyArgs q{};
    q.wt = m->wqkv_t[l];
    q.M = n, q.N = 3 * d, q.K = d;
    q.x = m->x, q.ln_w = m->P(L.ln1_w), q.ln_b = m->P(L.ln1_b);
    q.bias_f = m->bqkv[l];
    q.q = m->qh, q.kcache = m->kc[l], q.vcache = m->vc[l], q.pos = m->cur_pos;
    q.H = H, q.dh = dh, q.max_len = c.ctx_len, q.qkv_fp32 = m->fp32;
    TRY_HIP(skinny_gemm(kProLn, kEpiQkv, q, s), "skinny QKV");
    if (attn_ev) TRY_HIP(hipEventRecord(attn_ev[2 * l], s), "hipEventRecord");
    if (int st = attention_decode(m, l, n, scale)) return attn_fail(m, st, "decode attention");
    if (attn_ev) TRY_HIP(hipEventRecord(attn_ev[2 * l + 1], s), "hipEventRecord");
    // the attention output [n, H, dh] is the [n, d] row layout; fp32 attention's is rounded to
    // bf16 inside the Wo kernel (the skinny path runs with bf16 projections only)
    SkinnyArgs o{};
    o.wt = m->wo_t[l];
    o.M = n, o.N = d, o.K = d;
    if (m->fp32)
      o.act32 = (const float*)m->ao;
    else
      o.act = (const bf16*)m->ao;
    o.bias = m->P(L.bo), o.x_out = m->x;
    TRY_HIP(skinny_gemm(m->fp32 ? kProRowsF32 : kProRows, kEpiResidual, o, s), "skinny Wo");

    SkinnyArgs f1{};
    f1.wt = m->w1_t[l];
    f1.M = n, f1.N = c.d_ff, f1.K = d;
    f1.x = m->x, f1.ln_w = m->P(L.ln2_w), f1.ln_b = m->P(L.ln2_b);
    f1.bias = m->P(L.fc1_b), f1.g = m->g;
    TRY_HIP(skinny_gemm(kProLn, kEpiGelu, f1, s), "skinny fc1");

    SkinnyArgs f2{};
    f2.wt = m->w2_t[l];
    f2.M = n, f2.N = d, f2.K = c.d_ff;
    f2.act = m->g;  // K-blocked by fc1's epilogue
    f2.bias = m->P(L.fc2_b), f2.x_out = m->x;
    TRY_HIP(skinny_gemm(kProRowsBlocked, kEpiResidual, f2, s), "skinny fc2");
  }
  // final LayerNorm, then the tied logits
  TRY_HIP(residual_layernorm<bf16>(m->x, nullptr, nullptr, m->h, m->P(m->off.lnf_w),
                                   m->P(m->off.lnf_b), n, d, s, 1, /*blocked=*/true),
          "residual_layernorm");
  SkinnyArgs lg{};
  lg.wt = m->P(m->off.tok_emb);  // [V, d]: already W^T of the tied projection
  lg.M = n, lg.N = c.vocab_size, lg.K = d;
  lg.act = m->h;
  lg.out = m->logits;
  lg.cand = m->pick;  // each workgroup's greedy candidate per row
  TRY_HIP(skinny_gemm(kProRowsBlocked, kEpiStore, lg, s), "skinny logits");
  TRY_HIP(pick_advance(m->out_tok, m->out_margin, m->cur_tok, m->cur_pos, m->cache_len,
                       m->lens, m->row_stop(), m->pick, skinny_store_parts(c.vocab_size),
                       kSkinnyRows, n,
                       c.vocab_size, m->x, m->P(m->off.tok_emb), m->P(m->off.pos_emb), d,
                       c.ctx_len, s),
          "pick_advance");
  return DADGPT_OK;
}

// The captured decode step for batch size n (captured on first use; hipBLASLt plans must
// already exist, so the caller runs one eager step first).
int step_graph(dadgpt_gpt2* m, int n, hipGraphExec_t* out) {
  auto it = m->graphs.find(n);
  if (it != m->graphs.end()) {
    *out = it->second;
    return DADGPT_OK;
  }
  hipGraph_t graph = nullptr;
  TRY_HIP(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal),
          "hipStreamBeginCapture");
  const int st = decode_step(m, n, nullptr);
  const hipError_t e = hipStreamEndCapture(m->stream, &graph);
  if (st) {
    if (graph) (void)hipGraphDestroy(graph);
    return st;
  }
  TRY_HIP(e, "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  TRY_HIP(ei, "hipGraphInstantiate");
  m->graphs[n] = exec;
  *out = exec;
  return DADGPT_OK;
}

int copy_logits(dadgpt_gpt2* m, float* host, int n, int step) {
  const size_t count = (size_t)n * m->c.vocab_size;
  TRY_HIP(hipMemcpyAsync(host + (size_t)step * count, m->logits, count * sizeof(float),
                         hipMemcpyDeviceToHost, m->stream),
          "hipMemcpyAsync(logits)");
  TRY_HIP(hipStreamSynchronize(m->stream), "hipStreamSynchronize");
  return DADGPT_OK;
}

int ensure_events(dadgpt_gpt2* m, size_t count) {
  while (m->events.size() < count) {
    hipEvent_t e;
    TRY_HIP(hipEventCreate(&e), "hipEventCreate");
    m->events.push_back(e);
  }
  return DADGPT_OK;
}

}  // namespace

extern "C" {

const char* dadgpt_gen_last_error(void) { return g_last_error.c_str(); }

size_t dadgpt_gpt2_param_count(const dadgpt_gpt2_config* config) {
  return config_ok(config) ? offsets_of(*config).total : 0;
}

int dadgpt_gpt2_init_params(uint16_t* params, const dadgpt_gpt2_config* config, uint64_t seed,
                            void* stream) {
  if (!params || !config_ok(config))
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "dadgpt_gpt2_init_params: bad arguments");
  const auto& c = *config;
  const Offsets o = offsets_of(c);
  bf16* p = reinterpret_cast<bf16*>(params);
  hipStream_t s = (hipStream_t)stream;
  const float sd = 0.02f;
  const float res_sd = sd / std::sqrt(2.0f * static_cast<float>(c.n_layers));  // model.cpp:139
  const size_t d = c.d_model, dd = d * d, dff = (size_t)c.d_ff * d;
  uint64_t tensor = 0;
  auto normal = [&](size_t off, size_t count, float stddev) {
    return check_hip(init_normal(p + off, count, mix64(seed ^ mix64(++tensor)), stddev, s),
                     "init_normal");
  };
  auto constant = [&](size_t off, size_t count, float v) {
    return check_hip(fill(p + off, count, v, s), "fill");
  };
  TRY(constant(0, o.total, 0.0f));  // biases
  TRY(normal(o.tok_emb, (size_t)c.vocab_size * d, sd));
  TRY(normal(o.pos_emb, (size_t)c.ctx_len * d, sd));
  for (const auto& L : o.layers) {
    TRY(constant(L.ln1_w, d, 1.0f));
    TRY(constant(L.ln2_w, d, 1.0f));
    TRY(normal(L.Wq, dd, sd));
    TRY(normal(L.Wk, dd, sd));
    TRY(normal(L.Wv, dd, sd));
    TRY(normal(L.Wo, dd, res_sd));
    TRY(normal(L.fc1_w, dff, sd));
    TRY(normal(L.fc2_w, dff, res_sd));
  }
  TRY(constant(o.lnf_w, d, 1.0f));
  return DADGPT_OK;
}

void dadgpt_gpt2_destroy(dadgpt_gpt2* m) {
  if (!m) return;
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  for (hipEvent_t e : m->events) (void)hipEventDestroy(e);
  for (hipEvent_t e : m->ndone_ev)
    if (e) (void)hipEventDestroy(e);
  if (m->h_ndone) (void)hipHostFree(m->h_ndone);
  for (auto& [n, g] : m->graphs) (void)hipGraphExecDestroy(g);
  for (void* p : m->allocs) (void)hipFree(p);
  if (m->blas) dadgpt_blas_destroy(m->blas);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
}

int dadgpt_gpt2_create(const dadgpt_gpt2_config* config, const uint16_t* params, int max_batch,
                       int attn_mode, dadgpt_gpt2** out) {
  const int attn = attn_mode & 0xff;
  const bool proj32 = (attn_mode & DADGPT_GPT2_FP32_PROJECTIONS) != 0;
  if (!out || !params || !config_ok(config) || max_batch < 1 || config->d_model > 2048 ||
      attn < DADGPT_GPT2_ATTN_BF16 || attn > DADGPT_GPT2_ATTN_FP32_MATERIALIZED ||
      (attn_mode & ~(0xff | DADGPT_GPT2_FP32_PROJECTIONS)) != 0 ||
      (proj32 && attn == DADGPT_GPT2_ATTN_BF16))
    return fail(DADGPT_ERR_INVALID_ARGUMENT,
                "dadgpt_gpt2_create: bad arguments (d_head must be 32 or 64, d_model <= 2048, "
                "max_batch >= 1, attention mode 0, 1 or 2, fp32 projections only with fp32 "
                "attention)");
  *out = nullptr;
  auto* m = new dadgpt_gpt2();
  m->c = *config;
  m->off = offsets_of(m->c);
  m->params = reinterpret_cast<const bf16*>(params);
  m->max_batch = max_batch;
  m->fp32 = attn != DADGPT_GPT2_ATTN_BF16;
  m->materialized = attn == DADGPT_GPT2_ATTN_FP32_MATERIALIZED;
  m->proj32 = proj32;
  m->dh = m->c.d_model / m->c.n_heads;
  m->esz = m->fp32 ? sizeof(float) : sizeof(bf16);
  const auto& c = m->c;
  const size_t d = c.d_model, rows = (size_t)max_batch * c.ctx_len;
  auto bail = [&](int st) {
    dadgpt_gpt2_destroy(m);
    return st;
  };
  if (hipStreamCreate(&m->stream) != hipSuccess)
    return bail(fail(DADGPT_ERR_HIP, "dadgpt_gpt2_create: hipStreamCreate failed"));
  if (int st = dadgpt_blas_create(&m->blas)) return bail(st);

  // fused QKV weights [d, 3d] (Wq | Wk | Wv along the output dimension) and fp32 biases
  m->wqkv.resize(c.n_layers);
  m->bqkv.resize(c.n_layers);
  m->kc.resize(c.n_layers);
  m->vc.resize(c.n_layers);
  const size_t cache = (size_t)max_batch * c.n_heads * c.ctx_len * m->dh * m->esz;
  for (int l = 0; l < c.n_layers; ++l) {
    const auto& L = m->off.layers[l];
    if (int st = m->alloc_n(&m->wqkv[l], d * 3 * d, "wqkv")) return bail(st);
    if (int st = m->alloc_n(&m->bqkv[l], 3 * d, "bqkv")) return bail(st);
    const size_t wbytes = d * sizeof(bf16);
    const size_t src[3] = {L.Wq, L.Wk, L.Wv};
    for (int j = 0; j < 3; ++j)
      if (hipMemcpy2DAsync(m->wqkv[l] + j * d, 3 * wbytes, m->P(src[j]), wbytes, wbytes, d,
                           hipMemcpyDeviceToDevice, m->stream) != hipSuccess)
        return bail(fail(DADGPT_ERR_HIP, "dadgpt_gpt2_create: QKV weight repack failed"));
    if (int st = check_hip(pack_bias(m->bqkv[l], m->P(L.bq), m->P(L.bk), m->P(L.bv), (int)d,
                                     m->stream),
                           "pack_bias"))
      return bail(st);
    if (int st = m->alloc(&m->kc[l], cache, "k cache")) return bail(st);
    if (int st = m->alloc(&m->vc[l], cache, "v cache")) return bail(st);
    // zero rows past a prompt: the bf16 prefill reads K and V from the cache, and padded
    // queries (discarded) see rows no prompt wrote
    if (hipMemsetAsync(m->kc[l], 0, cache, m->stream) != hipSuccess ||
        hipMemsetAsync(m->vc[l], 0, cache, m->stream) != hipSuccess)
      return bail(fail(DADGPT_ERR_HIP, "dadgpt_gpt2_create: cache clear failed"));
  }
  const size_t ab = m->esz;
  int st = DADGPT_OK;
  if ((st = m->alloc_n(&m->x, rows * d, "x")) || (st = m->alloc_n(&m->qkv, rows * 3 * d, "qkv")) ||
      (st = m->alloc_n(&m->y, rows * d, "y")) ||
      (st = m->alloc_n(&m->f, rows * c.d_ff, "fc1 out")) ||
      (st = m->alloc_n(&m->xl, (size_t)max_batch * d, "last rows")) ||
      (st = m->alloc_n(&m->logits, (size_t)max_batch * c.vocab_size, "logits")) ||
      // the two-stage pick's candidates, or the skinny logits' per-workgroup ones (16 rows)
      (st = m->alloc_n(&m->pick,
                       pick_scratch_floats(std::max(max_batch, kSkinnyRows),
                                           skinny_store_parts(c.vocab_size)),
                       "pick scratch")) ||
      (st = m->alloc_n(&m->lse, rows * c.n_heads, "lse")) ||
      // (the decode step's final LayerNorm writes, and the skinny logits read, 16 K-blocked
      // rows whatever max_batch * ctx_len is)
      (!proj32 && (st = m->alloc_n(&m->h, std::max(rows, (size_t)kSkinnyRows) * d, "ln out"))) ||
      (!proj32 && (st = m->alloc_n(&m->a, rows * d, "attn in"))) ||
      // (the skinny fc1 writes 16 K-blocked rows, whatever max_batch is)
      (!proj32 && (st = m->alloc_n(&m->g, std::max(rows, (size_t)kSkinnyRows) * c.d_ff,
                                   "gelu out"))) ||
      (proj32 && (st = m->alloc_n(&m->h32, rows * d, "ln out"))) ||
      (proj32 && (st = m->alloc_n(&m->a32, rows * d, "attn in"))) ||
      (proj32 && (st = m->alloc_n(&m->g32, rows * c.d_ff, "gelu out"))) ||
      (st = m->alloc(&m->qh, rows * d * ab, "q heads")) ||
      // split K and V heads: fp32 attention only (bf16 reads them from the cache)
      (m->fp32 && (st = m->alloc(&m->kh, rows * d * ab, "k heads"))) ||
      (m->fp32 && (st = m->alloc(&m->vh, rows * d * ab, "v heads"))) ||
      (st = m->alloc(&m->ao, rows * d * ab, "attn out")) ||
      (st = m->alloc_n(&m->tok_in, rows, "tokens")) ||
      (st = m->alloc_n(&m->rowmap, rows, "prefill row map")) ||
      (st = m->alloc_n(&m->lastrow, max_batch, "prefill last rows")) ||
      (st = m->alloc_n(&m->pos0, max_batch, "pos0")) ||
      (st = m->alloc_n(&m->nvalid, max_batch, "nvalid")) ||
      (st = m->alloc_n(&m->ones, max_batch, "ones")) ||
      (st = m->alloc_n(&m->lens, max_batch, "lens")) ||
      (st = m->alloc_n(&m->cur_tok, max_batch, "cur_tok")) ||
      (st = m->alloc_n(&m->cur_pos, max_batch, "cur_pos")) ||
      (st = m->alloc_n(&m->cache_len, max_batch, "cache_len")) ||
      (st = m->alloc_n(&m->stop_tok, max_batch, "stop tokens")) ||
      (st = m->alloc_n(&m->limit, max_batch, "length limits")) ||
      (st = m->alloc_n(&m->done, max_batch, "stopped rows")) ||
      (st = m->alloc_n(&m->ndone, 1, "stopped count")) ||
      (st = m->alloc_n(&m->out_tok, rows, "tokens out")) ||
      (st = m->alloc_n(&m->out_margin, rows, "margins out")) ||
      // materialized attention: the prefill's [n*H, S, S] probabilities (the decode's
      // [n*H, ctx] rows fit in the same buffer)
      (m->materialized && (st = m->alloc_n(&m->probs, rows * c.n_heads * c.ctx_len,
                                           "attention probabilities"))))
    return bail(st);
  // the skinny decode path: reduction lengths the kernels are built for, LayerNorm rows that
  // fit the prologue's registers
  m->skinny = !proj32 && skinny_supported(1, c.d_model) && skinny_supported(1, c.d_ff) &&
              c.d_model <= 1024;
  if (proj32) {  // fp32 weights: widened once from the bf16 arena (exact)
    m->wqkv32.resize(c.n_layers);
    m->wo32.resize(c.n_layers);
    m->w1_32.resize(c.n_layers);
    m->w2_32.resize(c.n_layers);
    auto widen = [&](float** dst, const bf16* src, size_t count, const char* what) {
      if (int e = m->alloc_n(dst, count, what)) return e;
      return check_hip(to_f32(*dst, src, count, m->stream), "to_f32");
    };
    for (int l = 0; l < c.n_layers; ++l) {
      const auto& L = m->off.layers[l];
      if ((st = widen(&m->wqkv32[l], m->wqkv[l], 3 * d * d, "wqkv fp32")) ||
          (st = widen(&m->wo32[l], m->P(L.Wo), d * d, "wo fp32")) ||
          (st = widen(&m->w1_32[l], m->P(L.fc1_w), d * c.d_ff, "fc1 fp32")) ||
          (st = widen(&m->w2_32[l], m->P(L.fc2_w), (size_t)c.d_ff * d, "fc2 fp32")))
        return bail(st);
    }
    if ((st = widen(&m->emb32, m->P(m->off.tok_emb), (size_t)c.vocab_size * d, "tok_emb fp32")))
      return bail(st);
  }
  if (m->skinny) {
    m->wqkv_t.resize(c.n_layers);
    m->wo_t.resize(c.n_layers);
    m->w1_t.resize(c.n_layers);
    m->w2_t.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
      const auto& L = m->off.layers[l];
      if ((st = m->alloc_n(&m->wqkv_t[l], 3 * d * d, "wqkv^T")) ||
          (st = m->alloc_n(&m->wo_t[l], d * d, "wo^T")) ||
          (st = m->alloc_n(&m->w1_t[l], (size_t)c.d_ff * d, "fc1^T")) ||
          (st = m->alloc_n(&m->w2_t[l], (size_t)d * c.d_ff, "fc2^T")))
        return bail(st);
      if ((st = check_hip(transpose(m->wqkv_t[l], m->wqkv[l], (int)d, 3 * (int)d, m->stream),
                          "transpose")) ||
          (st = check_hip(transpose(m->wo_t[l], m->P(L.Wo), (int)d, (int)d, m->stream),
                          "transpose")) ||
          (st = check_hip(transpose(m->w1_t[l], m->P(L.fc1_w), (int)d, c.d_ff, m->stream),
                          "transpose")) ||
          (st = check_hip(transpose(m->w2_t[l], m->P(L.fc2_w), c.d_ff, (int)d, m->stream),
                          "transpose")))
        return bail(st);
    }
  }
  m->ws_bytes = dadgpt_decode_workspace_bytes(max_batch, c.n_heads, c.ctx_len, m->dh);
  if (m->ws_bytes) {
    if ((st = m->alloc(&m->ws, m->ws_bytes, "decode workspace"))) return bail(st);
    if (hipMemsetAsync(m->ws, 0, m->ws_bytes, m->stream) != hipSuccess)
      return bail(fail(DADGPT_ERR_HIP, "dadgpt_gpt2_create: workspace clear failed"));
  }
  // Split heads: a packed prefill writes only the prompt rows. The padded K/V rows of fp32
  // attention are multiplied by exact-zero probabilities and must not hold NaN or Inf bit
  // patterns; the padded Q rows are discarded queries, kept finite too (zero until a call
  // writes them).
  if (hipMemsetAsync(m->qh, 0, rows * d * ab, m->stream) != hipSuccess ||
      (m->fp32 && (hipMemsetAsync(m->kh, 0, rows * d * ab, m->stream) != hipSuccess ||
                   hipMemsetAsync(m->vh, 0, rows * d * ab, m->stream) != hipSuccess)))
    return bail(fail(DADGPT_ERR_HIP, "dadgpt_gpt2_create: split-head clear failed"));
  if (hipHostMalloc((void**)&m->h_ndone, 2 * sizeof(int), hipHostMallocDefault) != hipSuccess) {
    m->h_ndone = nullptr;
    return bail(fail(DADGPT_ERR_HIP, "dadgpt_gpt2_create: hipHostMalloc failed"));
  }
  for (hipEvent_t& e : m->ndone_ev)
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
      e = nullptr;
      return bail(fail(DADGPT_ERR_HIP, "dadgpt_gpt2_create: hipEventCreate failed"));
    }
  std::vector<int> ones(max_batch, 1), zeros(max_batch, 0);
  if (hipMemcpyAsync(m->ones, ones.data(), max_batch * sizeof(int), hipMemcpyHostToDevice,
                     m->stream) != hipSuccess ||
      hipMemcpyAsync(m->pos0, zeros.data(), max_batch * sizeof(int), hipMemcpyHostToDevice,
                     m->stream) != hipSuccess ||
      hipStreamSynchronize(m->stream) != hipSuccess)
    return bail(fail(DADGPT_ERR_HIP, "dadgpt_gpt2_create: initial copies failed"));
  *out = m;
  return DADGPT_OK;
}

int dadgpt_gpt2_set_graphs(dadgpt_gpt2* m, int enable) {
  if (!m) return fail(DADGPT_ERR_INVALID_ARGUMENT, "dadgpt_gpt2_set_graphs: null model");
  m->use_graphs = enable != 0;
  return DADGPT_OK;
}

}  // extern "C"

namespace {

// Greedy generation over validated prompts (1 <= len[b] <= prompt_stride, tokens in the
// vocabulary, len[b] < limit[b] <= ctx_len): row b stops at its stop token (stop[b], -1 for
// none) or when it reaches limit[b] tokens, prompt included (src/generate.cpp:121-135).
// max_new = max_b (limit[b] - len[b]) picks at most. tk/mg receive the picks and margins
// step-major [max_new][n]: row b's entries are valid up to its last pick. With early_exit, the
// step loop ends once every row has stopped (checked every kCheck steps, one check late, so
// the host never waits on a step it has just queued).
int generate_core(dadgpt_gpt2* m, const int32_t* prompts, const int32_t* prompt_lens, int n,
                  int prompt_stride, const int* limit, const int* stop, int max_new,
                  bool early_exit, std::vector<int>& tk, std::vector<float>& mg, float* logits,
                  dadgpt_gpt2_timing* timing) {
  const auto& c = m->c;
  int S = 0;
  for (int b = 0; b < n; ++b) S = std::max(S, (int)prompt_lens[b]);
  hipStream_t s = m->stream;
  const size_t outs = (size_t)max_new * n;  // <= ctx_len * max_batch, the buffers' size

  // padded prompt rows, lengths, the position before the first generated token, and the
  // packed prefill rows (every prompt position once, no padding): their padded positions and
  // each prompt's last one
  std::vector<int> tok((size_t)n * S, 0), len(prompt_lens, prompt_lens + n), pos(n), rowmap,
      lastrow(n), stops(n, -1), limits(limit, limit + n);
  rowmap.reserve((size_t)n * S);
  for (int b = 0; b < n; ++b) {
    for (int t = 0; t < len[b]; ++t) {
      tok[(size_t)b * S + t] = prompts[(size_t)b * prompt_stride + t];
      rowmap.push_back(b * S + t);
    }
    lastrow[b] = (int)rowmap.size() - 1;
    pos[b] = len[b] - 1;
    if (stop) stops[b] = stop[b];
  }
  const int rows = (int)rowmap.size();
  TRY_HIP(hipMemcpyAsync(m->tok_in, tok.data(), tok.size() * sizeof(int), hipMemcpyHostToDevice, s),
          "hipMemcpyAsync(tokens)");
  TRY_HIP(hipMemcpyAsync(m->rowmap, rowmap.data(), rows * sizeof(int), hipMemcpyHostToDevice, s),
          "hipMemcpyAsync(row map)");
  TRY_HIP(hipMemcpyAsync(m->lastrow, lastrow.data(), n * sizeof(int), hipMemcpyHostToDevice, s),
          "hipMemcpyAsync(last rows)");
  TRY_HIP(hipMemcpyAsync(m->nvalid, len.data(), n * sizeof(int), hipMemcpyHostToDevice, s),
          "hipMemcpyAsync(lens)");
  TRY_HIP(hipMemcpyAsync(m->lens, len.data(), n * sizeof(int), hipMemcpyHostToDevice, s),
          "hipMemcpyAsync(lens)");
  TRY_HIP(hipMemcpyAsync(m->cur_pos, pos.data(), n * sizeof(int), hipMemcpyHostToDevice, s),
          "hipMemcpyAsync(pos)");
  TRY_HIP(hipMemcpyAsync(m->stop_tok, stops.data(), n * sizeof(int), hipMemcpyHostToDevice, s),
          "hipMemcpyAsync(stop tokens)");
  TRY_HIP(hipMemcpyAsync(m->limit, limits.data(), n * sizeof(int), hipMemcpyHostToDevice, s),
          "hipMemcpyAsync(length limits)");
  TRY_HIP(hipMemsetAsync(m->done, 0, n * sizeof(int), s), "hipMemsetAsync(stopped rows)");
  TRY_HIP(hipMemsetAsync(m->ndone, 0, sizeof(int), s), "hipMemsetAsync(stopped count)");

  const int steps = max_new - 1;
  const bool timed = timing != nullptr;
  // Only a decode step made of this library's own kernels is captured and replayed (the
  // skinny step of up to 16 sequences with bf16 projections and flash decode attention). A
  // step with hipBLASLt calls (more than 16 sequences, shapes the skinny kernels are not
  // built for, fp32 projections, materialized attention) runs eagerly: the library may record
  // memory-set nodes of its own into a capture, which are not safe to replay.
  const bool graphs = m->use_graphs && m->skinny && n <= kSkinnyRows && !m->materialized;
  if (timed) TRY(ensure_events(m, 3 + (graphs ? 0 : 2 * (size_t)steps * c.n_layers)));
  hipEvent_t* ev = m->events.data();
  if (timed) TRY_HIP(hipEventRecord(ev[0], s), "hipEventRecord");

  // ---- prefill: the packed prompt rows (attention over the padded batch [n, S]), then the
  //      pick after each prompt ----
  TRY_HIP(embed(m->x, m->tok_in, m->pos0, m->P(m->off.tok_emb), m->P(m->off.pos_emb), m->rowmap,
                rows, S, c.d_model, s),
          "embed");
  TRY(first_layernorm(m, rows));
  for (int l = 0; l < c.n_layers; ++l) TRY(block(m, l, n, S, rows, true, nullptr));
  TRY_HIP(gather_rows<float>(m->xl, m->x, m->lastrow, n, c.d_model, s), "gather_rows(last)");
  TRY(layernorm_h(m, m->xl, nullptr, nullptr, m->P(m->off.lnf_w), m->P(m->off.lnf_b), n));
  TRY(head(m, n));
  if (timed) TRY_HIP(hipEventRecord(ev[1], s), "hipEventRecord");
  if (logits) TRY(copy_logits(m, logits, n, 0));

  // ---- decode: feed token t-1 at its position, pick token t ----
  // With graphs, step 1 runs eagerly (it builds any missing hipBLASLt plan) and every later
  // step replays the captured step. Without graphs, timing brackets each attention launch.
  const bool attn_events = timed && !graphs;
  constexpr int kCheck = 16;
  int ran = 0;
  for (int t = 1; t <= steps; ++t) {
    if (early_exit && t % kCheck == 0) {
      const int slot = (t / kCheck) & 1;
      if (t >= 2 * kCheck) {  // the count copied kCheck steps ago
        TRY_HIP(hipEventSynchronize(m->ndone_ev[slot ^ 1]), "hipEventSynchronize");
        if (m->h_ndone[slot ^ 1] >= n) break;
      }
      TRY_HIP(hipMemcpyAsync(m->h_ndone + slot, m->ndone, sizeof(int), hipMemcpyDeviceToHost, s),
              "hipMemcpyAsync(stopped count)");
      TRY_HIP(hipEventRecord(m->ndone_ev[slot], s), "hipEventRecord");
    }
    if (graphs && t > 1) {
      hipGraphExec_t g = nullptr;
      TRY(step_graph(m, n, &g));
      TRY_HIP(hipGraphLaunch(g, s), "hipGraphLaunch");
    } else {
      TRY(decode_step(m, n, attn_events ? ev + 3 + 2 * (size_t)(t - 1) * c.n_layers : nullptr));
    }
    if (logits) TRY(copy_logits(m, logits, n, t));
    ran = t;
  }
  if (timed) TRY_HIP(hipEventRecord(ev[2], s), "hipEventRecord");

  tk.assign(outs, 0);
  mg.assign(outs, 0.f);
  TRY_HIP(hipMemcpyAsync(tk.data(), m->out_tok, outs * sizeof(int), hipMemcpyDeviceToHost, s),
          "hipMemcpyAsync(tokens)");
  TRY_HIP(hipMemcpyAsync(mg.data(), m->out_margin, outs * sizeof(float), hipMemcpyDeviceToHost,
                         s),
          "hipMemcpyAsync(margins)");
  TRY_HIP(hipStreamSynchronize(s), "hipStreamSynchronize");
  if (timed) {
    float ms = 0.f;
    timing->decode_steps = ran;
    TRY_HIP(hipEventElapsedTime(&ms, ev[0], ev[1]), "hipEventElapsedTime");
    timing->prefill_ms = ms;
    TRY_HIP(hipEventElapsedTime(&ms, ev[1], ev[2]), "hipEventElapsedTime");
    timing->decode_ms = logits ? NAN : ms;  // per-step host copies would be counted
    double attn = 0.0;
    for (size_t i = 0; attn_events && i < (size_t)ran * c.n_layers; ++i) {
      TRY_HIP(hipEventElapsedTime(&ms, ev[3 + 2 * i], ev[4 + 2 * i]), "hipEventElapsedTime");
      attn += ms;
    }
    timing->decode_attn_ms = attn_events ? (float)attn : -1.0f;
  }
  return DADGPT_OK;
}

// Prompts of n rows: 1 <= len <= stride and every token in the vocabulary.
int check_prompts(const dadgpt_gpt2* m, const char* fn, const int32_t* prompts,
                  const int32_t* prompt_lens, int n, int prompt_stride) {
  for (int b = 0; b < n; ++b) {
    const int len = prompt_lens[b];
    if (len < 1 || len > prompt_stride)
      return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: prompt %d has %d tokens (stride %d)", fn, b,
                  len, prompt_stride);
    for (int t = 0; t < len; ++t) {
      const int tok = prompts[(size_t)b * prompt_stride + t];
      if (tok < 0 || tok >= m->c.vocab_size)
        return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: token %d of prompt %d is %d (vocab %d)",
                    fn, t, b, tok, m->c.vocab_size);
    }
  }
  return DADGPT_OK;
}

}  // namespace

extern "C" {

int dadgpt_gpt2_truncate_prompt(const int32_t* prompt, int len, int max_len, int ctx_len,
                                int32_t* out, int32_t* out_len) {
  if (!prompt || !out || !out_len || len < 1 || ctx_len < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT,
                "dadgpt_gpt2_truncate_prompt: null buffer, len %d or ctx_len %d", len, ctx_len);
  // src/generate.cpp:97-110: the limit is capped at the context; a prompt that leaves no room
  // keeps its first token and its last max_len - 2 tokens
  const int eff = std::min(max_len, ctx_len);
  if (len >= eff && len > 1) {
    const int keep = std::max(eff - 2, 0);
    // (prompt and out may be the same buffer: the kept tail moves towards the front)
    out[0] = prompt[0];
    std::copy(prompt + (len - keep), prompt + len, out + 1);
    *out_len = 1 + keep;
  } else {
    if (out != prompt) std::copy(prompt, prompt + len, out);
    *out_len = len;
  }
  return DADGPT_OK;
}

int dadgpt_gpt2_generate(dadgpt_gpt2* m, const int32_t* prompts, const int32_t* prompt_lens,
                         int n, int prompt_stride, int new_tokens, int32_t* tokens,
                         float* margins, float* logits, dadgpt_gpt2_timing* timing) {
  const char* fn = "dadgpt_gpt2_generate";
  if (!m || !prompts || !prompt_lens || !tokens)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: null argument", fn);
  const auto& c = m->c;
  if (n < 1 || n > m->max_batch || new_tokens < 1)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: n=%d (max_batch %d), new_tokens=%d", fn, n,
                m->max_batch, new_tokens);
  TRY(check_prompts(m, fn, prompts, prompt_lens, n, prompt_stride));
  std::vector<int> limit(n);
  for (int b = 0; b < n; ++b) {
    if (prompt_lens[b] + new_tokens > c.ctx_len)
      return fail(DADGPT_ERR_INVALID_ARGUMENT,
                  "%s: prompt %d has %d tokens; prompt + %d new tokens must fit the context of "
                  "%d",
                  fn, b, prompt_lens[b], new_tokens, c.ctx_len);
    limit[b] = prompt_lens[b] + new_tokens;
  }
  std::vector<int> tk;
  std::vector<float> mg;
  TRY(generate_core(m, prompts, prompt_lens, n, prompt_stride, limit.data(), nullptr, new_tokens,
                    false, tk, mg, logits, timing));
  for (int b = 0; b < n; ++b)
    for (int t = 0; t < new_tokens; ++t) {
      tokens[(size_t)b * new_tokens + t] = tk[(size_t)t * n + b];
      if (margins) margins[(size_t)b * new_tokens + t] = mg[(size_t)t * n + b];
    }
  return DADGPT_OK;
}

int dadgpt_gpt2_generate_tokens(dadgpt_gpt2* m, const int32_t* prompts,
                                const int32_t* prompt_lens, int n, int prompt_stride,
                                int max_len, const int32_t* stop_tokens, int32_t* out,
                                int out_stride, int32_t* out_lens) {
  const char* fn = "dadgpt_gpt2_generate_tokens";
  if (!m || !prompts || !prompt_lens || !out || !out_lens)
    return fail(DADGPT_ERR_INVALID_ARGUMENT, "%s: null argument", fn);
  const auto& c = m->c;
  const int eff = std::min(max_len, c.ctx_len);
  if (n < 1 || n > m->max_batch || out_stride < std::max(eff, 1))
    return fail(DADGPT_ERR_INVALID_ARGUMENT,
                "%s: n=%d (max_batch %d), out_stride %d (needs %d)", fn, n, m->max_batch,
                out_stride, std::max(eff, 1));
  TRY(check_prompts(m, fn, prompts, prompt_lens, n, prompt_stride));
  // each row's (truncated) prompt goes to its output row; rows with room to generate form
  // the batch, in order
  std::vector<int> act, act_len, limit, stop;
  std::vector<int32_t> act_prompts((size_t)n * out_stride);
  for (int b = 0; b < n; ++b) {
    int32_t* row = out + (size_t)b * out_stride;
    int32_t len = 0;
    TRY(dadgpt_gpt2_truncate_prompt(prompts + (size_t)b * prompt_stride, prompt_lens[b],
                                    max_len, c.ctx_len, row, &len));
    out_lens[b] = len;
    if (len < eff) {
      std::copy(row, row + len, act_prompts.data() + act.size() * out_stride);
      act.push_back(b);
      act_len.push_back(len);
      limit.push_back(eff);
      stop.push_back(stop_tokens ? stop_tokens[b] : -1);
    }
  }
  if (act.empty()) return DADGPT_OK;
  const int na = (int)act.size();
  int max_new = 0;
  for (int j = 0; j < na; ++j) max_new = std::max(max_new, eff - act_len[j]);
  std::vector<int> tk;
  std::vector<float> mg;
  TRY(generate_core(m, act_prompts.data(), act_len.data(), na, out_stride, limit.data(),
                    stop.data(), max_new, true, tk, mg, nullptr, nullptr));
  // each row's picks up to and including its stop token, or up to its length limit
  for (int j = 0; j < na; ++j) {
    const int b = act[j];
    int32_t* row = out + (size_t)b * out_stride;
    int len = out_lens[b];
    for (int t = 0; len < eff; ++t) {
      const int tok = tk[(size_t)t * na + j];
      row[len++] = tok;
      if (tok == stop[j]) break;
    }
    out_lens[b] = len;
  }
  return DADGPT_OK;
}

}  // extern "C"
