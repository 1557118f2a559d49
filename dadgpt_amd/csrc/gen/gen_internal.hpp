// Internal interface of libdadgpt_gen: error reporting, the GEMM entry point and the launch
// functions of the model's elementwise kernels (gpt2_ops.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

struct dadgpt_blas;

namespace dadgpt::gen {

typedef __bf16 bf16;

// Records a printf-style message as this thread's last error and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// DADGPT_OK, or DADGPT_ERR_HIP with the HIP error's name recorded.
int check_hip(hipError_t e, const char* what);

// Row-major out[M,N] (fp32) = a[M,K] x b[K,N] (or x b[N,K]^T when trans_b); bf16 operands.
int gemm(dadgpt_blas* h, float* out, const bf16* a, const bf16* b, int M, int K, int N,
         bool trans_b, hipStream_t stream);

// fp32 row-major GEMM (blaslt.cpp): out[M,N] = op(a) op(b) + beta out over `count` matrices
// sa/sb/sc elements apart; op 'N', 'A' (a [K,M] transposed) or 'B' (b [N,K] transposed); the
// multiply precision is the process-wide one (dadgpt_set_matmul_precision).
int gemm_f32(dadgpt_blas* h, float* out, const float* a, const float* b, int M, int K, int N,
             char op, float beta, int count, long long sa, long long sb, long long sc,
             hipStream_t stream);

// Materialized attention (materialized_attn.cpp). Forward over BH heads whose q / k and v /
// out slices start stride_q / stride_kv / stride_o elements apart (rows of dh contiguous);
// probs [BH, S, S] is written. Decode: scores over each cache's max_len rows masked by
// lens[seq] (device), probs [n_seq * H, max_len] scratch, out [n_seq, H, dh].
int materialized_forward(dadgpt_blas* h, float* out, float* probs, const float* q,
                         const float* k, const float* v, int BH, int S, int dh, float scale,
                         long long stride_q, long long stride_kv, long long stride_o,
                         hipStream_t s);
int materialized_decode(dadgpt_blas* h, float* out, float* probs, const float* q,
                        const float* kcache, const float* vcache, const int* lens, int n_seq,
                        int H, int max_len, int dh, float scale, hipStream_t s);

// ---- kernels (gpt2_ops.hip); every launcher returns hipGetLastError() ----

// p[i] = bf16(std * N(0,1)) from a counter-based splitmix64/Box-Muller stream of `seed`.
hipError_t init_normal(bf16* p, size_t n, uint64_t seed, float stddev, hipStream_t s);
hipError_t fill(bf16* p, size_t n, float value, hipStream_t s);

// Prompt rows: row r of x [rows, d] fp32 = wte[tok[p]] + wpe[pos0[b] + s] for the padded
// position p = b*S + s = rowmap[r] (the prompts packed without padding), or p = r when rowmap
// is null (tok holds the padded [n, S] prompts).
hipError_t embed(float* x, const int* tok, const int* pos0, const bf16* wte, const bf16* wpe,
                 const int* rowmap, int rows, int S, int d, hipStream_t s);

// Per row (d <= 2048): if y, x[r] += sum_{s < splits} y[s][r] + bias (the residual add of a
// projection, y holding `splits` partial sums [splits][rows][d]); then, if w,
// out[r] = O(LayerNorm(x[r]) * w + b) with eps 1e-5 (two-pass mean and variance, fp32); O is
// bf16 or float (the precision of the projection that reads it). blocked (rows <= 16, d a
// multiple of 32): out in the skinny projections' K-blocked layout, element (r, c) at
// ((c/32)*16 + r)*32 + c%32.
template <typename O>
hipError_t residual_layernorm(float* x, const float* y, const bf16* bias, O* out,
                              const bf16* w, const bf16* b, int rows, int d, hipStream_t s,
                              int splits = 1, bool blocked = false);

// qkv [rows, 3d] fp32 (+ bias bqkv [3d] fp32), row r at padded position b*S + s = rowmap[r]
// (r itself when rowmap is null): q -> qh [n*H, S, dh]; k, v -> kh, vh [n*H, S, dh] when kh
// is not null; k, v of the rows s < nvalid[b] -> caches [n_cap, H, max_len, dh] at position
// pos0[b] + s. T is bf16 or float.
template <typename T>
hipError_t qkv_split(T* qh, T* kh, T* vh, T* kcache, T* vcache, const float* qkv,
                     const float* bqkv, const int* pos0, const int* nvalid, const int* rowmap,
                     int rows, int S, int H, int dh, int max_len, hipStream_t s);

// out [rows, d] (O: bf16 or float) <- heads [n*H, S, dh] (T), row r from padded position
// rowmap[r] (r when rowmap is null).
template <typename T, typename O>
hipError_t merge_heads(O* out, const T* heads, const int* rowmap, int rows, int S, int H, int dh,
                       hipStream_t s);

// out[i] = bf16(in[i]); out[i] = float(in[i]).
hipError_t to_bf16(bf16* out, const float* in, size_t count, hipStream_t s);
hipError_t to_f32(float* out, const bf16* in, size_t count, hipStream_t s);

// out[r, c] = O(gelu_tanh(y[r, c] + bias[c])), O bf16 or float.
template <typename O>
hipError_t bias_gelu(O* out, const float* y, const bf16* bias, int rows, int cols,
                     hipStream_t s);

// out[r] = in[idx[r]] (rows of d elements; T float or bf16).
template <typename T>
hipError_t gather_rows(T* out, const T* in, const int* idx, int rows, int d, hipStream_t s);

// Where each row of a generate call stops (src/generate.cpp:121-135): stop[b] is the row's
// stop token (-1: none), limit[b] the sequence length (prompt + generated) at which it ends;
// done[b] is set once the row has stopped, and ndone counts the stopped rows.
struct RowStop {
  const int* stop;
  const int* limit;
  int* done;
  int* ndone;
};

// Greedy pick per row of logits [n, V]: the first maximum (as std::max_element) and its
// margin over the runner-up, stored at step = pos[b] - (prompt_len[b] - 1) in tokens
// [step*n + b] and margins; then the decode state advances: tok[b] = pick, pos[b] += 1,
// cache_len[b] = pos[b] + 1, and the next decode step's input row is embedded:
// x[b] = wte[tok[b]] + wpe[pos[b]] (d floats; skipped where pos[b] >= ctx, past the last step).
// A row with no comparable logit (all NaN) picks column 0, as std::max_element does.
// A pick equal to the row's stop token, or one that brings the row to its length limit, stops
// the row (rs.done[b] = 1, rs.ndone += 1) after that advance. A stopped row emits nothing more
// and keeps its state: every later step re-feeds its last token at its last position (the
// step repeats, appending the same K/V to the same cache row), so it stays inside its context.
// Two launches: 32 blocks per row reduce slices into candidates (scratch of
// pick_scratch_floats(n, 0) floats), then one block per row merges them and embeds.
size_t pick_scratch_floats(int n, int parts);
hipError_t argmax_advance(int* tokens, float* margins, int* tok, int* pos, int* cache_len,
                          const int* prompt_len, RowStop rs, const float* logits,
                          float* scratch, int n, int V, float* x, const bf16* wte,
                          const bf16* wpe, int d, int ctx, hipStream_t s);
// The same pick from candidates already reduced per workgroup by the logits projection
// (kEpiStore with SkinnyArgs::cand): `parts` candidates per row in three planes of `rows`
// rows (values, columns, runner-up values). One launch.
hipError_t pick_advance(int* tokens, float* margins, int* tok, int* pos, int* cache_len,
                        const int* prompt_len, RowStop rs, const float* cand, int parts,
                        int rows, int n, int V, float* x, const bf16* wte, const bf16* wpe,
                        int d, int ctx, hipStream_t s);

// ---- skinny projections of the decode step (skinny.hip) ----

enum SkinnyPrologue { kProRows = 0, kProLn = 1, kProRowsBlocked = 2, kProRowsF32 = 3 };
constexpr int kSkinnyRows = 16;  // rows of the skinny path; kEpiGelu's g holds this many
enum SkinnyEpilogue { kEpiStore = 0, kEpiQkv = 1, kEpiGelu = 2, kEpiResidual = 3 };

struct SkinnyArgs {
  const bf16* wt;        // W^T [N][K]
  int M, N, K;           // rows (<= 16), columns, reduction length
  const bf16* act;       // kProRows: A [M][K]; kProRowsBlocked: A [K/32][16][32]
  const float* act32;    // kProRowsF32: A [M][K] fp32, rounded to bf16 as it is loaded
  const float* x;        // kProLn: A = LayerNorm(x [M][K]) * ln_w + ln_b
  const bf16* ln_w;
  const bf16* ln_b;
  float* out;            // kEpiStore: [M][N]
  float* cand;           // kEpiStore, optional: each workgroup's greedy candidate per row,
                         //   planes [3][16][skinny_store_parts(N)] (value, column, runner-up)
  const float* bias_f;   // kEpiQkv: fp32 bias [N]
  const bf16* bias;      // kEpiGelu, kEpiResidual: bias [N]
  bf16* g;               // kEpiGelu: gelu(A W + bias), K-blocked [N/32][16][32]
  float* x_out;          // kEpiResidual: residual stream [M][N], += A W + bias in place
  void* q;               // kEpiQkv: q [M, H, dh] and k, v into the caches
  void* kcache;          //   [.., H, max_len, dh] at row pos[m]; bf16, or fp32 if qkv_fp32
  void* vcache;
  const int* pos;
  int H, dh, max_len, qkv_fp32;
};

bool skinny_supported(int M, int K);  // M <= 16 and a K the kernels are built for
int skinny_store_parts(int N);        // workgroups of a kProRows/kEpiStore launch over N columns
hipError_t skinny_gemm(int prologue, int epilogue, const SkinnyArgs& args, hipStream_t s);
// out [cols][rows] = in [rows][cols]^T (bf16)
hipError_t transpose(bf16* out, const bf16* in, int rows, int cols, hipStream_t s);

// bqkv [3d] fp32 <- (bq, bk, bv) bf16.
hipError_t pack_bias(float* bqkv, const bf16* bq, const bf16* bk, const bf16* bv, int d,
                     hipStream_t s);

}  // namespace dadgpt::gen
