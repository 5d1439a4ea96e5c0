// decode.hpp -- shared declarations of the Gemma-3 decode engine (device
// kernel arguments and the host-side encoder).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rt {

// Decode attention (k_attn): each wave of a workgroup walks kpw keys, so a
// workgroup (chunk) covers kpw*waves keys; the host sizes the chunk counts
// from the window (sliding-window layers) and from max_seq (global layers),
// and k_attn_combine merges the chunks.
constexpr int kAttnLocalKpw = 4, kAttnLocalWaves = 4;
constexpr int kAttnGlobalKpw = 8, kAttnGlobalWaves = 4;
// Dimensions per k_attn_combine workgroup (the rest of its 256 threads are
// chunk groups).
constexpr int kCombineDims = 32;
// Upper bound on the number of chunks a KV head is split into.
constexpr int kAttnMaxChunks = 4096;
// Step parameter block (device): ints [0, 16) (token, position), then the
// RoPE cos/sin table of the step's position for local layers at float offset
// kParamRopeLocal ([head_dim/2] cos, [head_dim/2] sin) and for global layers
// after it.
constexpr int kParamRopeLocal = 16;
// Batched verify (decode_step_batch): up to kMaxBatch tokens per call, each
// with its own parameter slot of kParamRopeLocal + 2*head_dim floats.
constexpr int kMaxBatch = 8;
inline int param_slot_floats(int head_dim) { return kParamRopeLocal + 2 * head_dim; }

struct DecodeShape {
  int hidden, ffn, n_q_heads, n_kv_heads, head_dim, n_layers, vocab;
  int nchunk_local, nchunk_global;
};

// Per-layer device pointers and constants (all device memory).
struct LayerArgs {
  const uint8_t *wq, *wk, *wv, *wo, *wgate, *wup, *wdown;  // Q4_K, rows=out
  const float *g_in, *g_post_attn, *g_pre_ffn, *g_post_ffn, *g_q, *g_k;
  float *kc, *vc;          // [max_seq, n_kv_heads*head_dim] f32
  const float *rope_cs;    // [head_dim] cos | sin of this step's angles (in the params block)
  int window;              // sliding window in keys, 0 = global layer
  int global;              // 1: global layer (RoPE theta_global; never windowed)
  int fmt[7];              // RT_LINEAR_* of q, k, v, o, gate, up, down (Q4K for the fused kernels)
  const int *ew[7];        // Q4_K projections: the GEMM's row exponents of the weight, [rows] (else null)
  float gu_bound;          // Q4_K gate and up: >= max_n |Wgate row n| |Wup row n| (else 0)
};
enum Proj { kProjQ, kProjK, kProjV, kProjO, kProjGate, kProjUp, kProjDown };

// Step-wide device buffers and constants.
struct DecodeArgs {
  const int *params;       // {token, position}
  const uint16_t *embed;   // [vocab, hidden] bf16 token embedding
  const uint16_t *lm_bf16; // BF16 lm_head [vocab, hidden]: the tied embedding unless set apart
  const uint8_t *lm_q4k;   // Q4_K lm_head [vocab][hidden/256] blocks (replaces lm_bf16), or null
  void *lm_stage;          // Q4_K head, several rows: staged activations (mb_stage_bytes(hidden))
  float *lm_part;          // and split-K partials (mb_head_part_bytes(vocab, hidden)), or null
  const float *g_final;
  float *hid, *x2, *q, *k, *v, *attn, *o, *h, *dn, *logits;
  float *xn, *u;           // normalised input of a split projection set [hidden]; up output [ffn]
  float *part_m, *part_l, *part_o;  // [n_q_heads, nchunk(, head_dim)]
  float embed_scale, eps, attn_scale;
  int vocab, n_q_heads, n_kv_heads, head_dim;
};

// Shapes of the fused single-token kernels (templated on the Gemma-3-4B and
// test widths) ...
bool decode_shape_supported(const DecodeShape &s, const char **why);
bool decode_rows_divisible(const DecodeShape &s, const char **why);
// ... and the wider set the rows kernels serve (every projection Q4_K).
bool decode_shape_generic(const DecodeShape &s, const char **why);
constexpr int kLmHeadMaxHidden = 4096;
// Allows the batched lm_head's LDS for `hidden` (once per process and width).
hipError_t prepare_lm_head_batch(int hidden);
hipError_t enqueue_decode_step(const DecodeShape &s, const DecodeArgs &a, const LayerArgs *layers, hipStream_t stream);
// Final residual, final norm and lm_head of the token whose last-layer x2
// and down-projection output sit in a.x2 / a.dn; logits into a.logits.
hipError_t enqueue_lm_head(const DecodeShape &s, const DecodeArgs &a, const LayerArgs &last, hipStream_t stream);
// M tokens at consecutive positions (params slots 0..M-1): the layer kernels
// of each token in turn, the final norm of each into xn[m][hidden], then one
// batched lm_head into logits_b[m][vocab].
hipError_t enqueue_decode_batch(const DecodeShape &s, const DecodeArgs &a, const LayerArgs *layers, int m,
                                float *xn, float *logits_b, hipStream_t stream);

// ---------------------------------------------------------------------------
// Prefill (prefill.hip): a prompt chunk of n tokens through every layer at
// once.  Device scratch for up to `cap` rows per chunk.
// ---------------------------------------------------------------------------
struct PrefillBuffers {
  int cap = 0;                      // rows the buffers hold
  int *tokens = nullptr;            // [cap]
  float *hid = nullptr, *x2 = nullptr, *xn = nullptr, *o = nullptr, *dn = nullptr;  // [cap][hidden]
  float *q = nullptr, *attn = nullptr;  // [cap][n_q_heads*head_dim]
  float *k = nullptr, *v = nullptr;     // [cap][n_kv_heads*head_dim]
  float *g = nullptr, *u = nullptr;     // [cap][ffn]
  float *nrm2 = nullptr;                // [cap]: |xn|^2 of each row of the gate|up input
  void *ws = nullptr;                   // Q4_K GEMM workspace
  void *mb_stage = nullptr;             // batched-GEMV staging (rows <= 8)
  float *mb_part = nullptr;             // batched-GEMV partial sums
  float *attn_ml = nullptr, *attn_o = nullptr;  // key-split attention partials, or null
  int attn_rows = 0;                             // rows the partials hold
};
// Key splits of the attention of a few rows: at most this many per KV head.
constexpr int kPfMaxSplits = 64;
inline size_t attn_part_floats(const DecodeShape &s, int rows, bool o) {
  return (size_t)kPfMaxSplits * rows * s.n_q_heads * (o ? s.head_dim : 2);
}
size_t prefill_gemm_workspace_bytes(const DecodeShape &s, int cap);
// Batched-GEMV staging and partial-sum bytes for every projection set.
size_t rows_mb_stage_bytes(const DecodeShape &s);
size_t rows_mb_part_bytes(const DecodeShape &s);
// Whether the batched GEMVs serve a layer with these projection formats
// (q, k, v, o, gate, up, down): Q4_K, Q6_K (rows of whole super-blocks),
// Q8_0 and BF16 (rows of whole 64-element chunks).
bool rows_mb_formats_ok(const DecodeShape &s, const int *fmt);

// n rows through every layer: rows p0 .. p0+n-1 (p0 from *p0_dev when that
// is set), token of row t at tokens[t*tok_stride], its cos/sin tables at
// cs + t*cs_stride (local | global).  Local layers attend keys
// [max(lo_fixed, pos + 1 - window), pos] of each row (window 0: no per-row
// window).  Projections run on the Q4_K GEMM, or with mb (n <= 8) on the
// batched GEMV.  Logits: none, the last row's into a.logits (a.x2 / a.dn are
// overwritten), or every row's final norm into xn_b and logits into logits_b.
struct RowsPlan {
  enum { kNone = 0, kLastRow = 1, kEveryRow = 2 };
  int n = 0, p0 = 0;
  const int *p0_dev = nullptr;
  const int *tokens = nullptr;
  int tok_stride = 1;
  const float *cs = nullptr;
  int cs_stride = 0;
  int lo_fixed = 0, window = 0;
  int max_pos = 0;  // bound on p0 + n (sizes the key split of a device-side p0)
  bool mb = false;
  int logits = kNone;
  float *xn_b = nullptr, *logits_b = nullptr;
  // Layers [layer_begin, n_layers); qkv_done: the first of them has its
  // q|k|v step done (normalised, rotated q in the buffers' q rows, K/V in
  // the cache) and starts at its attention; last_layer_kv_only: the last
  // layer stops after its q|k|v step (no logits then).
  int layer_begin = 0;
  bool qkv_done = false, last_layer_kv_only = false;
};
hipError_t enqueue_rows(const DecodeShape &s, const DecodeArgs &a, const LayerArgs *layers, const PrefillBuffers &b,
                        const RowsPlan &plan, hipStream_t stream);
// Batched lm_head of m <= 8 final-normed rows xn[m][hidden] into logits_b[m][vocab].
hipError_t enqueue_lm_head_batch(const DecodeShape &s, const DecodeArgs &a, const float *xn, float *logits_b, int m,
                                 hipStream_t stream);

}  // namespace rt
