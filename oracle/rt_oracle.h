/*
 * rt_oracle.h -- CPU restatement of rich-triplet's portable (x86, non-BLAS)
 * Q4_K / BF16 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * product path is compared against.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product library never links it.
 *
 * Every function cites the reference file:line it restates.  Paths are
 * relative to the reference checkout (src/...).  Arithmetic follows the
 * reference's scalar f32 order; the file is compiled with -ffp-contract=off so
 * `a*b - c` stays two roundings, as in Rust.
 */
#ifndef RT_ORACLE_H
#define RT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ------------------------------------------------ */
float    orc_f16_to_f32(uint16_t bits);            /* autograd2.rs:1048-1070, gguf_loader.rs:947-976 */
uint16_t orc_f32_to_f16_rne(float v);              /* synthetic-data writer only (own RNE, not the ref's truncating one) */
float    orc_bf16_to_f32(uint16_t bits);           /* autograd2.rs:700-703 */
uint16_t orc_f32_to_bf16(float v);                 /* autograd2.rs:709-719 */

/* ---- Q4_K block format ------------------------------------------------- */
void orc_q4k_scale_min(const uint8_t *sc, int j, float *sv, float *mv);     /* autograd2.rs:1075-1085 */
void orc_q4k_pack_scales(const uint8_t sv[8], const uint8_t mv[8], uint8_t out[12]); /* autograd2.rs:1119-1132 */
void orc_q4k_dequant_row(const uint8_t *blocks, size_t cols, size_t row, float *out); /* autograd2.rs:1326-1366 */
void orc_q4k_dequant_gguf(const uint8_t *bytes, size_t n_elem, float *out); /* gguf_loader.rs:551-621 */

/* ---- GGUF tensor formats and Q4_K quantisation --------------------------- */
uint16_t orc_f32_to_f16_trunc(float v);            /* autograd2.rs:1090-1117 (Q4KMat::f32_to_f16: truncates) */
void orc_q4k_quantize_block(const float *x256, uint8_t out[144]);          /* autograd2.rs:1171-1245 */
void orc_q4k_quantize(const float *m, size_t rows, size_t cols, uint8_t *blocks); /* autograd2.rs:1138-1168 */
void orc_q4_0_dequant(const uint8_t *bytes, size_t n_elem, float *out);    /* gguf_loader.rs:425-480 */
void orc_q4_0_to_q4k(const uint8_t *bytes, size_t rows, size_t cols, uint8_t *blocks);
     /* gguf_loader.rs:282-357 + autograd2.rs:1291-1320 (Q4KMat::from_q4mat) + 2390-2414 */
void orc_q6k_dequant(const uint8_t *bytes, size_t n_elem, float *out);     /* gguf_loader.rs:482-549 */
void orc_q5k_dequant(const uint8_t *bytes, size_t n_elem, float *out);     /* gguf_loader.rs:664-743 */
void orc_q8_0_dequant(const uint8_t *bytes, size_t n_elem, float *out);    /* gguf_loader.rs:628-650 */

/* ---- GEMV -------------------------------------------------------------- */
float orc_q4k_dot_row(const uint8_t *blocks, size_t cols, size_t row, const float *a); /* autograd2.rs:1654-1701 */
void  orc_q4k_gemv_mt(const uint8_t *blocks, size_t rows, size_t cols,
                      const float *a, float *y, int hw_threads);                     /* autograd2.rs:1953-2035 */
void  orc_q4k_gemv_f64(const uint8_t *blocks, size_t rows, size_t cols,
                       const float *a, double *y);          /* fp64 twin: sum_k dequant(w)*a in double */
float orc_bf16_dot_row(const uint16_t *w, size_t cols, size_t row, const float *a); /* autograd2.rs:879-887 */
void  orc_bf16_gemv_mt(const uint16_t *w, size_t rows, size_t cols,
                       const float *a, float *y, int hw_threads);                    /* autograd2.rs:954-1000 */
void  orc_bf16_gemv_f64(const uint16_t *w, size_t rows, size_t cols, const float *a, double *y);

/* ---- GEMM (M>1): C[M,N] = A[M,K] * dequant(W[N,K])^T -------------------- */
void orc_q4k_matmul(const float *a, size_t m, const uint8_t *blocks, size_t n, size_t k,
                    float *c, int hw_threads);              /* autograd2.rs:1437-1457 (scalar order) */
void orc_q4k_matmul_f64(const float *a, size_t m, const uint8_t *blocks, size_t n, size_t k,
                        double *c, int hw_threads);

/* ---- decode-step math ---------------------------------------------------- */
void  orc_rms_norm_gemma3(const float *x, const float *gamma, size_t d, float eps, float *out); /* autograd2.rs:3477-3496 */
void  orc_per_head_norm(const float *x, const float *gamma, size_t n_heads, size_t head_dim,
                        float eps, float *out);              /* transformer4.rs:2485-2508 */
void  orc_rope_neox(float *x, size_t n_heads, size_t head_dim, float theta, size_t pos,
                    float freq_scale);                        /* transformer4.rs:2742-2772 */
float orc_gelu_tanh(float x);                                 /* autograd2.rs:3082-3091 */
void  orc_gqa_attention_decode(const float *q, const float *k_cache, const float *v_cache,
                               size_t k_start, size_t k_end, size_t n_q_heads, size_t n_kv_heads,
                               size_t d_head, float scale, float *out); /* transformer4.rs:2806-2879 */

/* Gemma-3 shape (Config4, transformer4.rs:112-131). */
typedef struct {
    int32_t hidden, ffn, n_q_heads, n_kv_heads, head_dim, n_layers;
    int32_t vocab, sliding_window, global_every;   /* layer i is global iff i % global_every == global_every-1 */
    float   rope_theta_local, rope_theta_global, rope_fs_local, rope_fs_global, eps, attn_scale;
} orc_gemma3_cfg;

/* Per-layer weights (transformer4.rs Gemma3Block); all host pointers. */
typedef struct {
    const uint8_t *q, *k, *v, *o, *gate, *up, *down;          /* rows=out, cols=in, format fmt[i] */
    const float *in_norm, *post_attn_norm, *pre_ffn_norm, *post_ffn_norm, *q_norm, *k_norm;
    float *k_cache, *v_cache;                                  /* [max_seq, n_kv_heads*head_dim] f32 */
    int32_t fmt[7];  /* q, k, v, o, gate, up, down: 0 or 1 Q4_K, 2 BF16, 4 Q6_K (GGUF blocks), 5 Q8_0 (GGUF blocks) */
} orc_layer;

/* y = W x (rows x cols) for a projection of format fmt (as orc_layer.fmt):
 * Q4_K through dot_row; Q6_K / Q8_0 dequantised per row by decode_q6k_to_f32
 * / decode_q8_0_to_f32 and a sequential f32 dot; BF16 through its dot_row. */
void orc_proj_gemv(int fmt, const uint8_t *w, size_t rows, size_t cols, const float *x, float *y, int hw_threads);
/* C[m,n] = A[m,k] . W[n,k]^T for a projection of format fmt (as orc_layer.fmt);
 * a sequential f32 dot per output, as orc_q4k_matmul. */
void orc_proj_matmul(int fmt, const float *a, size_t m, const uint8_t *w, size_t n, size_t k, float *c,
                     int hw_threads);
/* QLinear::forward (qlinear.rs:82-111): orc_proj_matmul of fmt (3 = F32
 * weights, Mat::matmul_bt) plus add_bias_rows (qlinear.rs:49-60); bias may be
 * NULL (no bias). */
void orc_qlinear_forward(int fmt, const float *a, size_t m, const uint8_t *w, const float *bias, size_t n, size_t k,
                         float *c, int hw_threads);

/* One CPU decode step (transformer4.rs:2358-2385 with forward_cached 1900-1964).
 * Appends K/V at row `pos` of every layer's cache and writes vocab logits.
 * hidden_out (optional, may be NULL) receives the final hidden state before the
 * final norm. */
void orc_gemma3_decode_step(const orc_gemma3_cfg *cfg, const orc_layer *layers,
                            const uint16_t *embed_bf16, const float *final_norm,
                            uint32_t token, uint32_t pos, float *logits, float *hidden_out,
                            int hw_threads);

/* One layer (Gemma3Block::forward_cached, transformer4.rs:1954-1964), in place on x. */
void orc_gemma3_layer(const orc_gemma3_cfg *cfg, const orc_layer *L, int layer_idx,
                      float *x, uint32_t pos, int hw_threads);

/* Attention of T query rows (positions p0 .. p0+T-1) against the cache; row
 * r sees keys [max(lo_fixed, window ? r+1-window : 0), r] (transformer4.rs:
 * 2882-2940 with lo_fixed = k_start; 2661-2700 with window). */
void orc_gqa_attention_prefill(const float *q, const float *k_cache, const float *v_cache, size_t p0, size_t T,
                               size_t lo_fixed, size_t window, size_t n_q_heads, size_t n_kv_heads, size_t d_head,
                               float scale, float *out);

/* Prefill of T tokens at positions p0.. (mode 0: the reference's prefill
 * window rule, p0 = 0; mode 1: per-row sliding window); last row's logits. */
void orc_gemma3_prefill(const orc_gemma3_cfg *cfg, const orc_layer *layers, const uint16_t *embed_bf16,
                        const float *final_norm, const uint32_t *tokens, size_t T, size_t p0, int mode,
                        float *logits, int hw_threads);

/* ---- seeded synthetic data (counter-based splitmix64) -------------------- */
uint64_t orc_rng_u64(uint64_t seed, uint64_t i);
void orc_synth_normal_f32(uint64_t seed, size_t n, float mean, float std, float *out);
void orc_synth_bf16(uint64_t seed, size_t n, float std, uint16_t *out);
void orc_synth_q4k(uint64_t seed, size_t n_blocks, float d_std, uint8_t *out);

/* ---- timing helper for the CPU baseline ---------------------------------- */
int orc_hw_threads(void);

#ifdef __cplusplus
}
#endif
#endif
