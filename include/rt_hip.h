/*
 * rt_hip.h -- C ABI of librt_hip.so, the MI355X (gfx950) implementation of
 * rich-triplet's Q4_K / BF16 decode hot path.
 *
 * Conventions
 *   - Every entry point returns rt_status (0 = RT_OK); on failure
 *     rt_last_error() returns a message for the calling thread.  Nothing
 *     aborts the process: the reference panics (assert_eq!/expect) on the same
 *     conditions, callers that want that behaviour check the status.
 *   - "dev" pointers are HIP device pointers (or host-pinned memory mapped for
 *     the device); "host" pointers are ordinary host memory and are copied.
 *   - `stream` is a hipStream_t or NULL for the default stream.  Device-pointer
 *     calls are asynchronous on that stream; host-pointer calls are
 *     synchronous, like the reference's commit()+waitUntilCompleted().
 *   - Q4_K weights are the GGUF super-block bytes, uploaded verbatim: 144 bytes
 *     per 256 elements, row-major [rows=out_features, cols=in_features], with
 *     cols a multiple of 256 (autograd2.rs:1035-1042, gguf_loader.rs:360-381).
 *   - Device buffers must be 16-byte aligned (hipMalloc guarantees 256).
 *
 * Reference paths are relative to the rich-triplet checkout (src/...).
 */
#ifndef RT_HIP_H
#define RT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t rt_status;
#define RT_OK 0
#define RT_EINVAL 1   /* bad shape, null pointer, misalignment, out-of-range token/position */
#define RT_EHIP 2     /* HIP runtime error (message carries hipGetErrorString) */
#define RT_ENOMEM 3   /* device allocation failed */
#define RT_ESTATE 4   /* call out of order (e.g. decode before weights are set) */

/* Message for the last failed call on this thread ("" if none). */
const char *rt_last_error(void);
/* ABI version, bumped on any signature change. */
int32_t rt_abi_version(void);

/* ---------------------------------------------------------------------------
 * Q4_K dequantisation (bit-exact with Q4KMat::dequantize_row_into,
 * autograd2.rs:1326-1366, and gguf_loader::decode_q4k_to_f32,
 * gguf_loader.rs:551-621).  out holds n_blocks*256 values.
 * ------------------------------------------------------------------------- */
rt_status rt_q4k_dequant_f32(const void *blocks_dev, size_t n_blocks, float *out_dev, void *stream);
/* Same values rounded to bf16 (RNE, MatBf16::f32_to_bf16 rule autograd2.rs:709-719). */
rt_status rt_q4k_dequant_bf16(const void *blocks_dev, size_t n_blocks, uint16_t *out_dev, void *stream);

/* ---------------------------------------------------------------------------
 * GEMV, y[n] = W[n,k] . x[k], f32 in/out, f32 accumulation.
 * rt_q4k_gemv replaces the GPU kernel gemv_q4k_t (metal_decode.rs:368-425,
 * metal_ops.rs:281-339) and the CPU Q4KMat::gemv_mt (autograd2.rs:1953-2035).
 * rt_bf16_gemv replaces gemv_bf16_t (metal_decode.rs:430-454) and
 * MatBf16::gemv_mt (autograd2.rs:954-1000).
 * ------------------------------------------------------------------------- */
rt_status rt_q4k_gemv(const void *w_dev, const float *x_dev, float *y_dev, int64_t n, int64_t k, void *stream);
rt_status rt_bf16_gemv(const uint16_t *w_dev, const float *x_dev, float *y_dev, int64_t n, int64_t k,
                       void *stream);
/* y_i = W_i . x for count <= 4 Q4_K matrices sharing x, in one launch: the
 * q, k, v (or gate, up) GEMVs the reference dispatches one by one
 * (metal_decode.rs:1948-1954, 2001-2004).  Host arrays of device pointers and
 * row counts; each as rt_q4k_gemv requires. */
rt_status rt_q4k_gemv_multi(const void *const *w_dev, float *const *y_dev, const int64_t *n, int32_t count,
                            const float *x_dev, int64_t k, void *stream);

/* ---------------------------------------------------------------------------
 * Host-pointer drop-ins for the reference's per-call GPU API
 * (metal_ops.rs:799-860 metal_gemv_q4k_t, 887-946 metal_gemv_bf16_t).
 * Weights are uploaded once and cached by (host pointer, byte length), as the
 * reference caches its MTLBuffers (metal_ops.rs:811-815); a caller that frees
 * or rewrites a weight buffer must call rt_weight_cache_clear().
 * a is [1, k] (the reference's Mat with rows == 1); out receives `rows` floats.
 * ------------------------------------------------------------------------- */
rt_status rt_gemv_q4k_t(const float *a_host, size_t k, const uint8_t *blocks_host, size_t rows, float *out_host);
rt_status rt_gemv_bf16_t(const float *a_host, size_t k, const uint16_t *w_host, size_t rows, float *out_host);
rt_status rt_weight_cache_clear(void);

/* ---------------------------------------------------------------------------
 * Q4_K GEMM, C[m,n] = A[m,k] . W[n,k]^T, f32 out (row-major), on the matrix
 * cores.  Replaces Q4KMat::matmul_q4k_t / matmul_q4k_t_exact
 * (autograd2.rs:1437-1625), reached from QLinear::forward (qlinear.rs:82-111)
 * and Linear2::fused_linear (nn2.rs:317-375), and the FLUX GPU GEMM
 * flux_dequant_q4k + flux_gemm_bt (metal_flux.rs:108-190, gemm_into 809-835).
 * Products use f16 operands (weights dequantised once, rounded to f16; each
 * A row and W row carries a power-of-two scale so f16 cannot overflow) with
 * f32 accumulation: ~2e-4 rel-L2 from the f32 CPU result, where bf16-rounded
 * weights (the reference's GPU path) give ~1.6e-3.
 * A is bf16 bits (rt_q4k_gemm_bf16) or f32 (rt_q4k_gemm_f32), row-major
 * [m,k]; every row of A must start 16-byte aligned (k % 256 == 0 ensures it).
 * The library keeps a workspace of about m*k*2 bytes per (host thread,
 * device, stream), shared with rt_linear_gemm_f32 and rt_q4k_gemv_batch on
 * that stream.  It grows on demand, but not while the stream is being
 * captured: a captured call that would need more returns RT_ESTATE, so make
 * the same call once outside capture first.  Outgrown buffers stay
 * allocated (a graph captured earlier may still read them) until
 * rt_gemm_workspace_release.  Cost per stream: the largest request made on
 * it (e.g. m=512, n=k=2560 Q4_K GEMM: A as f16, 2.6 MB, plus the row scales
 * and split-K partials), grown by at least doubling, plus every buffer it
 * outgrew: at most about 2x the largest request in all.
 * ------------------------------------------------------------------------- */
rt_status rt_q4k_gemm_bf16(const uint16_t *a_dev, const void *w_dev, float *c_dev, int64_t m, int64_t n, int64_t k,
                           void *stream);
rt_status rt_q4k_gemm_f32(const float *a_dev, const void *w_dev, float *c_dev, int64_t m, int64_t n, int64_t k,
                          void *stream);
/* Frees the calling host thread's workspace for `stream` on the current
 * device (no counterpart in the reference, whose Metal buffers live as long
 * as its context).  Synchronises `stream` first; RT_ESTATE while the stream
 * is being captured.  A graph captured over calls on that stream must not be
 * replayed afterwards (it reads the freed buffers).  The next call on the
 * stream allocates again. */
rt_status rt_gemm_workspace_release(void *stream);
/* Bytes the calling thread's workspace for `stream` holds on the current
 * device, outgrown buffers included (0 when none). */
size_t rt_gemm_workspace_held(void *stream);
/* Weight formats of a linear layer on the device. */
#define RT_LINEAR_Q4K 1    /* 144-byte Q4_K blocks as in the file */
#define RT_LINEAR_BF16 2   /* bf16 [rows][cols] */
#define RT_LINEAR_F32 3    /* f32 [rows][cols] */
#define RT_LINEAR_Q6K 4    /* planar Q6_K (rt_q6k_repack) */
#define RT_LINEAR_Q8_0 5   /* planar Q8_0 (rt_q8_0_repack) */

/* ---------------------------------------------------------------------------
 * Q6_K and Q8_0 weights kept packed on the device.  No counterpart in the
 * reference, which widens both to f32 and then BF16 at load
 * (load_linear_from_gguf, transformer4.rs:1233-1242; decode_q6k_to_f32,
 * gguf_loader.rs:482-549; decode_q8_0_to_f32, 628-650) and runs its BF16
 * GEMV on them.  The device layout is planar (each block field in its own
 * plane, so every load is aligned), the same size as the GGUF tensor:
 *   Q6_K (n_blocks 256-element blocks): ql [n][128] | qh [n][64] |
 *        int8 scales [n][16] | f16 d [n]
 *   Q8_0 (n_blocks 32-element blocks):  int8 q [n][32] | f16 d [n]
 * Matrices are row-major [rows][k] in block order, as in the file.
 * ------------------------------------------------------------------------- */
/* GGUF block bytes (host) -> planar layout (host); n_blocks*210 / *34 bytes. */
/* Measurement floors (no counterpart in the reference).  rt_stream_read
 * reads `bytes` of device memory with 16-byte loads and discards them, on
 * `stream`; `sink` is a device word the kernel writes only on an impossible
 * checksum.  rt_stream_read_cfg picks the access pattern (kind 0: strided
 * over all threads with the next batch of loads in flight; kind 1: one
 * contiguous slice per workgroup; kinds 2 and 3: the same with nontemporal
 * loads) and the grid (0: by size).  bench.py times
 * the fastest of several on the same bytes as a GEMV to give that GEMV's
 * fraction of a plain streaming read.  rt_empty_launch launches a kernel with
 * no body: in a graph, the cost of one dependent launch. */
rt_status rt_stream_read(const void *buf, size_t bytes, void *sink, void *stream);
rt_status rt_stream_read_cfg(const void *buf, size_t bytes, void *sink, void *stream, int kind, int grid);
rt_status rt_empty_launch(int grid, int threads, void *stream);

/* Per-wave timeline of the decode step's launches (no counterpart in the
 * reference; the tracing of the survey's auxiliary subsystems).  Only a
 * library built with RT_TRACE=1 (`make -C rich-triplet_amd trace`, which writes
 * librt_hip_trace.so) records it; librt_hip.so returns RT_ESTATE.  The record
 * is uint64 [kernels][slots][4]: per wave (slot = workgroup * waves + wave) the
 * 100 MHz real-time counter at entry, once the activation staging is done,
 * once every load of the wave has landed (an explicit wait the traced build
 * adds), and at exit.  Kernels: 0 q|k|v, 1 attention, 2 chunk merge, 3 o
 * projection, 4 gate|up, 5 down projection, 6 lm_head; each launch overwrites
 * its kernel's slots, so after a step they hold the last layer's launches.
 * With host_dst NULL only *kernels and *slots are set; otherwise bytes must be
 * kernels * slots * 32. */
rt_status rt_trace_read(void *host_dst, size_t bytes, int32_t *kernels, int32_t *slots);

/* y = gelu_tanh(x) (autograd2.rs:3082-3091), n floats, device pointers: the
 * activation exactly as the decode step and prefill kernels compute it. */
rt_status rt_gelu_tanh(const float *x, float *y, size_t n, void *stream);

rt_status rt_q6k_repack(const void *gguf_blocks, size_t n_blocks, void *dst);
rt_status rt_q8_0_repack(const void *gguf_blocks, size_t n_blocks, void *dst);
/* Device dequantisation, bit-exact with decode_q6k_to_f32 / decode_q8_0_to_f32. */
rt_status rt_q6k_dequant_f32(const void *w, size_t n_blocks, float *out, void *stream);
rt_status rt_q8_0_dequant_f32(const void *w, size_t n_elem, float *out, void *stream);
/* y[n] = W[n,k] . x[k] on planar Q6_K (k % 256 == 0) / Q8_0 (k % 32 == 0)
 * weights; device pointers, w and x 16-byte aligned. */
rt_status rt_q6k_gemv(const void *w, const float *x, float *y, int64_t n, int64_t k, void *stream);
rt_status rt_q8_0_gemv(const void *w, const float *x, float *y, int64_t n, int64_t k, void *stream);
/* c[m][n] = a[m][k] . W[n][k] for a weight in any RT_LINEAR_* format (Q6_K
 * and Q8_0 planar): the matmul of QLinear::forward (qlinear.rs:82-111).
 * Replaces matmul_q4k_t_exact for RT_LINEAR_Q4K (as rt_q4k_gemm_f32),
 * MatBf16::matmul_by_t (autograd2.rs:757-852) for BF16 and for the Q6_K /
 * Q8_0 weights the reference widens to BF16, and Mat::matmul_bt
 * (autograd2.rs:378-429) for RT_LINEAR_F32.  Non-Q4_K rows are widened to f16
 * with a power-of-two scale per row, A likewise, f32 accumulation on the
 * matrix cores (f32 weights: ~2e-4 rel-L2 from the f32 product); F32 and
 * BF16 weights with m <= 8, or k not a multiple of 64, run a GEMV that streams
 * them once per 8 rows in f32.  k % 256 == 0 (Q4_K, Q6_K), k % 64 == 0
 * (Q8_0, and BF16 with m > 8), k % 8 == 0 (BF16, m <= 8), k % 4 == 0 (F32);
 * device pointers, a and w 16-byte aligned.  Uses the
 * per-(thread, device, stream) workspace of rt_q4k_gemm_f32, about
 * (m + n) * k * 2 bytes (none for the f32 GEMV). */
rt_status rt_linear_gemm_f32(int32_t fmt, const void *w, const float *a, float *c, int64_t m, int64_t n, int64_t k,
                             void *stream);
/* QLinear::forward (qlinear.rs:82-111): out[m][n] = x[m][k] . W[n][k], then
 * add_bias_rows (qlinear.rs:49-60), out[r][j] += bias[j] in f32, when bias
 * (n floats, device) is not NULL.  Formats and constraints as
 * rt_linear_gemm_f32. */
rt_status rt_qlinear_forward(int32_t fmt, const void *w, const float *bias, const float *x, float *out, int64_t m,
                             int64_t n, int64_t k, void *stream);
/* Host drop-in for QLinear::forward (qlinear.rs:82-111) on the formats a
 * QLinear holds: RT_LINEAR_Q4K (w_bytes = n*(k/256)*144), RT_LINEAR_BF16
 * (n*k*2) or RT_LINEAR_F32 (n*k*4).  The weight is uploaded once and cached
 * by (host pointer, bytes) like rt_gemv_q4k_t's (rt_weight_cache_clear drops
 * it); x [m, k], bias [n] (or NULL) and out [m, n] are host f32; synchronous. */
rt_status rt_qlinear_forward_host(int32_t fmt, const void *w, size_t w_bytes, const float *bias, const float *x,
                                  float *out, int64_t m, int64_t n, int64_t k);

/* gemv_q4k_t_batch (metal_decode.rs:459-521): c[m][n] = a[m][k] . W[n][k]
 * for m = 1..8 rows (the speculative verify batch), reading the weights once
 * for all rows (int8 matrix cores); device pointers, a and w 16-byte
 * aligned, k % 256 == 0.  Uses the per-(thread, device, stream) workspace of
 * rt_q4k_gemm_f32 (see there for graph capture). */
rt_status rt_q4k_gemv_batch(const void *w, const float *a, float *c, int64_t m, int64_t n, int64_t k, void *stream);

/* The same batched GEMV for the other projection formats a decode layer can
 * hold: gemv_bf16_t_batch (metal_decode.rs:527-558) for RT_LINEAR_BF16, and
 * RT_LINEAR_Q6K / RT_LINEAR_Q8_0 kept packed (planar layout, rt_q6k_repack /
 * rt_q8_0_repack) where the reference widens them to BF16 first.  Reads the
 * weights once for all m = 1..8 rows; device pointers, a and w 16-byte
 * aligned; k % 256 == 0 for Q6_K, k % 64 == 0 otherwise; fmt RT_LINEAR_Q4K
 * is rt_q4k_gemv_batch.  Workspace as rt_q4k_gemv_batch. */
rt_status rt_linear_gemv_batch(int32_t fmt, const void *w, const float *a, float *c, int64_t m, int64_t n, int64_t k,
                               void *stream);

/* rt_q4k_gemv_batch that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as rt_q4k_gemv_batch; its
 * workspace is a fixed per-GPU device array of rt_noalloc_scratch_bytes()
 * (8 MiB), which bounds n and k: the staged rows, (k/64)*1152 bytes rounded
 * up to 256, plus the split-K partials, (k/256)*32*n bytes for
 * 256 < k < 8192 ((k/1024)*32*n for k >= 8192 divisible by 1024), must fit,
 * else RT_EINVAL.  Every call on one GPU
 * shares that array: calls that overlap on one GPU (two streams, two host
 * threads) race and must be serialised by the caller. */
rt_status rt_q4k_gemv_batch_noalloc(const void *w, const float *a, float *c, int64_t m, int64_t n, int64_t k,
                                    void *stream);
size_t rt_noalloc_scratch_bytes(void);

/* Host drop-in for Q4KMat::matmul_q4k_t_exact (autograd2.rs:1490-1625):
 * a is [m, k] f32, out receives [m, rows] f32.  m == 1 takes the GEMV path, as
 * matmul_q4k_t does (autograd2.rs:1440-1443).  Weights are cached like
 * rt_gemv_q4k_t's. */
rt_status rt_matmul_q4k_t(const float *a_host, size_t m, size_t k, const uint8_t *blocks_host, size_t rows,
                          float *out_host);

/* ---------------------------------------------------------------------------
 * Gemma-3 decode engine -- replaces MetalDecodeContext (metal_decode.rs:754-829).
 * One step = embedding lookup, n_layers Gemma-3 blocks (4-norm, GQA with
 * sliding-window / global layers, NeoX RoPE, gated GELU-tanh) and the BF16
 * tied lm_head, executed as one hipGraph on the context's stream.  The KV
 * cache is f32 and device-resident, [max_seq, n_kv_heads*head_dim] per layer.
 * Semantics follow the reference CPU path (transformer4.rs:1900-1964,
 * 2358-2385); the GPU path of the reference keeps an f16 cache capped at
 * 2048 rows (metal_decode.rs:1186), this engine does not.
 * ------------------------------------------------------------------------- */
typedef struct {
    /* Config4 fields (transformer4.rs:112-131). */
    int32_t hidden, ffn, n_q_heads, n_kv_heads, head_dim, n_layers, vocab;
    int32_t sliding_window;   /* keys attended by local layers, 0 = none */
    int32_t global_every;     /* layer i is global iff i % global_every == global_every-1 (6 for Gemma 3) */
    int32_t max_seq;          /* KV rows allocated per layer */
    float rope_theta_local, rope_theta_global, rope_fs_local, rope_fs_global;
    float eps, attn_scale;    /* rms_norm_eps; 1/sqrt(query_pre_attn_scalar) */
} rt_gemma3_config;

/* One layer's weights: Q4_K blocks (rows = out features) and RMSNorm gammas
 * as used in x/rms*(1+gamma).  LayerWeightBuffers, metal_decode.rs:720-748. */
typedef struct {
    const void *q, *k, *v, *o, *gate, *up, *down;
    const float *in_norm, *post_attn_norm, *pre_ffn_norm, *post_ffn_norm, *q_norm, *k_norm;
} rt_gemma3_layer;

typedef struct rt_decode rt_decode;

/* MetalDecodeContext::new (metal_decode.rs:971-1254) minus the weight upload,
 * which the two calls below perform.  Supported shapes: hidden 512|2560,
 * n_q_heads*head_dim 512|2048, ffn 1024|10240, head_dim 128|256, group 1|2|4. */
rt_status rt_decode_create(const rt_gemma3_config *cfg, rt_decode **out);
rt_status rt_decode_destroy(rt_decode *d);
/* device_ptrs = 0: host pointers, copied (Q4_K bytes verbatim, 144-B blocks
 * stay packed; upload_linear_detect_type, metal_decode.rs:1259-1277).
 * device_ptrs = 1: device pointers, borrowed; the caller keeps them alive
 * and unchanged until the layer is set again (the prefill GEMM's per-row
 * exponents of each Q4_K weight are computed here, once: 4 bytes per row). */
rt_status rt_decode_set_layer(rt_decode *d, int32_t layer, const rt_gemma3_layer *w, int32_t device_ptrs);
/* Same, with the format of each projection in the order q, k, v, o, gate,
 * up, down: RT_LINEAR_Q4K, RT_LINEAR_Q6K, RT_LINEAR_Q8_0 or RT_LINEAR_BF16
 * (the device layouts of rt_gguf_load_linear_ex).  The reference's context
 * takes Q4_K or BF16 per projection (upload_linear_detect_type,
 * metal_decode.rs:1259-1277, with Q6_K/Q8_0 widened to BF16 at load); here
 * Q6_K and Q8_0 also run natively, in decode, batch and prefill.
 * Failure (a null or misaligned pointer, an unsupported format, a failed
 * upload) is checked before anything is uploaded, and the new binding
 * replaces the old one only when it is whole; but a failed call still
 * leaves the layer UNSET (its previous binding released, captured graphs
 * dropped) and rt_decode_step answers RT_ESTATE until the layer is set
 * again.  A caller that frees borrowed weights and then re-binds therefore
 * never runs over freed memory, whichever way the re-bind ends.
 * rt_decode_set_embed behaves the same way for the embedding. */
rt_status rt_decode_set_layer_formats(rt_decode *d, int32_t layer, const rt_gemma3_layer *w,
                                      const int32_t *formats, int32_t device_ptrs);
/* BF16 [vocab, hidden] embedding, also the tied lm_head (1097-1105), and the final norm gamma. */
rt_status rt_decode_set_embed(rt_decode *d, const uint16_t *embed, const float *final_norm, int32_t device_ptrs);
/* An lm_head apart from the embedding (metal_decode.rs:1079-1107):
 * RT_LINEAR_Q4K, Q4_K blocks [vocab][hidden/256] (hidden % 256 == 0): the
 * model's own Q4_K head, or the BF16 one requantised by rt_q4k_quantize_bf16
 * (the reference's q4k-lm-head feature, 1082-1094); every logit then comes
 * from the Q4_K GEMV (one token) or the batched Q4_K GEMV (verify, prefill)
 * of the final-normed hidden state, as dispatch_gemv / dispatch_gemv_q4k_batch
 * do (2053-2063, 2164-2172), reading 0.28x the BF16 head's bytes.
 * RT_LINEAR_BF16: an untied BF16 head [vocab, hidden].  w = NULL (fmt
 * ignored) restores the tied embedding, the default.  device_ptrs as for
 * rt_decode_set_layer.  A failed call leaves the tied embedding as the
 * head. */
rt_status rt_decode_set_lm_head(rt_decode *d, int32_t fmt, const void *w, int32_t device_ptrs);
/* sync_kv_from_cpu (metal_decode.rs:1366-1396) for one layer: seq_len rows of K and V. */
rt_status rt_decode_sync_kv(rt_decode *d, int32_t layer, const float *k, const float *v, int32_t seq_len,
                            int32_t device_ptrs);
/* decode_step (metal_decode.rs:2028-2074): appends K/V at row `position`
 * and writes vocab logits to logits_host (may be NULL); synchronous. */
rt_status rt_decode_step(rt_decode *d, int32_t token, int32_t position, float *logits_host);
/* Same step, only enqueued on the context stream; logits stay on the device. */
rt_status rt_decode_step_async(rt_decode *d, int32_t token, int32_t position);
/* decode_step_batch (metal_decode.rs:2079-2179): m (1..8) tokens at positions
 * start_position .. start_position+m-1, as used by speculative verify.  Each
 * token attends to the K/V of the tokens before it in the batch; logits_host
 * (may be NULL) receives m x vocab floats, row i for token i.  The lm_head
 * reads the embedding once for all m tokens. */
rt_status rt_decode_step_batch(rt_decode *d, const int32_t *tokens, int32_t m, int32_t start_position,
                               float *logits_host);
rt_status rt_decode_step_batch_async(rt_decode *d, const int32_t *tokens, int32_t m, int32_t start_position);
/* Device buffer of the last batch's logits, [8][vocab]. */
rt_status rt_decode_logits_batch(rt_decode *d, float **logits_dev);
/* Prefill on the GPU: replaces the CPU prefill of generate_cached_streaming
 * (transformer4.rs:2103-2139, Gemma3Block::forward_cached over the prompt)
 * plus sync_kv_from_cpu (metal_decode.rs:1366-1396).  Runs tokens[0..n) at
 * positions start_position .. start_position+n-1 through every layer, fills
 * those KV rows and leaves the last token's logits in the logits buffer
 * (copied to logits_host when not NULL); synchronous.  Window rule of the
 * sliding-window layers:
 *   RT_PREFILL_REFERENCE  forward_cached's prefill (gqa_attention_cached,
 *       transformer4.rs:2882-2940): the window is anchored at the end of the
 *       prompt, so row r sees keys [max(0, n - window), r] and rows before
 *       n - window get a zero attention output; start_position must be 0.
 *   RT_PREFILL_SLIDING    each row r sees keys [r + 1 - window, r], the rule
 *       of the uncached forward (gqa_attention_windowed, 2661-2700) and of
 *       every decode step, so a prefill equals n decode steps. */
#define RT_PREFILL_REFERENCE 0
#define RT_PREFILL_SLIDING 1
rt_status rt_decode_prefill(rt_decode *d, const int32_t *tokens, int32_t n, int32_t start_position, int32_t mode,
                            float *logits_host);
/* Rows per prefill chunk (default 4096): a prompt is processed in chunks of
 * at most this many tokens, bounding the prefill scratch (about 180 KB per
 * row at the Gemma-3-4B shape).  No counterpart in the reference. */
rt_status rt_decode_set_prefill_chunk(rt_decode *d, int32_t rows);
rt_status rt_decode_synchronize(rt_decode *d);
/* Use the captured hipGraph (default) or launch the kernels one by one. */
rt_status rt_decode_set_graph(rt_decode *d, int32_t enabled);
/* print_metal_memory (metal_decode.rs:1285-1354): device bytes of a context by
 * what they hold.  weights counts uploads and device-pointer bindings alike
 * (projections and their GEMM row exponents, norms, embedding / tied
 * lm_head); prefill is the chunk
 * scratch, 0 until the first rt_decode_prefill. */
typedef struct {
  uint64_t weights, kv_cache, activation, batch, prefill, total;
} rt_decode_memory_info;
rt_status rt_decode_memory(const rt_decode *d, rt_decode_memory_info *out);
/* How rt_decode_step_batch runs (no counterpart in the reference, whose
 * verify batch always runs its batched GEMVs): *batched = 1 when every bound
 * layer's projections are served by the batched GEMVs (Q4_K, Q6_K, Q8_0,
 * BF16) and the M tokens go through each layer together, reading each
 * weight once; 0 when they run as M single-token passes. */
rt_status rt_decode_verify_batched(const rt_decode *d, int32_t *batched);
/* Device buffers of the context, for inspection. */
rt_status rt_decode_logits(rt_decode *d, float **logits_dev);
rt_status rt_decode_kv(rt_decode *d, int32_t layer, float **k_dev, float **v_dev);
rt_status rt_decode_hidden(rt_decode *d, float **x2_dev, float **dn_dev);
rt_status rt_decode_get_stream(rt_decode *d, void **stream);

#ifdef __cplusplus
}
#endif
#endif /* RT_HIP_H */
