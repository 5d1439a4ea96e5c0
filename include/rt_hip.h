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

#ifdef __cplusplus
}
#endif
#endif /* RT_HIP_H */
