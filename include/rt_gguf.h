/*
 * rt_gguf.h -- GGUF reader and weight loader of librt_hip.so: the on-disk
 * format that feeds the Q4_K decode path (host side, C ABI).
 *
 * Replaces the reference's GgufFile (src/gguf_loader.rs) and
 * load_linear_from_gguf (src/transformer4.rs:1177-1256).  Conventions are
 * those of rt_hip.h: rt_status return codes, messages via rt_last_error().
 * A handle is read-only after rt_gguf_open and may be shared between threads.
 */
#ifndef RT_GGUF_H
#define RT_GGUF_H

#include "rt_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type ids (GgufType, gguf_loader.rs:41-72). */
#define RT_GGUF_F32 0
#define RT_GGUF_F16 1
#define RT_GGUF_Q4_0 2
#define RT_GGUF_Q8_0 8
#define RT_GGUF_Q4_K 12
#define RT_GGUF_Q5_K 13
#define RT_GGUF_Q6_K 14
#define RT_GGUF_BF16 30

/* Metadata value types (GgufMetaValue, gguf_loader.rs:828-905). */
#define RT_GGUF_META_U8 0
#define RT_GGUF_META_I8 1
#define RT_GGUF_META_U16 2
#define RT_GGUF_META_I16 3
#define RT_GGUF_META_U32 4
#define RT_GGUF_META_I32 5
#define RT_GGUF_META_F32 6
#define RT_GGUF_META_BOOL 7
#define RT_GGUF_META_STR 8
#define RT_GGUF_META_ARRAY 9
#define RT_GGUF_META_U64 10
#define RT_GGUF_META_I64 11
#define RT_GGUF_META_F64 12

typedef struct rt_gguf rt_gguf;

/* One tensor directory entry (GgufTensorInfo, gguf_loader.rs:139-154). */
typedef struct {
    const char *name;     /* owned by the handle, valid until rt_gguf_close */
    int32_t n_dims;       /* at most 4 */
    int64_t dims[4];      /* GGUF order: dims[0] varies fastest (in_features of a weight) */
    int32_t type;         /* ggml type id */
    uint64_t offset;      /* byte offset from the start of the data section */
    uint64_t n_bytes;     /* GgufType::byte_size (gguf_loader.rs:120-126); 0 for unsupported types */
} rt_gguf_tensor;

/* GgufFile::open (gguf_loader.rs:167-230): header, metadata and tensor
 * directory; tensor data is read on demand.  Versions 2 and 3. */
rt_status rt_gguf_open(const char *path, rt_gguf **out);
rt_status rt_gguf_close(rt_gguf *g);
int64_t rt_gguf_n_tensors(const rt_gguf *g);
int64_t rt_gguf_n_metadata(const rt_gguf *g);
/* Byte offset of the data section (header padded to general.alignment, default 32). */
uint64_t rt_gguf_data_start(const rt_gguf *g);
rt_status rt_gguf_tensor_info(const rt_gguf *g, int64_t idx, rt_gguf_tensor *out);
/* GgufFile::find_tensor (gguf_loader.rs:248-250): index, or -1. */
int64_t rt_gguf_find_tensor(const rt_gguf *g, const char *name);

/* Metadata key i, in file order (0 <= i < rt_gguf_n_metadata). */
rt_status rt_gguf_meta_key(const rt_gguf *g, int64_t i, const char **key);
/* Metadata lookups.  rt_gguf_meta_type reports the value type and, for
 * arrays, the element type and count.  The scalar getters follow
 * GgufMetaValue::as_u64 / as_f32 / as_str (gguf_loader.rs:880-905):
 * as_u64 accepts u8/u16/u32/u64/i32/i64, as_f32 accepts f32/f64. */
rt_status rt_gguf_meta_type(const rt_gguf *g, const char *key, int32_t *type, int32_t *elem_type,
                            uint64_t *count);
rt_status rt_gguf_meta_u64(const rt_gguf *g, const char *key, uint64_t *out);
rt_status rt_gguf_meta_f32(const rt_gguf *g, const char *key, float *out);
rt_status rt_gguf_meta_str(const rt_gguf *g, const char *key, const char **out);
/* Element i of a string array (e.g. tokenizer.ggml.tokens). */
rt_status rt_gguf_meta_array_str(const rt_gguf *g, const char *key, uint64_t i, const char **out);

/* GgufFile::read_tensor_bytes (gguf_loader.rs:233-246): the raw bytes. */
rt_status rt_gguf_read_tensor(const rt_gguf *g, int64_t idx, void *dst, uint64_t capacity);

/* tensor_to_f32 (gguf_loader.rs:745-760): F32, F16, Q8_0, Q4_K, Q6_K, Q5_K,
 * Q4_0 to f32 in GGUF element order; other types (BF16 included, as in the
 * reference) return RT_EINVAL. */
rt_status rt_gguf_tensor_to_f32(const rt_gguf *g, int64_t idx, float *dst, uint64_t n_elem);

/* Q4KMat::quantize (autograd2.rs:1138-1168, quantize_block 1171-1245):
 * f32 [rows, cols] -> Q4_K blocks, cols % 256 == 0. */
rt_status rt_q4k_quantize(const float *src, size_t rows, size_t cols, uint8_t *blocks);

/* Q4KMat::quantize_from_bf16 (autograd2.rs:1252-1289): bf16 [rows, cols] ->
 * Q4_K blocks, row by row (no f32 copy of the whole matrix), cols % 256 == 0;
 * the same blocks as rt_q4k_quantize of the widened rows.  The reference's
 * q4k-lm-head feature requantises the tied lm_head this way at upload
 * (metal_decode.rs:1082-1094); see rt_decode_set_lm_head. */
rt_status rt_q4k_quantize_bf16(const uint16_t *src, size_t rows, size_t cols, uint8_t *blocks);

/* The weight of a linear layer as the hot path consumes it (RT_LINEAR_*
 * formats are defined in rt_hip.h). */
typedef struct {
    int32_t format;       /* RT_LINEAR_* */
    int32_t src_type;     /* ggml type id of the file tensor */
    int64_t rows, cols;   /* out_features, in_features (the file's [in, out] flipped) */
    void *data;           /* device buffer, row-major; freed by rt_linear_free */
    uint64_t bytes;
} rt_linear;

/* load_linear_from_gguf (transformer4.rs:1177-1256) plus the device upload
 * (metal_decode.rs:1259-1277): Q4_K stays packed (decode_q4k_to_q4kmat,
 * gguf_loader.rs:360-381); Q4_0 is requantised to Q4_K (Q4KMat::from_q4mat,
 * autograd2.rs:1291-1320; cols % 256 == 0); BF16 stays BF16; F16, Q8_0, Q5_K
 * and Q6_K widen to f32 and round to BF16; F32 stays F32.  Other types return
 * RT_EINVAL (the reference warns and skips the tensor). */
rt_status rt_gguf_load_linear(const rt_gguf *g, int64_t idx, rt_linear *out);
/* Same, with flags.  RT_LOAD_KEEP_PACKED keeps Q6_K (cols % 256 == 0) and
 * Q8_0 (cols % 32 == 0) tensors packed, in the planar layout the native
 * Q6_K / Q8_0 GEMVs read (formats RT_LINEAR_Q6K / RT_LINEAR_Q8_0), instead of
 * widening them to BF16 as the reference does.  No counterpart in the
 * reference. */
#define RT_LOAD_KEEP_PACKED 1
rt_status rt_gguf_load_linear_ex(const rt_gguf *g, int64_t idx, int32_t flags, rt_linear *out);
rt_status rt_linear_free(rt_linear *l);

#ifdef __cplusplus
}
#endif
#endif /* RT_GGUF_H */
