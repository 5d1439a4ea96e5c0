/*
 * rt_oracle.c -- CPU restatement of rich-triplet's portable x86 decode path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped).
 * Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -pthread).  Contraction
 * must stay off: the reference's Rust code rounds every `*` and `-` separately.
 * Citations are reference file:line (src/...).
 */
#include "rt_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------ */
/* bit casts                                                                 */
/* ------------------------------------------------------------------------ */
static inline float u32_as_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_as_u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* f16 -> f32, exact, subnormals normalised, Inf/NaN keep payload << 13.
 * autograd2.rs:1048-1070 (identical to gguf_loader.rs:947-976). */
float orc_f16_to_f32(uint16_t bits)
{
    uint32_t sign = (bits >> 15) & 1u;
    uint32_t exponent = (bits >> 10) & 0x1Fu;
    uint32_t mantissa = bits & 0x3FFu;
    uint32_t out;
    if (exponent == 0) {
        if (mantissa == 0) {
            out = sign << 31;
        } else {
            uint32_t m = mantissa, e = 0;
            while ((m & 0x400u) == 0) { m <<= 1; e += 1; }
            m &= 0x3FFu;
            out = (sign << 31) | ((127u - 14u - e) << 23) | (m << 13);
        }
    } else if (exponent == 0x1F) {
        out = (sign << 31) | (0xFFu << 23) | (mantissa << 13);
    } else {
        out = (sign << 31) | ((exponent + 127u - 15u) << 23) | (mantissa << 13);
    }
    return u32_as_f32(out);
}

/* f32 -> f16 with round-to-nearest-even.  Used only to write synthetic d/dmin;
 * the reference's own Q4KMat::f32_to_f16 (autograd2.rs:1090-1114) truncates,
 * so synthetic blocks are produced here and the oracle only ever decodes. */
uint16_t orc_f32_to_f16_rne(float v)
{
    uint32_t x = f32_as_u32(v);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                 /* Inf / NaN */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   /* rounds to >= 65520 -> Inf */
    if (ax < 0x38800000u) {                  /* result is f16 subnormal or zero */
        /* value = ax as float; f16 subnormal step = 2^-24 */
        float f = u32_as_f32(ax);
        float scaled = f * 16777216.0f;      /* exact: power of two */
        /* round half to even */
        float r = nearbyintf(scaled);        /* default rounding mode is RNE */
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

/* autograd2.rs:700-703 */
float orc_bf16_to_f32(uint16_t bits) { return u32_as_f32((uint32_t)bits << 16); }

/* autograd2.rs:709-719: RNE via bias 0x7fff + lsb, NaN keeps a set quiet bit. */
uint16_t orc_f32_to_bf16(float v)
{
    uint32_t bits = f32_as_u32(v);
    if (isnan(v)) return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t rounding_bias = 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + rounding_bias) >> 16);
}

/* ------------------------------------------------------------------------ */
/* Q4_K                                                                      */
/* ------------------------------------------------------------------------ */

/* get_scale_min_k4: autograd2.rs:1075-1085 (gguf_loader.rs:547-550, 565-575). */
void orc_q4k_scale_min(const uint8_t *sc, int j, float *sv, float *mv)
{
    uint8_t s, m;
    if (j < 4) {
        s = sc[j] & 0x3F;
        m = sc[j + 4] & 0x3F;
    } else {
        s = (uint8_t)((sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4));
        m = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
    }
    *sv = (float)s;
    *mv = (float)m;
}

/* pack_scales: autograd2.rs:1119-1132 -- inverse of scale_min. */
void orc_q4k_pack_scales(const uint8_t sv[8], const uint8_t mv[8], uint8_t out[12])
{
    for (int j = 0; j < 4; j++) {
        out[j] = (uint8_t)((sv[j] & 0x3F) | ((sv[j + 4] & 0x30) << 2));
        out[j + 4] = (uint8_t)((mv[j] & 0x3F) | ((mv[j + 4] & 0x30) << 2));
    }
    for (int j = 0; j < 4; j++)
        out[8 + j] = (uint8_t)((sv[j + 4] & 0x0F) | ((mv[j + 4] & 0x0F) << 4));
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* dequantize_row_into, scalar branch: autograd2.rs:1326-1366 (1359-1363).
 * w = (d*sv)*q - (dmin*mv), each product and the difference rounded in f32. */
void orc_q4k_dequant_row(const uint8_t *blocks, size_t cols, size_t row, float *out)
{
    size_t n_blocks = cols / 256;
    size_t base_block = row * n_blocks;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t *bp = blocks + (base_block + b) * 144;
        float d = orc_f16_to_f32(rd16(bp));
        float dmin = orc_f16_to_f32(rd16(bp + 2));
        const uint8_t *sc = bp + 4, *qs = bp + 16;
        float *o = out + b * 256;
        for (int chunk = 0; chunk < 4; chunk++) {
            float sv1, mv1, sv2, mv2;
            orc_q4k_scale_min(sc, chunk * 2, &sv1, &mv1);
            orc_q4k_scale_min(sc, chunk * 2 + 1, &sv2, &mv2);
            float scale1 = d * sv1, min1 = dmin * mv1;
            float scale2 = d * sv2, min2 = dmin * mv2;
            const uint8_t *q = qs + chunk * 32;
            float *lo = o + chunk * 64, *hi = lo + 32;
            for (int l = 0; l < 32; l++) {
                lo[l] = scale1 * (float)(q[l] & 0x0F) - min1;
                hi[l] = scale2 * (float)(q[l] >> 4) - min2;
            }
        }
    }
}

/* decode_q4k_to_f32: gguf_loader.rs:551-621.  A second, independently worded
 * restatement (running element counter, tail clip) -- tests require it to
 * agree bit-for-bit with orc_q4k_dequant_row. */
void orc_q4k_dequant_gguf(const uint8_t *bytes, size_t n_elem, float *out)
{
    size_t n_blocks = (n_elem + 255) / 256;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t *bp = bytes + b * 144;
        float d = orc_f16_to_f32(rd16(bp));
        float dmin = orc_f16_to_f32(rd16(bp + 2));
        const uint8_t *sc = bp + 4, *qs = bp + 16;
        size_t base = b * 256, end = base + 256 < n_elem ? base + 256 : n_elem;
        size_t q_off = 0, elem = 0;
        int is = 0;
        for (int c = 0; c < 4; c++) {
            float d1, m1, d2, m2;
            orc_q4k_scale_min(sc, is, &d1, &m1);
            orc_q4k_scale_min(sc, is + 1, &d2, &m2);
            float scale1 = d * d1, min1 = dmin * m1, scale2 = d * d2, min2 = dmin * m2;
            for (size_t l = 0; l < 32; l++, elem++)
                if (base + elem < end) out[base + elem] = scale1 * (float)(qs[q_off + l] & 0x0F) - min1;
            for (size_t l = 0; l < 32; l++, elem++)
                if (base + elem < end) out[base + elem] = scale2 * (float)(qs[q_off + l] >> 4) - min2;
            q_off += 32;
            is += 2;
        }
    }
}

/* ---- GGUF tensor formats and Q4_K quantisation ------------------------- */

/* Q4KMat::f32_to_f16 (autograd2.rs:1090-1117).  Its comment says
 * round-to-nearest, but the code drops the low 13 mantissa bits: truncation
 * toward zero.  Restated as the code computes it (the quantiser stores d and
 * dmin with it, so quantised bytes depend on it). */
uint16_t orc_f32_to_f16_trunc(float val)
{
    uint32_t bits = f32_as_u32(val);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant >> 13));
    int32_t new_exp = exp - 127 + 15;
    if (new_exp >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (new_exp <= 0) {
        if (new_exp < -10) return (uint16_t)sign;
        uint32_t m = mant | 0x800000u;
        uint32_t shift = (uint32_t)(1 - new_exp) + 13u;
        return (uint16_t)(sign | (m >> shift));
    }
    return (uint16_t)(sign | ((uint32_t)new_exp << 10) | (mant >> 13));
}

/* Rust's `f as u8`: saturating, NaN -> 0, truncation toward zero. */
static uint8_t rust_f32_as_u8(float x)
{
    if (!(x > 0.0f)) return 0;
    if (x >= 255.0f) return 255;
    return (uint8_t)x;
}

/* Q4KMat::quantize_block (autograd2.rs:1171-1245). */
void orc_q4k_quantize_block(const float *x, uint8_t out[144])
{
    float sub_scales[8], sub_mins[8];
    for (int sb = 0; sb < 8; sb++) {
        const float *sub = x + sb * 32;
        float smin = INFINITY, smax = -INFINITY;
        for (int i = 0; i < 32; i++) {
            float v = sub[i];
            if (v < smin) smin = v;
            if (v > smax) smax = v;
        }
        if (smin >= 0.0f) {
            sub_mins[sb] = 0.0f;
            sub_scales[sb] = smax > 0.0f ? smax / 15.0f : 0.0f;
        } else {
            sub_mins[sb] = smin;
            sub_scales[sb] = smax > smin ? (smax - smin) / 15.0f : 0.0f;
        }
    }
    /* fold(0.0, f32::max): f32::max returns the non-NaN operand, like fmaxf */
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        max_scale = fmaxf(max_scale, sub_scales[j]);
        max_min = fmaxf(max_min, -sub_mins[j]);
    }
    float d = max_scale > 0.0f ? max_scale / 63.0f : 0.0f;
    float dmin = max_min > 0.0f ? max_min / 63.0f : 0.0f;
    uint8_t sv[8] = {0}, mv[8] = {0};
    if (d > 0.0f) {
        float inv_d = 1.0f / d;
        for (int j = 0; j < 8; j++) {
            uint8_t q = rust_f32_as_u8(sub_scales[j] * inv_d + 0.5f);
            sv[j] = q < 63 ? q : 63;
        }
    }
    if (dmin > 0.0f) {
        float inv_dmin = 1.0f / dmin;
        for (int j = 0; j < 8; j++) {
            uint8_t q = rust_f32_as_u8((-sub_mins[j]) * inv_dmin + 0.5f);
            mv[j] = q < 63 ? q : 63;
        }
    }
    uint16_t d16 = orc_f32_to_f16_trunc(d), dmin16 = orc_f32_to_f16_trunc(dmin);
    out[0] = (uint8_t)(d16 & 0xFF); out[1] = (uint8_t)(d16 >> 8);
    out[2] = (uint8_t)(dmin16 & 0xFF); out[3] = (uint8_t)(dmin16 >> 8);
    orc_q4k_pack_scales(sv, mv, out + 4);
    float d_val = orc_f16_to_f32(d16), dmin_val = orc_f16_to_f32(dmin16);
    for (int chunk = 0; chunk < 4; chunk++) {
        float scale1 = d_val * (float)sv[chunk * 2];
        float min1 = dmin_val * (float)mv[chunk * 2];
        float scale2 = d_val * (float)sv[chunk * 2 + 1];
        float min2 = dmin_val * (float)mv[chunk * 2 + 1];
        const float *lo = x + chunk * 64, *hi = x + chunk * 64 + 32;
        for (int l = 0; l < 32; l++) {
            uint8_t q_lo = 0, q_hi = 0;
            if (scale1 > 0.0f) {
                q_lo = rust_f32_as_u8((lo[l] + min1) / scale1 + 0.5f);
                if (q_lo > 15) q_lo = 15;
            }
            if (scale2 > 0.0f) {
                q_hi = rust_f32_as_u8((hi[l] + min2) / scale2 + 0.5f);
                if (q_hi > 15) q_hi = 15;
            }
            out[16 + chunk * 32 + l] = (uint8_t)(q_lo | (q_hi << 4));
        }
    }
}

/* Q4KMat::quantize (autograd2.rs:1138-1168): block by block, row-major. */
void orc_q4k_quantize(const float *m, size_t rows, size_t cols, uint8_t *blocks)
{
    size_t nb = cols / 256;
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < nb; b++)
            orc_q4k_quantize_block(m + r * cols + b * 256, blocks + (r * nb + b) * 144);
}

/* decode_q4_0_to_f32 (gguf_loader.rs:425-480): 18-byte blocks, f16 scale then
 * 16 bytes whose low nibble is element k and high nibble element k+16. */
void orc_q4_0_dequant(const uint8_t *bytes, size_t n_elem, float *out)
{
    size_t n_blocks = (n_elem + 31) / 32;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t *bp = bytes + b * 18;
        float scale = orc_f16_to_f32(rd16(bp));
        size_t start = b * 32, end = start + 32 < n_elem ? start + 32 : n_elem;
        for (size_t k = 0; k < 16; k++) {
            uint8_t src = bp[2 + k];
            if (start + k < end) out[start + k] = (float)((int)(src & 0x0F) - 8) * scale;
            if (start + k + 16 < end) out[start + k + 16] = (float)((int)((src >> 4) & 0x0F) - 8) * scale;
        }
    }
}

/* load_linear_from_gguf's Q4_0 branch (transformer4.rs:1198-1207):
 * decode_q4_0_to_q4mat (gguf_loader.rs:282-357) stores the nibbles as signed
 * v-8 with the block's scale, Q4Mat::dequantize_row_into (autograd2.rs:
 * 2390-2414) returns q*scale for each element of a row, and
 * Q4KMat::from_q4mat (autograd2.rs:1291-1320) requantises every 256 of them. */
void orc_q4_0_to_q4k(const uint8_t *bytes, size_t rows, size_t cols, uint8_t *blocks)
{
    float *row = (float *)malloc(cols * sizeof(float));
    size_t nb = cols / 256;
    for (size_t r = 0; r < rows; r++) {
        for (size_t p = 0; p < cols; p++) {
            size_t flat = r * cols + p, blk = flat / 32, k = flat % 32;
            const uint8_t *bp = bytes + blk * 18;
            uint8_t nib = k < 16 ? (bp[2 + k] & 0x0F) : ((bp[2 + k - 16] >> 4) & 0x0F);
            int q = (int)((uint8_t)(nib - 8) & 0x0F);   /* the stored two's complement nibble */
            if (q >= 8) q -= 16;
            row[p] = (float)q * orc_f16_to_f32(rd16(bp));
        }
        for (size_t b = 0; b < nb; b++) orc_q4k_quantize_block(row + b * 256, blocks + (r * nb + b) * 144);
    }
    free(row);
}

/* decode_q6k_to_f32 (gguf_loader.rs:482-549): 210-byte blocks of ql[128],
 * qh[64], int8 scales[16], f16 d; two halves of 128 elements. */
void orc_q6k_dequant(const uint8_t *bytes, size_t n_elem, float *out)
{
    size_t n_blocks = (n_elem + 255) / 256;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t *bp = bytes + b * 210;
        const uint8_t *ql_all = bp, *qh_all = bp + 128, *sc_all = bp + 192;
        float d = orc_f16_to_f32(rd16(bp + 208));
        size_t base = b * 256, end = base + 256 < n_elem ? base + 256 : n_elem;
        for (int j = 0; j < 2; j++) {
            const uint8_t *ql = ql_all + j * 64, *qh = qh_all + j * 32, *sc = sc_all + j * 8;
            size_t y = base + (size_t)j * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                float s0 = d * (float)(int8_t)sc[is], s1 = d * (float)(int8_t)sc[is + 2];
                float s2 = d * (float)(int8_t)sc[is + 4], s3 = d * (float)(int8_t)sc[is + 6];
                if (y + l < end) out[y + l] = s0 * (float)q1;
                if (y + l + 32 < end) out[y + l + 32] = s1 * (float)q2;
                if (y + l + 64 < end) out[y + l + 64] = s2 * (float)q3;
                if (y + l + 96 < end) out[y + l + 96] = s3 * (float)q4;
            }
        }
    }
}

/* decode_q5k_to_f32 (gguf_loader.rs:664-743): 176-byte blocks of f16 d, f16
 * dmin, scales[12] (Q4_K packing), qh[32], qs[128]. */
void orc_q5k_dequant(const uint8_t *bytes, size_t n_elem, float *out)
{
    size_t n_blocks = (n_elem + 255) / 256;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t *bp = bytes + b * 176;
        float d = orc_f16_to_f32(rd16(bp)), dmin = orc_f16_to_f32(rd16(bp + 2));
        const uint8_t *sc = bp + 4, *qh = bp + 16, *qs = bp + 48;
        size_t base = b * 256, end = base + 256 < n_elem ? base + 256 : n_elem;
        size_t q_off = 0, elem = 0;
        int is = 0;
        for (int c = 0; c < 4; c++) {
            float d1, m1, d2, m2;
            orc_q4k_scale_min(sc, is, &d1, &m1);
            orc_q4k_scale_min(sc, is + 1, &d2, &m2);
            float scale1 = d * d1, min1 = dmin * m1, scale2 = d * d2, min2 = dmin * m2;
            for (size_t l = 0; l < 32; l++, elem++) {
                unsigned lo = qs[q_off + l] & 0x0F, hi = (qh[l] >> is) & 1;
                if (base + elem < end) out[base + elem] = scale1 * (float)(lo | (hi << 4)) - min1;
            }
            for (size_t l = 0; l < 32; l++, elem++) {
                unsigned lo = qs[q_off + l] >> 4, hi = (qh[l] >> (is + 1)) & 1;
                if (base + elem < end) out[base + elem] = scale2 * (float)(lo | (hi << 4)) - min2;
            }
            q_off += 32;
            is += 2;
        }
    }
}

/* decode_q8_0_to_f32 (gguf_loader.rs:628-650): 34-byte blocks, f16 d then 32
 * int8 quants. */
void orc_q8_0_dequant(const uint8_t *bytes, size_t n_elem, float *out)
{
    size_t n_blocks = (n_elem + 31) / 32;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t *bp = bytes + b * 34;
        float d = orc_f16_to_f32(rd16(bp));
        size_t base = b * 32;
        for (size_t i = 0; i < 32; i++)
            if (base + i < n_elem) out[base + i] = d * (float)(int8_t)bp[2 + i];
    }
}

/* dot_row, x86 scalar branch: autograd2.rs:1654-1701 ("integer trick"). */
float orc_q4k_dot_row(const uint8_t *blocks, size_t cols, size_t row, const float *a)
{
    size_t n_blocks = cols / 256;
    size_t base_block = row * n_blocks;
    float acc = 0.0f;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t *bp = blocks + (base_block + b) * 144;
        float d = orc_f16_to_f32(rd16(bp));
        float dmin = orc_f16_to_f32(rd16(bp + 2));
        const uint8_t *sc = bp + 4, *qs = bp + 16;
        size_t a_base = b * 256;
        for (int chunk = 0; chunk < 4; chunk++) {
            float sv1, mv1, sv2, mv2;
            orc_q4k_scale_min(sc, chunk * 2, &sv1, &mv1);
            orc_q4k_scale_min(sc, chunk * 2 + 1, &sv2, &mv2);
            float scale1 = d * sv1, min1 = dmin * mv1;
            float scale2 = d * sv2, min2 = dmin * mv2;
            const uint8_t *q = qs + chunk * 32;
            size_t a_off = a_base + (size_t)chunk * 64;
            float dot_lo = 0.0f, dot_hi = 0.0f, sum_a_lo = 0.0f, sum_a_hi = 0.0f;
            for (int l = 0; l < 32; l++) {
                float a_lo = a[a_off + l];
                dot_lo += (float)(q[l] & 0x0F) * a_lo;
                sum_a_lo += a_lo;
                float a_hi = a[a_off + 32 + l];
                dot_hi += (float)(q[l] >> 4) * a_hi;
                sum_a_hi += a_hi;
            }
            acc += scale1 * dot_lo - min1 * sum_a_lo + scale2 * dot_hi - min2 * sum_a_hi;
        }
    }
    return acc;
}

/* ------------------------------------------------------------------------ */
/* row-band threading as in gemv_mt (autograd2.rs:1961-2011):               */
/* n_threads = min(hw, N/128).max(1); contiguous [j0, j1) per thread.        */
/* ------------------------------------------------------------------------ */
typedef void (*band_fn)(void *ctx, size_t j0, size_t j1);
typedef struct { band_fn fn; void *ctx; size_t j0, j1; } band_job;

static void *band_main(void *p)
{
    band_job *j = (band_job *)p;
    j->fn(j->ctx, j->j0, j->j1);
    return NULL;
}

/* Threads for the row bands: RT_ORACLE_THREADS if set, else the online CPU
 * count capped at 16 (the share of host cores a one-GPU job may use). */
int orc_hw_threads(void)
{
    const char *env = getenv("RT_ORACLE_THREADS");
    if (env && atoi(env) > 0) return atoi(env);
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    if (n > 16) n = 16;
    return n > 0 ? (int)n : 1;
}

static void run_bands(size_t n, int hw_threads, size_t min_rows_per_thread, band_fn fn, void *ctx)
{
    if (hw_threads <= 0) hw_threads = orc_hw_threads();
    size_t nt = (size_t)hw_threads;
    size_t cap = n / min_rows_per_thread;
    if (nt > cap) nt = cap;
    if (nt < 1) nt = 1;
    if (nt == 1) { fn(ctx, 0, n); return; }
    size_t chunk = (n + nt - 1) / nt;
    pthread_t *th = (pthread_t *)malloc(nt * sizeof(pthread_t));
    band_job *jobs = (band_job *)malloc(nt * sizeof(band_job));
    size_t started = 0;
    for (size_t t = 0; t < nt; t++) {
        size_t j0 = t * chunk, j1 = (t + 1) * chunk;
        if (j0 >= n) break;
        if (j1 > n) j1 = n;
        jobs[t] = (band_job){fn, ctx, j0, j1};
        pthread_create(&th[t], NULL, band_main, &jobs[t]);
        started++;
    }
    for (size_t t = 0; t < started; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

typedef struct { const uint8_t *blocks; size_t cols; const float *a; float *y; } q4k_gemv_ctx;
static void q4k_gemv_band(void *p, size_t j0, size_t j1)
{
    q4k_gemv_ctx *c = (q4k_gemv_ctx *)p;
    for (size_t j = j0; j < j1; j++) c->y[j] = orc_q4k_dot_row(c->blocks, c->cols, j, c->a);
}

/* gemv_mt: autograd2.rs:1953-2035 (x86 branch calls dot_row per row). */
void orc_q4k_gemv_mt(const uint8_t *blocks, size_t rows, size_t cols, const float *a, float *y, int hw_threads)
{
    q4k_gemv_ctx c = {blocks, cols, a, y};
    run_bands(rows, hw_threads, 128, q4k_gemv_band, &c);
}

/* fp64 twin: dequantise (bit-exact f32 weights) and accumulate in double. */
typedef struct { const uint8_t *blocks; size_t cols; const float *a; double *y; } q4k_f64_ctx;
static void q4k_f64_band(void *p, size_t j0, size_t j1)
{
    q4k_f64_ctx *c = (q4k_f64_ctx *)p;
    float *row = (float *)malloc(c->cols * sizeof(float));
    for (size_t j = j0; j < j1; j++) {
        orc_q4k_dequant_row(c->blocks, c->cols, j, row);
        double s = 0.0;
        for (size_t p2 = 0; p2 < c->cols; p2++) s += (double)row[p2] * (double)c->a[p2];
        c->y[j] = s;
    }
    free(row);
}
void orc_q4k_gemv_f64(const uint8_t *blocks, size_t rows, size_t cols, const float *a, double *y)
{
    q4k_f64_ctx c = {blocks, cols, a, y};
    run_bands(rows, 0, 16, q4k_f64_band, &c);
}

/* BF16 dot_row, x86 scalar branch: autograd2.rs:879-887. */
float orc_bf16_dot_row(const uint16_t *w, size_t cols, size_t row, const float *a)
{
    const uint16_t *r = w + row * cols;
    float acc = 0.0f;
    for (size_t p = 0; p < cols; p++) acc += orc_bf16_to_f32(r[p]) * a[p];
    return acc;
}

typedef struct { const uint16_t *w; size_t cols; const float *a; float *y; } bf16_ctx;
static void bf16_band(void *p, size_t j0, size_t j1)
{
    bf16_ctx *c = (bf16_ctx *)p;
    for (size_t j = j0; j < j1; j++) c->y[j] = orc_bf16_dot_row(c->w, c->cols, j, c->a);
}
/* MatBf16::gemv_mt: autograd2.rs:954-1000. */
void orc_bf16_gemv_mt(const uint16_t *w, size_t rows, size_t cols, const float *a, float *y, int hw_threads)
{
    bf16_ctx c = {w, cols, a, y};
    run_bands(rows, hw_threads, 128, bf16_band, &c);
}

typedef struct { const uint16_t *w; size_t cols; const float *a; double *y; } bf16_f64_ctx;
static void bf16_f64_band(void *p, size_t j0, size_t j1)
{
    bf16_f64_ctx *c = (bf16_f64_ctx *)p;
    for (size_t j = j0; j < j1; j++) {
        const uint16_t *r = c->w + j * c->cols;
        double s = 0.0;
        for (size_t k = 0; k < c->cols; k++) s += (double)orc_bf16_to_f32(r[k]) * (double)c->a[k];
        c->y[j] = s;
    }
}
void orc_bf16_gemv_f64(const uint16_t *w, size_t rows, size_t cols, const float *a, double *y)
{
    bf16_f64_ctx c = {w, cols, a, y};
    run_bands(rows, 0, 16, bf16_f64_band, &c);
}

/* ------------------------------------------------------------------------ */
/* GEMM                                                                      */
/* ------------------------------------------------------------------------ */
typedef struct { const float *a; size_t m; const uint8_t *blocks; size_t n, k; float *c; double *c64; int fmt; } mm_ctx;
static void proj_row(int fmt, const uint8_t *w, size_t cols, size_t j, float *row);
static void mm_band(void *p, size_t j0, size_t j1)
{
    mm_ctx *c = (mm_ctx *)p;
    float *row = (float *)malloc(c->k * sizeof(float));
    for (size_t j = j0; j < j1; j++) {
        proj_row(c->fmt, c->blocks, c->k, j, row);
        for (size_t i = 0; i < c->m; i++) {
            const float *ai = c->a + i * c->k;
            if (c->c64) {
                double acc = 0.0;
                for (size_t p2 = 0; p2 < c->k; p2++) acc += (double)ai[p2] * (double)row[p2];
                c->c64[i * c->n + j] = acc;
            } else {
                float acc = 0.0f;
                for (size_t p2 = 0; p2 < c->k; p2++) acc += ai[p2] * row[p2];
                c->c[i * c->n + j] = acc;
            }
        }
    }
    free(row);
}
/* matmul_q4k_t, M>1 branch: autograd2.rs:1437-1457 -- dequantise row j, then
 * a sequential f32 dot per output.  (The BLAS build's matmul_q4k_t_exact,
 * 1507-1625, computes the same products through third-party sgemm, whose
 * summation order is unspecified; the f64 twin below pins that path.)
 * Threaded over output columns; every output is computed independently. */
void orc_q4k_matmul(const float *a, size_t m, const uint8_t *blocks, size_t n, size_t k, float *c, int hw_threads)
{
    mm_ctx ctx = {a, m, blocks, n, k, c, NULL, 1};
    run_bands(n, hw_threads, 1, mm_band, &ctx);
}
/* The same GEMM for a projection in any orc_layer.fmt format: row j is
 * widened to f32 as the format's decoder does (the reference widens Q6_K and
 * Q8_0 to BF16 at load, transformer4.rs:1233-1242, and multiplies with
 * MatBf16::matmul_by_t, autograd2.rs:757-852), then a sequential f32 dot. */
void orc_proj_matmul(int fmt, const float *a, size_t m, const uint8_t *w, size_t n, size_t k, float *c, int hw_threads)
{
    mm_ctx ctx = {a, m, w, n, k, c, NULL, fmt};
    run_bands(n, hw_threads, 1, mm_band, &ctx);
}
/* QLinear::forward (qlinear.rs:82-111): the format's matmul (Q4_K:
 * matmul_q4k_t_exact, BF16: matmul_by_t, F32: matmul_bt -- each a dot per
 * output of the widened row, as orc_proj_matmul), then add_bias_rows
 * (qlinear.rs:49-60): out[r][c] += bias[c], skipped when bias is NULL. */
void orc_qlinear_forward(int fmt, const float *a, size_t m, const uint8_t *w, const float *bias, size_t n, size_t k,
                         float *c, int hw_threads)
{
    orc_proj_matmul(fmt, a, m, w, n, k, c, hw_threads);
    if (!bias) return;
    for (size_t r = 0; r < m; r++)
        for (size_t j = 0; j < n; j++) c[r * n + j] += bias[j];
}
void orc_q4k_matmul_f64(const float *a, size_t m, const uint8_t *blocks, size_t n, size_t k, double *c, int hw_threads)
{
    mm_ctx ctx = {a, m, blocks, n, k, NULL, c, 1};
    run_bands(n, hw_threads, 1, mm_band, &ctx);
}

/* ------------------------------------------------------------------------ */
/* decode-step math                                                          */
/* ------------------------------------------------------------------------ */

/* rms_norm_gemma3: autograd2.rs:3477-3496.
 * mean_sq = (sum_c x^2) * (1/d); rms_inv = 1/sqrt(mean_sq+eps);
 * out = (x*rms_inv) * (1+gamma). */
void orc_rms_norm_gemma3(const float *x, const float *gamma, size_t d, float eps, float *out)
{
    float inv_d = 1.0f / (float)d;
    float ss = 0.0f;
    for (size_t c = 0; c < d; c++) ss += x[c] * x[c];
    float mean_sq = ss * inv_d;
    float rms_inv = 1.0f / sqrtf(mean_sq + eps);
    for (size_t c = 0; c < d; c++) {
        float xh = x[c] * rms_inv;
        out[c] = xh * (1.0f + gamma[c]);
    }
}

/* apply_per_head_norm: transformer4.rs:2485-2508 (gamma shared across heads). */
void orc_per_head_norm(const float *x, const float *gamma, size_t n_heads, size_t head_dim, float eps, float *out)
{
    for (size_t h = 0; h < n_heads; h++)
        orc_rms_norm_gemma3(x + h * head_dim, gamma, head_dim, eps, out + h * head_dim);
}

/* apply_rope_at_offset (single row): transformer4.rs:2742-2772, NeoX half split.
 * angle = (pos*fs) / theta^(2i/d). */
void orc_rope_neox(float *x, size_t n_heads, size_t head_dim, float theta, size_t pos, float freq_scale)
{
    size_t half = head_dim / 2;
    for (size_t h = 0; h < n_heads; h++) {
        for (size_t i = 0; i < half; i++) {
            float angle = ((float)pos * freq_scale) / powf(theta, 2.0f * (float)i / (float)head_dim);
            float cos_a = cosf(angle), sin_a = sinf(angle);
            size_t c0 = h * head_dim + i, c1 = c0 + half;
            float x0 = x[c0], x1 = x[c1];
            x[c0] = x0 * cos_a - x1 * sin_a;
            x[c1] = x0 * sin_a + x1 * cos_a;
        }
    }
}

/* gelu_tanh: autograd2.rs:3082-3091. */
float orc_gelu_tanh(float xv)
{
    const float SQRT_2_OVER_PI = 0.7978845608028654f;
    const float COEFF = 0.044715f;
    float inner = SQRT_2_OVER_PI * (xv + COEFF * xv * xv * xv);
    return xv * 0.5f * (1.0f + tanhf(inner));
}

/* gqa_attention_cached, t_q == 1, non-BLAS loops: transformer4.rs:2806-2879. */
void orc_gqa_attention_decode(const float *q, const float *k_cache, const float *v_cache,
                              size_t k_start, size_t k_end, size_t n_q_heads, size_t n_kv_heads,
                              size_t d_head, float scale, float *out)
{
    size_t t_kv = k_end - k_start;
    size_t kv_stride = n_kv_heads * d_head;
    size_t group = n_q_heads / n_kv_heads;
    float *scores = (float *)malloc((t_kv ? t_kv : 1) * sizeof(float));
    memset(out, 0, n_q_heads * d_head * sizeof(float));
    for (size_t qh = 0; qh < n_q_heads; qh++) {
        size_t kvh = qh / group;
        size_t q_off = qh * d_head, kv_off = kvh * d_head, out_off = qh * d_head;
        for (size_t ci = 0; ci < t_kv; ci++) {
            size_t k_base = (k_start + ci) * kv_stride + kv_off;
            float dot = 0.0f;
            for (size_t di = 0; di < d_head; di++) dot += q[q_off + di] * k_cache[k_base + di];
            scores[ci] = dot * scale;
        }
        float max_s = -INFINITY;
        for (size_t ci = 0; ci < t_kv; ci++) max_s = fmaxf(max_s, scores[ci]);
        float sum_exp = 0.0f;
        for (size_t ci = 0; ci < t_kv; ci++) {
            scores[ci] = expf(scores[ci] - max_s);
            sum_exp += scores[ci];
        }
        if (sum_exp > 0.0f)
            for (size_t ci = 0; ci < t_kv; ci++) scores[ci] /= sum_exp;
        for (size_t ci = 0; ci < t_kv; ci++) {
            size_t v_base = (k_start + ci) * kv_stride + kv_off;
            float w = scores[ci];
            for (size_t di = 0; di < d_head; di++) out[out_off + di] += w * v_cache[v_base + di];
        }
    }
    free(scores);
}

/* Row j of a projection in format fmt (1 Q4_K, 2 BF16, 4 Q6_K, 5 Q8_0). */
static void proj_row(int fmt, const uint8_t *w, size_t cols, size_t j, float *row)
{
    if (fmt == 2) {
        const uint16_t *r = (const uint16_t *)w + j * cols;
        for (size_t i = 0; i < cols; i++) row[i] = orc_bf16_to_f32(r[i]);
    } else if (fmt == 3) {  /* f32 weights: Mat::matmul_bt, scalar branch (autograd2.rs:410-429) */
        memcpy(row, (const float *)w + j * cols, cols * sizeof(float));
    } else if (fmt == 4) orc_q6k_dequant(w + j * (cols / 256) * 210, cols, row);
    else if (fmt == 5) orc_q8_0_dequant(w + j * (cols / 32) * 34, cols, row);
    else orc_q4k_dequant_row(w, cols, j, row);
}

/* Per-format projection GEMV (formats of orc_layer.fmt). */
typedef struct { int fmt; const uint8_t *w; size_t cols; const float *x; float *y; } pg_ctx;
static void pg_band(void *p, size_t j0, size_t j1)
{
    pg_ctx *c = (pg_ctx *)p;
    float *row = (float *)malloc(c->cols * sizeof(float));
    for (size_t j = j0; j < j1; j++) {
        proj_row(c->fmt, c->w, c->cols, j, row);
        float acc = 0.0f;
        for (size_t i = 0; i < c->cols; i++) acc += row[i] * c->x[i];
        c->y[j] = acc;
    }
    free(row);
}
void orc_proj_gemv(int fmt, const uint8_t *w, size_t rows, size_t cols, const float *x, float *y, int hw)
{
    if (fmt == 2) { orc_bf16_gemv_mt((const uint16_t *)w, rows, cols, x, y, hw); return; }
    if (fmt == 4 || fmt == 5) {
        pg_ctx ctx = {fmt, w, cols, x, y};
        run_bands(rows, hw, 1, pg_band, &ctx);
        return;
    }
    orc_q4k_gemv_mt(w, rows, cols, x, y, hw);
}

static int is_global(const orc_gemma3_cfg *cfg, int layer)
{
    /* Config4::is_global_layer: transformer4.rs:141-143 (layer % 6 == 5).
     * global_every <= 0 (a config knob of this restatement; the reference
     * fixes 6) means every layer is a sliding-window layer. */
    if (cfg->global_every <= 0) return 0;
    return (layer % cfg->global_every) == cfg->global_every - 1;
}

/* Gemma3Block::forward_cached: transformer4.rs:1954-1964, with
 * Gemma3Attention::forward_cached 1900-1946 and Gemma3Mlp::forward 328-334. */
void orc_gemma3_layer(const orc_gemma3_cfg *cfg, const orc_layer *L, int layer_idx, float *x, uint32_t pos, int hw)
{
    size_t H = (size_t)cfg->hidden, F = (size_t)cfg->ffn, D = (size_t)cfg->head_dim;
    size_t NQ = (size_t)cfg->n_q_heads, NKV = (size_t)cfg->n_kv_heads;
    size_t QD = NQ * D, KVD = NKV * D;
    int glob = is_global(cfg, layer_idx);
    float theta = glob ? cfg->rope_theta_global : cfg->rope_theta_local;
    float fs = glob ? cfg->rope_fs_global : cfg->rope_fs_local;

    float *normed = (float *)malloc(H * sizeof(float));
    float *q = (float *)malloc(QD * sizeof(float)), *qn = (float *)malloc(QD * sizeof(float));
    float *k = (float *)malloc(KVD * sizeof(float)), *kn = (float *)malloc(KVD * sizeof(float));
    float *v = (float *)malloc(KVD * sizeof(float));
    float *attn = (float *)malloc(QD * sizeof(float));
    float *o = (float *)malloc(H * sizeof(float)), *on = (float *)malloc(H * sizeof(float));
    float *x2 = (float *)malloc(H * sizeof(float)), *n2 = (float *)malloc(H * sizeof(float));
    float *g = (float *)malloc(F * sizeof(float)), *u = (float *)malloc(F * sizeof(float));
    float *m = (float *)malloc(H * sizeof(float)), *mn = (float *)malloc(H * sizeof(float));

    orc_rms_norm_gemma3(x, L->in_norm, H, cfg->eps, normed);
    orc_proj_gemv(L->fmt[0], L->q, QD, H, normed, q, hw);
    orc_proj_gemv(L->fmt[1], L->k, KVD, H, normed, k, hw);
    orc_proj_gemv(L->fmt[2], L->v, KVD, H, normed, v, hw);
    orc_per_head_norm(q, L->q_norm, NQ, D, cfg->eps, qn);
    orc_per_head_norm(k, L->k_norm, NKV, D, cfg->eps, kn);
    orc_rope_neox(qn, NQ, D, theta, pos, fs);
    orc_rope_neox(kn, NKV, D, theta, pos, fs);
    /* Gemma3LayerKvCache::append at row seq_len == pos: transformer4.rs:1813-1823 */
    memcpy(L->k_cache + (size_t)pos * KVD, kn, KVD * sizeof(float));
    memcpy(L->v_cache + (size_t)pos * KVD, v, KVD * sizeof(float));
    size_t k_end = (size_t)pos + 1;
    size_t k_start = 0;
    if (!glob && cfg->sliding_window > 0)
        k_start = k_end > (size_t)cfg->sliding_window ? k_end - (size_t)cfg->sliding_window : 0;
    orc_gqa_attention_decode(qn, L->k_cache, L->v_cache, k_start, k_end, NQ, NKV, D, cfg->attn_scale, attn);
    orc_proj_gemv(L->fmt[3], L->o, H, QD, attn, o, hw);
    orc_rms_norm_gemma3(o, L->post_attn_norm, H, cfg->eps, on);
    for (size_t c = 0; c < H; c++) x2[c] = x[c] + on[c];
    orc_rms_norm_gemma3(x2, L->pre_ffn_norm, H, cfg->eps, n2);
    orc_proj_gemv(L->fmt[4], L->gate, F, H, n2, g, hw);
    orc_proj_gemv(L->fmt[5], L->up, F, H, n2, u, hw);
    for (size_t c = 0; c < F; c++) g[c] = orc_gelu_tanh(g[c]) * u[c];
    orc_proj_gemv(L->fmt[6], L->down, H, F, g, m, hw);
    orc_rms_norm_gemma3(m, L->post_ffn_norm, H, cfg->eps, mn);
    for (size_t c = 0; c < H; c++) x[c] = x2[c] + mn[c];

    free(normed); free(q); free(qn); free(k); free(kn); free(v); free(attn);
    free(o); free(on); free(x2); free(n2); free(g); free(u); free(m); free(mn);
}

/* Decode step, CPU branch: transformer4.rs:2358-2385. */
void orc_gemma3_decode_step(const orc_gemma3_cfg *cfg, const orc_layer *layers,
                            const uint16_t *embed_bf16, const float *final_norm,
                            uint32_t token, uint32_t pos, float *logits, float *hidden_out, int hw)
{
    size_t H = (size_t)cfg->hidden;
    float scale = sqrtf((float)H);        /* transformer4.rs:2092 */
    float *x = (float *)malloc(H * sizeof(float));
    float *xn = (float *)malloc(H * sizeof(float));
    for (size_t c = 0; c < H; c++) x[c] = orc_bf16_to_f32(embed_bf16[(size_t)token * H + c]) * scale;
    for (int l = 0; l < cfg->n_layers; l++) orc_gemma3_layer(cfg, &layers[l], l, x, pos, hw);
    if (hidden_out) memcpy(hidden_out, x, H * sizeof(float));
    orc_rms_norm_gemma3(x, final_norm, H, cfg->eps, xn);
    orc_bf16_gemv_mt(embed_bf16, (size_t)cfg->vocab, H, xn, logits, hw);
    free(x);
    free(xn);
}

/* ------------------------------------------------------------------------ */
/* prefill (many query rows per layer)                                       */
/* ------------------------------------------------------------------------ */

/* Attention of T query rows at absolute positions p0 .. p0+T-1 against the
 * cache.  Row t (position r = p0 + t) sees keys [lo(r), r] with
 * lo(r) = max(lo_fixed, window > 0 ? r + 1 - window : 0); an empty range
 * leaves the row zero.  With lo_fixed = seq_len - window (p0 = 0) this is
 * gqa_attention_cached's prefill branch (transformer4.rs:2882-2940: k_start
 * = lo_fixed, "r < k_start attends to nothing", max_kv = r - k_start); with
 * lo_fixed = 0 and window = w it is gqa_attention_windowed's mask
 * (2661-2700: c <= r && (r < w || c >= r + 1 - w)).  The arithmetic follows
 * 2897-2940: scores (q.k)*scale, row max over the valid keys, exp, row sum,
 * divide, then w.v accumulated over the keys. */
void orc_gqa_attention_prefill(const float *q, const float *k_cache, const float *v_cache, size_t p0, size_t T,
                               size_t lo_fixed, size_t window, size_t n_q_heads, size_t n_kv_heads, size_t d_head,
                               float scale, float *out)
{
    size_t kv_stride = n_kv_heads * d_head, q_stride = n_q_heads * d_head;
    size_t group = n_q_heads / n_kv_heads;
    float *w = (float *)malloc((p0 + T) * sizeof(float));
    memset(out, 0, T * q_stride * sizeof(float));
    for (size_t qh = 0; qh < n_q_heads; qh++) {
        size_t kv_off = (qh / group) * d_head;
        for (size_t t = 0; t < T; t++) {
            size_t r = p0 + t;
            size_t lo = lo_fixed;
            if (window > 0 && r + 1 > window && r + 1 - window > lo) lo = r + 1 - window;
            if (lo > r) continue;  /* no key: the row stays zero */
            const float *qr = q + t * q_stride + qh * d_head;
            float row_max = -INFINITY;
            for (size_t j = lo; j <= r; j++) {
                const float *kr = k_cache + j * kv_stride + kv_off;
                float dot = 0.0f;
                for (size_t d = 0; d < d_head; d++) dot += qr[d] * kr[d];
                w[j] = dot * scale;
                row_max = fmaxf(row_max, w[j]);
            }
            float row_sum = 0.0f;
            for (size_t j = lo; j <= r; j++) {
                w[j] = expf(w[j] - row_max);
                row_sum += w[j];
            }
            if (row_sum > 0.0f)
                for (size_t j = lo; j <= r; j++) w[j] /= row_sum;
            float *o = out + t * q_stride + qh * d_head;
            for (size_t j = lo; j <= r; j++) {
                const float *vr = v_cache + j * kv_stride + kv_off;
                for (size_t d = 0; d < d_head; d++) o[d] += w[j] * vr[d];
            }
        }
    }
    free(w);
}

/* Prefill of tokens[0..T) at positions p0 .. p0+T-1: Gemma3Block::
 * forward_cached over all rows at once (transformer4.rs:1900-1964, the
 * projections through matmul_q4k_t), then the last row's final norm and
 * lm_head (2131-2139).  mode 0: the reference's prefill window rule
 * (lo_fixed = T - window for sliding-window layers, p0 must be 0); mode 1:
 * per-row sliding window.  Appends rows p0 .. p0+T-1 to every layer's
 * cache. */
void orc_gemma3_prefill(const orc_gemma3_cfg *cfg, const orc_layer *layers, const uint16_t *embed_bf16,
                        const float *final_norm, const uint32_t *tokens, size_t T, size_t p0, int mode,
                        float *logits, int hw)
{
    size_t H = (size_t)cfg->hidden, F = (size_t)cfg->ffn, D = (size_t)cfg->head_dim;
    size_t NQ = (size_t)cfg->n_q_heads, NKV = (size_t)cfg->n_kv_heads;
    size_t QD = NQ * D, KVD = NKV * D;
    float scale = sqrtf((float)H);
    float *x = (float *)malloc(T * H * sizeof(float)), *xn = (float *)malloc(T * H * sizeof(float));
    float *q = (float *)malloc(T * QD * sizeof(float)), *k = (float *)malloc(T * KVD * sizeof(float));
    float *v = (float *)malloc(T * KVD * sizeof(float)), *att = (float *)malloc(T * QD * sizeof(float));
    float *o = (float *)malloc(T * H * sizeof(float)), *x2 = (float *)malloc(T * H * sizeof(float));
    float *g = (float *)malloc(T * F * sizeof(float)), *u = (float *)malloc(T * F * sizeof(float));
    float *tmp = (float *)malloc((QD > H ? QD : H) * sizeof(float));
    for (size_t t = 0; t < T; t++)
        for (size_t c = 0; c < H; c++) x[t * H + c] = orc_bf16_to_f32(embed_bf16[(size_t)tokens[t] * H + c]) * scale;
    for (int l = 0; l < cfg->n_layers; l++) {
        const orc_layer *L = &layers[l];
        int glob = is_global(cfg, l);
        float theta = glob ? cfg->rope_theta_global : cfg->rope_theta_local;
        float fs = glob ? cfg->rope_fs_global : cfg->rope_fs_local;
        for (size_t t = 0; t < T; t++) orc_rms_norm_gemma3(x + t * H, L->in_norm, H, cfg->eps, xn + t * H);
        orc_proj_matmul(L->fmt[0], xn, T, L->q, QD, H, q, hw);
        orc_proj_matmul(L->fmt[1], xn, T, L->k, KVD, H, k, hw);
        orc_proj_matmul(L->fmt[2], xn, T, L->v, KVD, H, v, hw);
        for (size_t t = 0; t < T; t++) {
            orc_per_head_norm(q + t * QD, L->q_norm, NQ, D, cfg->eps, tmp);
            memcpy(q + t * QD, tmp, QD * sizeof(float));
            orc_per_head_norm(k + t * KVD, L->k_norm, NKV, D, cfg->eps, tmp);
            memcpy(k + t * KVD, tmp, KVD * sizeof(float));
            orc_rope_neox(q + t * QD, NQ, D, theta, p0 + t, fs);
            orc_rope_neox(k + t * KVD, NKV, D, theta, p0 + t, fs);
            /* Gemma3LayerKvCache::append (transformer4.rs:1813-1823) */
            memcpy(L->k_cache + (p0 + t) * KVD, k + t * KVD, KVD * sizeof(float));
            memcpy(L->v_cache + (p0 + t) * KVD, v + t * KVD, KVD * sizeof(float));
        }
        size_t lo_fixed = 0, window = 0;
        if (!glob && cfg->sliding_window > 0) {
            size_t w = (size_t)cfg->sliding_window, seq_len = p0 + T;
            if (mode == 0) lo_fixed = seq_len > w ? seq_len - w : 0;  /* k_start, 1926-1929 */
            else window = w;
        }
        orc_gqa_attention_prefill(q, L->k_cache, L->v_cache, p0, T, lo_fixed, window, NQ, NKV, D, cfg->attn_scale, att);
        orc_proj_matmul(L->fmt[3], att, T, L->o, H, QD, o, hw);
        for (size_t t = 0; t < T; t++) {
            orc_rms_norm_gemma3(o + t * H, L->post_attn_norm, H, cfg->eps, tmp);
            for (size_t c = 0; c < H; c++) x2[t * H + c] = x[t * H + c] + tmp[c];
            orc_rms_norm_gemma3(x2 + t * H, L->pre_ffn_norm, H, cfg->eps, xn + t * H);
        }
        orc_proj_matmul(L->fmt[4], xn, T, L->gate, F, H, g, hw);
        orc_proj_matmul(L->fmt[5], xn, T, L->up, F, H, u, hw);
        for (size_t i = 0; i < T * F; i++) g[i] = orc_gelu_tanh(g[i]) * u[i];
        orc_proj_matmul(L->fmt[6], g, T, L->down, H, F, o, hw);
        for (size_t t = 0; t < T; t++) {
            orc_rms_norm_gemma3(o + t * H, L->post_ffn_norm, H, cfg->eps, tmp);
            for (size_t c = 0; c < H; c++) x[t * H + c] = x2[t * H + c] + tmp[c];
        }
    }
    orc_rms_norm_gemma3(x + (T - 1) * H, final_norm, H, cfg->eps, xn);
    orc_bf16_gemv_mt(embed_bf16, (size_t)cfg->vocab, H, xn, logits, hw);
    free(x); free(xn); free(q); free(k); free(v); free(att); free(o); free(x2); free(g); free(u); free(tmp);
}

/* ------------------------------------------------------------------------ */
/* seeded synthetic data                                                     */
/* ------------------------------------------------------------------------ */

/* i-th output of splitmix64 started at `seed` (counter based, so any element
 * can be generated independently and in parallel). */
uint64_t orc_rng_u64(uint64_t seed, uint64_t i)
{
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Box-Muller (cosine branch) from draws 2i, 2i+1. */
static double normal_at(uint64_t seed, uint64_t i)
{
    uint64_t a = orc_rng_u64(seed, 2 * i), b = orc_rng_u64(seed, 2 * i + 1);
    double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);   /* (0,1] */
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);           /* [0,1) */
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

typedef struct { uint64_t seed; float mean, std; float *out; uint16_t *out16; uint8_t *blocks; } synth_ctx;

static void normal_band(void *p, size_t j0, size_t j1)
{
    synth_ctx *c = (synth_ctx *)p;
    for (size_t i = j0; i < j1; i++) c->out[i] = (float)(c->mean + c->std * normal_at(c->seed, i));
}
void orc_synth_normal_f32(uint64_t seed, size_t n, float mean, float std, float *out)
{
    synth_ctx c = {seed, mean, std, out, NULL, NULL};
    run_bands(n, 0, 65536, normal_band, &c);
}

static void bf16_synth_band(void *p, size_t j0, size_t j1)
{
    synth_ctx *c = (synth_ctx *)p;
    for (size_t i = j0; i < j1; i++) c->out16[i] = orc_f32_to_bf16((float)(c->std * normal_at(c->seed, i)));
}
void orc_synth_bf16(uint64_t seed, size_t n, float std, uint16_t *out)
{
    synth_ctx c = {seed, 0.0f, std, NULL, out, NULL};
    run_bands(n, 0, 65536, bf16_synth_band, &c);
}

/* One Q4_K super-block per index g:
 *   d, dmin = f16_rne(|N(0, d_std)|); eight 6-bit scales and eight 6-bit mins
 *   uniform in 0..63, packed with pack_scales; 128 quant bytes uniform. */
static void q4k_band(void *p, size_t j0, size_t j1)
{
    synth_ctx *c = (synth_ctx *)p;
    for (size_t g = j0; g < j1; g++) {
        uint64_t s = orc_rng_u64(c->seed, g);
        uint8_t *bp = c->blocks + g * 144;
        uint16_t d = orc_f32_to_f16_rne((float)fabs(c->std * normal_at(s, 0)));
        uint16_t dm = orc_f32_to_f16_rne((float)fabs(c->std * normal_at(s, 1)));
        bp[0] = (uint8_t)(d & 0xFF); bp[1] = (uint8_t)(d >> 8);
        bp[2] = (uint8_t)(dm & 0xFF); bp[3] = (uint8_t)(dm >> 8);
        uint64_t r1 = orc_rng_u64(s, 4), r2 = orc_rng_u64(s, 5);
        uint8_t sv[8], mv[8];
        for (int j = 0; j < 8; j++) { sv[j] = (uint8_t)((r1 >> (6 * j)) & 63); mv[j] = (uint8_t)((r2 >> (6 * j)) & 63); }
        orc_q4k_pack_scales(sv, mv, bp + 4);
        for (int w = 0; w < 16; w++) {
            uint64_t r = orc_rng_u64(s, 6 + (uint64_t)w);
            memcpy(bp + 16 + 8 * w, &r, 8);
        }
    }
}
void orc_synth_q4k(uint64_t seed, size_t n_blocks, float d_std, uint8_t *out)
{
    synth_ctx c = {seed, 0.0f, d_std, NULL, NULL, out};
    run_bands(n_blocks, 0, 4096, q4k_band, &c);
}
