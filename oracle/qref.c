/*
 * oracle/qref.c -- CPU restatement of yudono/rust-inference's quantized
 * mat-vec path (src/quant.rs, src/math.rs, src/gpu_backend.rs fallback).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never the product.
 * See qref.h for the per-function pins.  Compiled with -ffp-contract=off so
 * that every multiply and add rounds separately, as rustc emits them.
 */
#include "qref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* quant.rs:57-65 */
size_t qref_block_size(uint32_t dtype)
{
    switch (dtype) {
    case QREF_Q4_0: case QREF_Q8_0: case QREF_Q5_0: return 32;
    case QREF_Q4_K: case QREF_Q5_K: case QREF_Q6_K: return 256;
    case QREF_F32: case QREF_F16: return 1;
    case QREF_Q4_1: case QREF_Q5_1: case QREF_Q8_1: case QREF_Q2_K: case QREF_Q3_K: return 256;
    default: return 0;
    }
}

/* quant.rs:67-79 */
size_t qref_block_bytes(uint32_t dtype)
{
    switch (dtype) {
    case QREF_F32: return 4;
    case QREF_F16: return 2;
    case QREF_Q8_0: return 34;
    case QREF_Q4_0: return 18;
    case QREF_Q5_0: return 22;
    case QREF_Q4_K: return 144;
    case QREF_Q5_K: return 176;
    case QREF_Q6_K: return 210;
    default: return 0;
    }
}

static float bits_to_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }

/* Rust's 2.0f32.powi(e) for the exponents used here (-14..15) is an exact
 * power of two; ldexpf gives the same exact value. */
static float pow2i(int e) { return ldexpf(1.0f, e); }

/* quant.rs:302-342 */
float qref_fp16_to_fp32(uint16_t bits)
{
    uint32_t sign = (bits >> 15) & 1u;
    int exp = (int)((bits >> 10) & 0x1Fu);
    uint32_t mantissa = bits & 0x3FFu;

    if (exp == 0) {
        if (mantissa == 0)
            return sign == 1 ? -0.0f : 0.0f;
        float value = (float)mantissa / 1024.0f;      /* quant.rs:313 */
        int e = 1 - 15;
        value = value * pow2i(e);                      /* quant.rs:315 */
        return sign == 1 ? -value : value;
    }
    if (exp == 31) {
        if (mantissa == 0)
            return sign == 1 ? -INFINITY : INFINITY;
        return bits_to_f32(0x7FC00000u);               /* f32::NAN, quant.rs:328 */
    }
    int e = exp - 15;
    float m = 1.0f + (float)mantissa / 1024.0f;        /* quant.rs:334 */
    float value = m * pow2i(e);
    return sign == 1 ? -value : value;
}

/* quant.rs:344-348 */
static float read_fp16_le(const uint8_t *b)
{
    return qref_fp16_to_fp32((uint16_t)(b[0] | (b[1] << 8)));
}

/* quant.rs:606-615 */
void qref_get_scale_min_k4(size_t j, const uint8_t *scales, float *sc, float *m)
{
    uint8_t s6, m6;
    if (j < 4) {
        s6 = scales[j] & 63;
        m6 = scales[j + 4] & 63;
    } else {
        s6 = (uint8_t)((scales[j + 4] & 0x0F) | ((scales[j - 4] >> 6) << 4));
        m6 = (uint8_t)((scales[j + 4] >> 4) | ((scales[j] >> 6) << 4));
    }
    *sc = (float)s6;
    *m = (float)m6;
}

/* quant.rs:210-228 */
static void dequant_q4_k_block(const uint8_t *s, float *buf)
{
    float d = read_fp16_le(s);
    float dmin = read_fp16_le(s + 2);
    const uint8_t *scales = s + 4;
    const uint8_t *qs = s + 16;
    size_t is = 0;
    for (int j = 0; j < 256; j += 64) {
        float sc0, m0, sc1, m1v;
        qref_get_scale_min_k4(is, scales, &sc0, &m0);
        float d1 = d * sc0;
        float m1 = dmin * m0;
        qref_get_scale_min_k4(is + 1, scales, &sc1, &m1v);
        float d2 = d * sc1;
        float m2 = dmin * m1v;
        const uint8_t *q = qs + (is / 2) * 32;
        for (int l = 0; l < 32; l++) buf[is / 2 * 64 + l] = d1 * (float)(q[l] & 0x0F) - m1;
        for (int l = 0; l < 32; l++) buf[is / 2 * 64 + 32 + l] = d2 * (float)((q[l] >> 4) & 0x0F) - m2;
        is += 2;
    }
}

/* quant.rs:231-262 */
static void dequant_q5_k_block(const uint8_t *s, float *buf)
{
    float d = read_fp16_le(s);
    float dmin = read_fp16_le(s + 2);
    const uint8_t *scales = s + 4;
    const uint8_t *qh = s + 16;
    const uint8_t *qs = s + 48;
    size_t is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < 256; j += 64) {
        float sc0, m0, sc1, m1v;
        qref_get_scale_min_k4(is, scales, &sc0, &m0);
        float d1 = d * sc0;
        float m1 = dmin * m0;
        qref_get_scale_min_k4(is + 1, scales, &sc1, &m1v);
        float d2 = d * sc1;
        float m2 = dmin * m1v;
        const uint8_t *ql = qs + (is / 2) * 32;
        for (int l = 0; l < 32; l++) {
            int lo = ql[l] & 0x0F;
            int hi = (qh[l] & u1) ? 16 : 0;
            buf[is / 2 * 64 + l] = d1 * (float)(lo + hi) - m1;
        }
        for (int l = 0; l < 32; l++) {
            int lo = ql[l] >> 4;
            int hi = (qh[l] & u2) ? 16 : 0;
            buf[is / 2 * 64 + 32 + l] = d2 * (float)(lo + hi) - m2;
        }
        is += 2;
        u1 = (uint8_t)(u1 << 2);
        u2 = (uint8_t)(u2 << 2);
    }
}

/* quant.rs:265-292 */
static void dequant_q6_k_block(const uint8_t *s, float *buf)
{
    const uint8_t *ql = s;
    const uint8_t *qh = s + 128;
    const uint8_t *sc_raw = s + 192;
    float d = read_fp16_le(s + 208);
    for (int n = 0; n < 256; n += 128) {
        int iter = n / 128;
        const uint8_t *ql_i = ql + iter * 64;
        const uint8_t *qh_i = qh + iter * 32;
        const uint8_t *sc_i = sc_raw + iter * 8;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (ql_i[l] & 0x0F) | (((qh_i[l] >> 0) & 3) << 4);
            int q2 = (ql_i[l + 32] & 0x0F) | (((qh_i[l] >> 2) & 3) << 4);
            int q3 = (ql_i[l] >> 4) | (((qh_i[l] >> 4) & 3) << 4);
            int q4 = (ql_i[l + 32] >> 4) | (((qh_i[l] >> 6) & 3) << 4);
            float sc0 = (float)(int8_t)sc_i[is + 0];
            float sc2 = (float)(int8_t)sc_i[is + 2];
            float sc4 = (float)(int8_t)sc_i[is + 4];
            float sc6 = (float)(int8_t)sc_i[is + 6];
            buf[n + l] = d * sc0 * (float)(q1 - 32);
            buf[n + l + 32] = d * sc2 * (float)(q2 - 32);
            buf[n + l + 64] = d * sc4 * (float)(q3 - 32);
            buf[n + l + 96] = d * sc6 * (float)(q4 - 32);
        }
    }
}

/* quant.rs:82-149 */
void qref_dequantize_block(const uint8_t *data, size_t nbytes, uint32_t dtype,
                           size_t block_idx, float *buf)
{
    size_t bs = qref_block_size(dtype);
    size_t bb = qref_block_bytes(dtype);
    size_t offset = block_idx * bb;
    size_t start = offset < nbytes ? offset : nbytes;     /* quant.rs:86 */
    const uint8_t *s = data + start;
    size_t slen = nbytes - start;

    switch (dtype) {
    case QREF_F32:
        for (size_t i = 0; i < bs; i++) {
            size_t off = i * 4;
            if (off + 3 < slen) {
                uint32_t bits = (uint32_t)s[off] | ((uint32_t)s[off + 1] << 8) |
                                ((uint32_t)s[off + 2] << 16) | ((uint32_t)s[off + 3] << 24);
                buf[i] = bits_to_f32(bits);
            }
        }
        break;
    case QREF_F16:
        for (size_t i = 0; i < bs; i++) {
            size_t off = i * 2;
            if (off + 1 < slen) buf[i] = read_fp16_le(s + off);
        }
        break;
    case QREF_Q8_0: {
        float d = read_fp16_le(s);
        for (size_t i = 0; i < bs; i++) {
            if (i < (slen >= 2 ? slen - 2 : 0))
                buf[i] = d * (float)(int8_t)s[2 + i];
        }
        break;
    }
    case QREF_Q4_0: {
        float d = read_fp16_le(s);
        for (size_t i = 0; i < bs; i++) {
            uint8_t byte_val = s[2 + i / 2];
            uint8_t nibble = (i % 2 == 0) ? (byte_val & 0x0F) : ((byte_val >> 4) & 0x0F);
            buf[i] = d * (float)((int8_t)nibble - 8);
        }
        break;
    }
    case QREF_Q5_0: {
        float d = read_fp16_le(s);
        uint32_t qh = (uint32_t)s[2] | ((uint32_t)s[3] << 8) | ((uint32_t)s[4] << 16) |
                      ((uint32_t)s[5] << 24);
        const uint8_t *qs = s + 6;
        for (int i = 0; i < 16; i++) {
            uint8_t xl = qs[i] & 0x0F;
            uint8_t xh = (uint8_t)(((qh >> i) & 1u) << 4);
            buf[i] = d * (float)((int8_t)(xl | xh) - 16);
        }
        for (int i = 16; i < 32; i++) {
            uint8_t xl = qs[i - 16] >> 4;
            uint8_t xh = (uint8_t)(((qh >> i) & 1u) << 4);
            buf[i] = d * (float)((int8_t)(xl | xh) - 16);
        }
        break;
    }
    case QREF_Q4_K: dequant_q4_k_block(s, buf); break;
    case QREF_Q5_K: dequant_q5_k_block(s, buf); break;
    case QREF_Q6_K: dequant_q6_k_block(s, buf); break;
    default: break; /* unsupported: leave buf as is (quant.rs:146-147) */
    }
}

size_t qref_dequantize_len(uint32_t dtype, size_t n)
{
    if (dtype == QREF_Q4_K || dtype == QREF_Q5_K)        /* quant.rs:640-666, 714-749 */
        return (n + 255) / 256 * 256;
    return n;
}

/* quant.rs:356-840.  The per-type bodies of dequantize_* compute the same
 * per-element values as dequantize_block (compare quant.rs:453-454 with 110,
 * 494-501 with 117-119, 565-579 with 126-135, 640-666 with 210-228, 714-749
 * with 231-262, 806-836 with 271-291), so they are restated by decoding whole
 * blocks and keeping the Vec length each body produces. */
long long qref_dequantize(const uint8_t *data, size_t nbytes, uint32_t dtype,
                          size_t n_elements, float *out)
{
    size_t bs = qref_block_size(dtype), bb = qref_block_bytes(dtype);
    switch (dtype) {
    case QREF_F32: case QREF_F16: case QREF_Q8_0: case QREF_Q4_0:
    case QREF_Q5_0: case QREF_Q4_K: case QREF_Q5_K: case QREF_Q6_K: break;
    default: return -1;                                      /* quant.rs:370 */
    }
    size_t n_blocks = (n_elements + bs - 1) / bs;
    if (nbytes < n_blocks * bb) return -1;                   /* short data -> Err */
    size_t len = qref_dequantize_len(dtype, n_elements);
    float buf[256];
    for (size_t b = 0; b < n_blocks; b++) {
        memset(buf, 0, sizeof buf);
        qref_dequantize_block(data, nbytes, dtype, b, buf);
        size_t base = b * bs;
        for (size_t i = 0; i < bs && base + i < len; i++) out[base + i] = buf[i];
    }
    return (long long)len;
}

/* quant.rs:188-205 */
void qref_mat_vec_mul(const uint8_t *data, size_t nbytes, uint32_t dtype,
                      size_t rows, size_t cols, const float *x, float *out)
{
    for (size_t r = 0; r < rows; r++) out[r] = 0.0f;          /* out.fill(0.0) */
    size_t total = rows * cols;
    size_t bs = qref_block_size(dtype);
    if (bs == 0) return;
    size_t n_blocks = (total + bs - 1) / bs;
    float block_buf[256];
    memset(block_buf, 0, sizeof block_buf);                   /* vec![0.0; bs] */
    for (size_t b = 0; b < n_blocks; b++) {
        qref_dequantize_block(data, nbytes, dtype, b, block_buf);
        size_t start = b * bs;
        size_t end = start + bs < total ? start + bs : total;
        for (size_t k = 0; k < end - start; k++) {
            size_t flat = start + k;
            size_t col = flat % cols;
            size_t row = flat / cols;
            out[row] += block_buf[k] * x[col];
        }
    }
}

/* math.rs:191-209 */
void qref_mat_vec_mul_transposed(const float *w, const float *x, float *out,
                                 size_t out_dim, size_t in_dim)
{
    for (size_t i = 0; i < out_dim; i++) {
        float sum = 0.0f;
        for (size_t j = 0; j < in_dim; j++) sum += w[j + in_dim * i] * x[j];
        out[i] = sum;
    }
}

/* gpu_backend.rs:556-567 */
int qref_fallback_cpu(const uint8_t *data, size_t nbytes, uint32_t dtype,
                      size_t rows, size_t cols, const float *x, float *out)
{
    size_t n = rows * cols;
    size_t len = qref_dequantize_len(dtype, n);
    float *w = (float *)malloc((len ? len : 1) * sizeof(float));
    if (!w) return -2;
    long long got = qref_dequantize(data, nbytes, dtype, n, w);
    int rc = 0;
    if (got < 0 || (size_t)got != n)   /* unwrap_or_default -> len 0, or length assert */
        rc = -1;                       /* math.rs:198 assert_eq! panics */
    else
        qref_mat_vec_mul_transposed(w, x, out, rows, cols);
    free(w);
    return rc;
}

/* quant.rs:152-174 */
void qref_dequantize_row(const uint8_t *data, size_t nbytes, uint32_t dtype,
                         size_t rows, size_t cols, size_t row, float *buf)
{
    size_t bs = qref_block_size(dtype);
    size_t n_blocks_per_row = (cols + bs - 1) / bs;
    size_t start_block = (row * cols) / bs;
    size_t col_offset = (row * cols) % bs;
    float block_buf[256];
    memset(block_buf, 0, sizeof block_buf);
    for (size_t bi = 0; bi < n_blocks_per_row; bi++) {
        size_t block_idx = start_block + bi;
        if (block_idx * bs >= rows * cols) break;
        qref_dequantize_block(data, nbytes, dtype, block_idx, block_buf);
        size_t src_start = bi == 0 ? col_offset : 0;
        size_t lim = cols + col_offset - bi * bs;
        size_t src_end = bs < lim ? bs : lim;
        for (size_t k = src_start; k < src_end; k++) {
            size_t dst = bi == 0 ? k - col_offset : bi * bs + k;   /* quant.rs:168 */
            if (dst < cols) buf[dst] = block_buf[k];
        }
    }
}

/* ---------------- decode-step helpers ---------------- */

/* math.rs:237-256 */
void qref_rmsnorm(const float *x, const float *w, float *out, size_t n, float eps)
{
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    float rms = sqrtf(ss / (float)n + eps);
    float scale = 1.0f / rms;
    for (size_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* rmsnorm.rs:22-29 */
void qref_rmsnorm_inplace(float *x, const float *w, size_t n, float eps)
{
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    float rms = sqrtf(ss / (float)n + eps);
    float scale = 1.0f / rms;
    for (size_t i = 0; i < n; i++) x[i] = x[i] * scale * w[i];
}

/* math.rs:135-146 */
float qref_silu(float x)
{
    if (x >= 0.0f) {
        float e = expf(-x);
        return x / (1.0f + e);
    }
    float e = expf(x);
    return x * e / (1.0f + e);
}

/* math.rs:104-118; the max fold uses f32::max, which ignores NaN */
void qref_softmax_inplace(float *a, size_t n)
{
    if (n == 0) return;
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = fmaxf(mx, a[i]);
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) { a[i] = expf(a[i] - mx); s += a[i]; }
    float inv = 1.0f / s;
    for (size_t i = 0; i < n; i++) a[i] *= inv;
}

/* math.rs:328-339: first maximum wins */
size_t qref_argmax(const float *a, size_t n)
{
    size_t idx = 0;
    float mv = a[0];
    for (size_t i = 1; i < n; i++)
        if (a[i] > mv) { mv = a[i]; idx = i; }
    return idx;
}

/* rope.rs:42-63 */
void qref_rope_tables(size_t dim, float base, size_t max_seq_len, float *cos_t, float *sin_t)
{
    size_t half = dim / 2;
    for (size_t pos = 0; pos < max_seq_len; pos++)
        for (size_t i = 0; i < half; i++) {
            float exponent = (float)(2 * i) / (float)dim;
            float theta = 1.0f / powf(base, exponent);
            float angle = (float)pos * theta;
            cos_t[pos * half + i] = cosf(angle);
            sin_t[pos * half + i] = sinf(angle);
        }
}

/* rope.rs:68-97 */
void qref_rope_apply(float *x, size_t dim, size_t position, const float *cos_t,
                     const float *sin_t, size_t max_pos)
{
    size_t half = dim / 2;
    if (position >= max_pos) {                      /* rope.rs:71-86 */
        float base = 10000.0f;
        for (size_t i = 0; i < half; i++) {
            float exponent = (float)(2 * i) / (float)(half * 2);
            float theta = 1.0f / powf(base, exponent);
            float angle = (float)position * theta;
            float c = cosf(angle), s = sinf(angle);
            float x0 = x[2 * i], x1 = x[2 * i + 1];
            x[2 * i] = x0 * c - x1 * s;
            x[2 * i + 1] = x0 * s + x1 * c;
        }
        return;
    }
    size_t b = position * half;
    for (size_t i = 0; i < half; i++) {
        float c = cos_t[b + i], s = sin_t[b + i];
        float x0 = x[2 * i], x1 = x[2 * i + 1];
        x[2 * i] = x0 * c - x1 * s;
        x[2 * i + 1] = x0 * s + x1 * c;
    }
}

/* sampler.rs:109-127 */
void qref_repetition_penalty(float *logits, size_t vocab, const size_t *recent,
                             size_t n_recent, float penalty, size_t window)
{
    size_t start = n_recent > window ? n_recent - window : 0;
    for (size_t k = start; k < n_recent; k++) {
        size_t t = recent[k];
        if (t < vocab) {
            if (logits[t] > 0.0f) logits[t] /= penalty;
            else logits[t] *= penalty;
        }
    }
}
