/*
 * oracle/qref.h -- CPU restatement of the reference's quantized mat-vec path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * implementation is compared against.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product library
 * (rust-inference_amd/libqgemv.so) never links, loads or calls it.
 *
 * Every function restates one function of yudono/rust-inference and cites the
 * reference file:line it follows.  Build flags (oracle/Makefile):
 * -O2 -ffp-contract=off -fno-fast-math, because rustc never contracts
 * a*b+c into an FMA and every f32 rounding below must happen where Rust's does.
 *
 * Pinning (what checks each function independently of this restatement):
 *   qref_fp16_to_fp32       exhaustive 65,536 patterns vs numpy float16->float32
 *   qref_get_scale_min_k4   exhaustive single-bit probes + bijection property
 *   qref_dequantize_block   hand-encoded known-answer blocks (tests/golden)
 *   qref_dequantize         equals per-block decode; short-data Err cases
 *   qref_mat_vec_mul        f64 brute force on tiny shapes, one-hot columns,
 *                           equality with qref_fallback_cpu (two reference paths)
 *   qref_mat_vec_mul_transposed  closed forms + f64 brute force
 *   qref_dequantize_row     straddle known-answer at cols=896 (source-only quirk)
 *   decode-step helpers     closed forms / numpy restatement of textbook ops
 */
#ifndef QREF_H
#define QREF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids, gguf.rs:43-59 */
enum {
    QREF_F32 = 0, QREF_F16 = 1, QREF_Q4_0 = 2, QREF_Q4_1 = 3, QREF_Q5_0 = 6,
    QREF_Q5_1 = 7, QREF_Q8_0 = 8, QREF_Q8_1 = 9, QREF_Q2_K = 10, QREF_Q3_K = 11,
    QREF_Q4_K = 12, QREF_Q5_K = 13, QREF_Q6_K = 14
};

/* quant.rs:57-65 / 67-79.  Returns 0 for an unknown id. */
size_t qref_block_size(uint32_t dtype);
size_t qref_block_bytes(uint32_t dtype);

/* quant.rs:302-342 */
float qref_fp16_to_fp32(uint16_t bits);

/* quant.rs:606-615; writes the 6-bit scale and min of sub-block j as f32 */
void qref_get_scale_min_k4(size_t j, const uint8_t *scales, float *sc, float *m);

/* quant.rs:82-149.  buf keeps prior contents where the reference leaves them
 * (short slices for F32/F16/Q8_0, unsupported types). */
void qref_dequantize_block(const uint8_t *data, size_t nbytes, uint32_t dtype,
                           size_t block_idx, float *buf);

/* quant.rs:356-840.  Returns the length of the reference's Vec<f32>
 * (n_blocks*256 for Q4_K/Q5_K, n_elements otherwise) and writes that many
 * floats to out (which must hold them), or returns -1 for the Err cases
 * (short data, unsupported type). */
long long qref_dequantize(const uint8_t *data, size_t nbytes, uint32_t dtype,
                          size_t n_elements, float *out);
/* Vec length qref_dequantize would produce (no data needed). */
size_t qref_dequantize_len(uint32_t dtype, size_t n_elements);

/* quant.rs:188-205: CPU branch of QuantizedMatrix::mat_vec_mul */
void qref_mat_vec_mul(const uint8_t *data, size_t nbytes, uint32_t dtype,
                      size_t rows, size_t cols, const float *x, float *out);

/* math.rs:191-209 */
void qref_mat_vec_mul_transposed(const float *w, const float *x, float *out,
                                 size_t out_dim, size_t in_dim);

/* gpu_backend.rs:556-567: dequantize + mat_vec_mul_transposed.  Returns 0,
 * or -1 where the reference panics (dequantize Err -> empty Vec, or a Vec
 * whose length is not rows*cols, tripping math.rs:198). */
int qref_fallback_cpu(const uint8_t *data, size_t nbytes, uint32_t dtype,
                      size_t rows, size_t cols, const float *x, float *out);

/* quant.rs:152-174, including the straddled-row placement quirk. */
void qref_dequantize_row(const uint8_t *data, size_t nbytes, uint32_t dtype,
                         size_t rows, size_t cols, size_t row, float *buf);

/* ---- decode-step helpers (transformer.rs / attention.rs / mlp.rs) ---- */

/* math.rs:237-256 */
void qref_rmsnorm(const float *x, const float *w, float *out, size_t n, float eps);
/* rmsnorm.rs:22-29 (forward_inplace) */
void qref_rmsnorm_inplace(float *x, const float *w, size_t n, float eps);
/* math.rs:135-146 */
float qref_silu(float x);
/* math.rs:104-118 */
void qref_softmax_inplace(float *a, size_t n);
/* math.rs:328-339 */
size_t qref_argmax(const float *a, size_t n);
/* rope.rs:42-63: fills cos/sin tables [max_seq_len * dim/2] */
void qref_rope_tables(size_t dim, float base, size_t max_seq_len, float *cos_t, float *sin_t);
/* rope.rs:68-97 */
void qref_rope_apply(float *x, size_t dim, size_t position, const float *cos_t,
                     const float *sin_t, size_t max_pos);
/* sampler.rs:109-127 (penalty 1.1, window 64 in main.rs:187-188) */
void qref_repetition_penalty(float *logits, size_t vocab, const size_t *recent,
                             size_t n_recent, float penalty, size_t window);

#ifdef __cplusplus
}
#endif

#endif /* QREF_H */
