/*
 * qgemv.h -- C ABI of the MI355X (gfx950) quantized mat-vec library
 * (rust-inference_amd/libqgemv.so).
 *
 * It replaces the wgpu backend of yudono/rust-inference on the path
 * QuantizedMatrix::mat_vec_mul (src/quant.rs:178-206) ->
 * GpuContext::mat_vec_mul (src/gpu_backend.rs:429-450).  Plain pointers and
 * sizes only.  Matrix types are the GGML ids of src/gguf.rs:43-59:
 * F32=0 F16=1 Q4_0=2 Q5_0=6 Q8_0=8 Q4_K=12 Q5_K=13 Q6_K=14 (Q4_1, Q5_1,
 * Q8_1, Q2_K, Q3_K are rejected, as src/model.rs:176-179 skips them).
 *
 * Layout: a matrix is the raw GGUF byte stream; element (r, c) is flat index
 * r*cols + c and block b starts at byte b*block_bytes (src/quant.rs:82-86,
 * 195-203).  Rows may straddle blocks (cols % block_elems != 0).
 *
 * Every function returns a qg_status (0 = QG_OK) and never aborts; a caller
 * maps a nonzero status to its CPU path, as the reference falls back to
 * fallback_cpu (src/gpu_backend.rs:438-447).  Contexts are not thread safe:
 * one per host thread, as the reference's GpuContext is !Sync
 * (src/gpu_backend.rs:17).  `stream` arguments are hipStream_t values passed
 * as void* (NULL = the context's own stream).
 */
#ifndef QGEMV_H
#define QGEMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum qg_status {
    QG_OK = 0,
    QG_ERR_INVALID_ARG = 1,      /* NULL pointer, bad device, misaligned buffer */
    QG_ERR_UNSUPPORTED_TYPE = 2, /* type id outside the supported set */
    QG_ERR_SHORT_DATA = 3,       /* fewer bytes than ceil(rows*cols/bs)*bb */
    QG_ERR_NO_DEVICE = 4,        /* no HIP device */
    QG_ERR_HIP = 5,              /* a HIP runtime call failed */
    QG_ERR_OUT_OF_MEMORY = 6,
    QG_ERR_SHAPE = 7             /* length / shape mismatch (quant.rs:179-180 asserts) */
} qg_status;

typedef struct qg_ctx qg_ctx;   /* one device + stream + staging buffers */
typedef struct qg_mat qg_mat;   /* one matrix resident in HBM */

/* Replaces GpuContext::try_init (src/gpu_backend.rs:317-348): opens HIP
 * device `device`, creates a stream.  QG_ERR_NO_DEVICE where the reference
 * returns None. */
int qg_init(int device, qg_ctx **out);
/* Releases the context (the reference drops GpuContext). Frees its matrices. */
int qg_destroy(qg_ctx *ctx);

/* Human-readable text for a status / the context's last error. */
const char *qg_status_string(int status);
const char *qg_last_error(const qg_ctx *ctx);

/* Replaces QuantizedMatrix::new (src/quant.rs:53-55) at the load_mat! site
 * (src/model.rs:197-203, lm_head 221-226): copies the raw GGUF bytes to HBM
 * once; they stay resident and are never expanded.  nbytes must cover
 * ceil(rows*cols/block_elems) blocks (extra bytes are ignored). */
int qg_upload(qg_ctx *ctx, const void *raw, size_t nbytes, uint32_t ggml_type,
              size_t rows, size_t cols, qg_mat **out);
/* Wraps bytes already in HBM (device pointer, at least 16-byte aligned,
 * followed by >= 512 readable bytes) without copying; the caller keeps them
 * alive for the handle's lifetime.  QG_ERR_INVALID_ARG when the device
 * allocation holding d_raw (hipMemGetAddressRange) ends less than 512 bytes
 * after the matrix's data, or when d_raw is in no allocation HIP knows. */
int qg_wrap_device(qg_ctx *ctx, const void *d_raw, size_t nbytes, uint32_t ggml_type,
                   size_t rows, size_t cols, qg_mat **out);
/* Frees a matrix.  QG_ERR_INVALID_ARG for a handle this context does not
 * hold (already freed, or another context's) and for a matrix a decode-step
 * model still uses through qg_model_share_matrix (destroy the model, or put
 * another matrix into its slot, first). */
int qg_mat_free(qg_ctx *ctx, qg_mat *mat);
int qg_mat_info(const qg_mat *mat, uint32_t *ggml_type, size_t *rows, size_t *cols,
                size_t *nbytes);
/* Kernel choice fixed at upload: 1 = stream kernel (fast path), 2 = the
 * stream kernel family with the LDS-ring kernel for the plain mat-vec
 * (repacked Q8_0 / Q4_K / Q5_K / Q6_K rows with several-wave teams that fit
 * its ring, e.g. the 14336- and 18944-wide down projections), 3 = the stream
 * kernel family with the wave-private column kernel for the plain mat-vec
 * (repacked Q4_K rows of 12288 or 14336 columns, at least 16 rows per compute
 * unit), 0 = generic per-element kernel
 * (cols % 32 != 0 and other shapes the planner rejects). */
int qg_mat_kernel_kind(const qg_mat *mat);

/* Device-resident mat-vec: y[r] = sum_c W[r,c] * x[c] (src/quant.rs:178-206).
 * d_x: cols floats, d_y: rows floats, both device pointers, 4-byte aligned.
 * A d_x that is not 16-byte aligned runs the generic kernel on matrices that
 * keep the GGUF layout; an uploaded Q8_0/Q4_K/Q5_K/Q6_K matrix keeps only
 * its repacked copy, so there x is first copied to an aligned buffer the
 * context owns: such calls on one context must not overlap (e.g. on two
 * streams), since they share that buffer and a longer x reallocates it.
 * Asynchronous on `stream`. */
int qg_matvec_dev(qg_ctx *ctx, const qg_mat *mat, const float *d_x, float *d_y, void *stream);

/* RmsNorm then mat_vec_mul, as every projection input of a decode step is
 * formed: y = W · (rmsnorm(xa + xb) * nw) (src/math.rs:237-257 as called by
 * src/rmsnorm.rs:14-29, the residual add of src/transformer.rs:31-46, then
 * src/quant.rs:178-206).  d_xb may be NULL (x = xa); d_sum_out, if not NULL,
 * receives xa + xb and must not overlap xa or xb.  xa, xb, nw, sum_out: cols
 * floats; y: rows floats; all device pointers, asynchronous on `stream`.
 * With 16-byte aligned vectors, a non-NULL d_xb and a stream-kernel matrix
 * the norm runs inside the mat-vec kernel; otherwise a separate RMSNorm kernel
 * writes the context's scratch vector first, so such calls on one context
 * must not overlap on different streams. */
int qg_matvec_norm_dev(qg_ctx *ctx, const qg_mat *mat, const float *d_xa, const float *d_xb,
                       const float *d_nw, float eps, float *d_sum_out, float *d_y, void *stream);

/* The MLP's gate and up projections with the SiLU product, from the norm of
 * the residual stream: h[j] = silu(gate_j · x) * (up_j · x) with
 * x = rmsnorm(xa + xb) * nw (src/mlp.rs:31-43 with silu as
 * src/math.rs:137-146, its input as in qg_matvec_norm_dev).  gu is the stacked
 * [gate; up] matrix (qg_mat_stack; 2 * H rows, gate rows first); h: H floats;
 * xa, xb, nw, sum_out as in qg_matvec_norm_dev.  With 16-byte aligned
 * vectors, a non-NULL d_xb, a quantized type and short rows (row groups of
 * at most 64 items: cols <= 8192 for Q4_K and <= 4096 for the other quant
 * types when a row is whole blocks) one kernel computes each gate row and its
 * up row back to back and writes h only; otherwise the [gate; up] outputs go to a context
 * scratch vector first (calls on one context must then not overlap on
 * different streams).  QG_ERR_SHAPE for an odd row count. */
int qg_matvec_norm_glu_dev(qg_ctx *ctx, const qg_mat *gu, const float *d_xa, const float *d_xb,
                           const float *d_nw, float eps, float *d_sum_out, float *d_h, void *stream);

/* No counterpart in the reference: qg_matvec_norm_glu_dev for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, kernels and
 * results; it calls no hipMalloc/hipFree.  Where its path needs scratch (the
 * normalised x and the [gate; up] outputs of the unfused path), it uses a
 * static 1 MiB device array that each GPU holds for the life of the process:
 * QG_ERR_SHAPE when round_up(cols, 64) + rows > 262144 floats.  All calls on
 * one GPU share that array and it keeps the last call's contents, so calls
 * that overlap on one GPU (other streams, other contexts, other host
 * threads) race; nothing in it needs to start at zero. */
int qg_matvec_norm_glu_dev_noalloc(qg_ctx *ctx, const qg_mat *gu, const float *d_xa, const float *d_xb,
                                   const float *d_nw, float eps, float *d_sum_out, float *d_h, void *stream);

/* One matrix whose rows are those of parts[0], parts[1], ... in order (the
 * same GGML type and cols; every part but the last a whole number of blocks),
 * as model.rs keeps wq/wk/wv and ffn_gate/ffn_up as separate
 * QuantizedMatrix values (src/model.rs:231-298) -- the stacked copy lets one
 * launch stream them together.  Synchronous device copies; the parts stay
 * valid.  Free with qg_mat_free. */
int qg_mat_stack(qg_ctx *ctx, qg_mat *const *parts, int n_parts, qg_mat **out);

/* The MLP's down projection input formed and consumed in one pass:
 * y = W · (silu(g) * u) (src/mlp.rs:36-45, silu as src/math.rs:137-146, then
 * src/quant.rs:178-206).  g, u: cols floats; y: rows floats; device pointers,
 * asynchronous on `stream`.  With 16-byte aligned g and u, at most 8192 cols
 * and a stream-kernel matrix the product is formed inside the mat-vec kernel;
 * otherwise a separate kernel writes the context's scratch vector first
 * (calls on one context must then not overlap on different streams). */
int qg_matvec_silu_dev(qg_ctx *ctx, const qg_mat *mat, const float *d_g, const float *d_u, float *d_y,
                       void *stream);

/* Host-buffer drop-in for QuantizedMatrix::mat_vec_mul(x, out, Some(gpu))
 * (src/quant.rs:178-186): synchronous; stages x/y through pinned buffers
 * allocated once per context.  x: cols floats, y: rows floats. */
int qg_matvec_host(qg_ctx *ctx, const qg_mat *mat, const float *x, float *y);

/* Exact drop-in for GpuContext::mat_vec_mul(weight_data, dtype, x, out, rows,
 * cols) (src/gpu_backend.rs:429-437), which uploads the current bytes on
 * every call (gpu_backend.rs:478-482).  Here device copies are keyed by
 * (weight_data, nbytes, dtype, rows, cols) and reused while a fingerprint of
 * the host bytes (64 bytes at 16 evenly spaced offsets, first and last
 * included) still matches the one taken at upload; on a mismatch the current
 * bytes are uploaded again.  A caller that edits weights in place where the
 * fingerprint does not look calls qg_gpu_invalidate first, or compares every
 * byte on every call (qg_gpu_set_freshness, QG_FRESH_EXACT).  On an error
 * `out` is left untouched. */
int qg_gpu_mat_vec_mul(qg_ctx *ctx, const void *weight_data, size_t nbytes, uint32_t dtype,
                       const float *x, float *out, size_t rows, size_t cols);
/* No counterpart in the reference (it keeps no device copies): drops every
 * device copy qg_gpu_mat_vec_mul keeps for host address `weight_data`. */
int qg_gpu_invalidate(qg_ctx *ctx, const void *weight_data);

/* How qg_gpu_mat_vec_mul decides that its device copy still holds the host
 * bytes.  No counterpart in the reference, which uploads on every call
 * (gpu_backend.rs:478-482):
 *   QG_FRESH_SAMPLED (the default): the 16-window fingerprint above;
 *   QG_FRESH_EXACT: the context keeps a host copy of every cached matrix's
 *     bytes and compares all of them on every call (memcmp), uploading again
 *     on any difference -- the reference's result for any in-place edit,
 *     with no qg_gpu_invalidate, at the cost of one host copy per cached
 *     matrix and a host compare of its bytes per call.
 * Copies made under the other mode are uploaded again on their next call.
 * Any other mode: QG_ERR_INVALID_ARG. */
enum { QG_FRESH_SAMPLED = 0, QG_FRESH_EXACT = 1 };
int qg_gpu_set_freshness(qg_ctx *ctx, int mode);

/* Arithmetic of this context's plain mat-vecs (qg_matvec_dev, qg_matvec_host,
 * qg_gpu_mat_vec_mul; the fused entry points and the decode step keep the
 * default).  No counterpart in the reference, whose loop rounds every product
 * w * x to f32 and sums in f32 (quant.rs:195-204):
 *   QG_PRECISION_FIXED22 (the default): x as 22-bit fixed point per
 *     32-element segment against exact integer sums of the weight codes --
 *     within 1e-4 normwise of the reference, but an element far below its
 *     segment's maximum keeps fewer bits (10^4 below: about 8), which shows
 *     where the maxima meet zero weights;
 *   QG_PRECISION_F32: every product rounded to f32 and summed in f32, one
 *     wave per row (the reference's per-product arithmetic, in another
 *     order), at several times the fixed-point kernels' time.
 * Any other mode: QG_ERR_INVALID_ARG. */
enum { QG_PRECISION_FIXED22 = 0, QG_PRECISION_F32 = 1 };
int qg_set_precision(qg_ctx *ctx, int mode);

/* Test hook, no counterpart in the reference: of the allocations this
 * context makes next (device matrices, repacked and stacked copies, pinned
 * and device staging), the first `skip` go through and the `n` after them
 * report QG_ERR_OUT_OF_MEMORY without calling HIP, so that tests can drive
 * the status-code path a caller maps to its CPU fallback
 * (gpu_backend.rs:444-447) without a device fault.  n = 0 switches it off. */
int qg_test_fail_allocations(qg_ctx *ctx, int skip, int n);

/* quant::dequantize (src/quant.rs:356-372) on device: rows*cols f32 values,
 * bit-exact with the CPU path.  The reference's Vec for Q4_K/Q5_K is padded
 * to whole blocks; only the first rows*cols values are written here. */
int qg_dequant_dev(qg_ctx *ctx, const qg_mat *mat, float *d_out, void *stream);
int qg_dequant_host(qg_ctx *ctx, const qg_mat *mat, float *out);

/* QuantizedMatrix::dequantize_row (src/quant.rs:152-174) on device, with the
 * reference's placement for rows that straddle blocks: only the positions the
 * reference writes are written (the caller zero-fills, as transformer.rs:74's
 * fresh vec! does). */
int qg_dequantize_row_dev(qg_ctx *ctx, const qg_mat *mat, size_t row, float *d_out,
                          void *stream);

/* Measurement only, no counterpart in the reference: n_launches calls of
 * qg_matvec_dev(ctx, mats[i % n_mats], d_x, d_y, stream), i = 0, 1, ..., issued
 * back to back from compiled code, as a Rust caller issues its mat-vecs
 * (a Python loop over the same calls is bound by its own per-call cost when a
 * launch takes less time than the interpreter).  Stops at the first error. */
int qg_matvec_dev_repeat(qg_ctx *ctx, const qg_mat *const *mats, size_t n_mats, const float *d_x, float *d_y,
                         size_t n_launches, void *stream);

/* Waits for all work on the context's stream. */
int qg_synchronize(qg_ctx *ctx);
/* The context's stream (a hipStream_t). */
void *qg_stream(qg_ctx *ctx);
/* Number of compute units of the context's device. */
int qg_device_cu_count(const qg_ctx *ctx);

#ifdef __cplusplus
}
#endif

#endif /* QGEMV_H */
