// qg_internal.h -- library-internal view of the C ABI's opaque handles,
// shared by qgemv_api.cpp and the decode-step engine (qg_model.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <map>
#include <set>
#include <string>
#include <tuple>
#include <vector>

#include "qg_common.h"
#include "qgemv.h"

struct qg_model;

struct qg_mat {
    qg_ctx *ctx;
    uint8_t *d;        // device bytes in the GGUF layout (nbytes data + kTailPad zeros), or NULL:
                       // an owned repacked matrix keeps only d_rp (qg_mat_gguf rebuilds the
                       // GGUF layout where a kernel needs it; qg_mat_keep_gguf keeps it)
    uint8_t *d_rp;     // the matrix in the repacked layout (owned Q8_0/Q4_K/Q5_K/Q6_K), or NULL
    size_t nbytes;     // bytes the kernels may treat as data
    uint32_t type;
    size_t rows, cols;
    bool owned;
    bool rp_view = false;  // d_rp points into a stacked matrix's repacked copy (not owned)
    int shares = 0;    // decode-step models using this matrix without owning it
    qg::Plan plan;     // plan.rp: the stream kernels read d_rp
};

// The bytes the stream GEMV kernels read (the dequant and generic kernels
// read the GGUF layout: d, or qg_mat_gguf).
inline const uint8_t *qg_gemv_bytes(const qg_mat *m) { return m->plan.rp ? m->d_rp : m->d; }

// Device bytes of the matrix (both layouts it holds, tail pads included).
inline size_t qg_mat_resident(const qg_mat *m)
{
    const size_t one = m->nbytes + qg::kTailPad;
    return (m->owned && m->d ? one : 0) + (m->d_rp && !m->rp_view ? one : 0);
}

struct qg_ctx {
    int device = 0;
    int n_cu = 0;
    hipStream_t stream = nullptr;
    std::string err;
    float *h_x = nullptr, *h_y = nullptr;   // pinned staging
    size_t h_x_cap = 0, h_y_cap = 0;
    float *d_x = nullptr, *d_y = nullptr;   // device staging
    size_t d_x_cap = 0, d_y_cap = 0;
    float *d_norm = nullptr;                // normalised x of qg_matvec_norm_dev's two-kernel path
    size_t d_norm_cap = 0;
    float *d_glu = nullptr;                 // gate and up outputs of qg_matvec_norm_glu_dev's unfused path
    size_t d_glu_cap = 0;
    float *d_xal = nullptr;                 // 16-byte aligned copy of an unaligned x (repacked-only matrices)
    size_t d_xal_cap = 0;
    // device address of this GPU's static scratch array (qg_matvec_norm_glu_dev_noalloc),
    // resolved once in qg_init; NULL if the runtime could not resolve it
    float *d_static_scratch = nullptr;
    std::set<qg_mat *> mats;
    std::set<qg_model *> models;            // decode-step engines on this context
    // qg_gpu_mat_vec_mul's device copies, keyed by (host address, bytes, type,
    // rows, cols), each with the host bytes it was made from: a fingerprint
    // (sampled windows), or all of them (exact, then fp.size() == the
    // matrix's bytes)
    struct Keyed {
        qg_mat *mat;
        std::vector<uint8_t> fp;
        bool exact;
    };
    std::map<std::tuple<uintptr_t, size_t, uint32_t, size_t, size_t>, Keyed> keyed;
    bool fresh_exact = false;               // qg_gpu_set_freshness(QG_FRESH_EXACT)
    bool prec_f32 = false;                  // qg_set_precision(QG_PRECISION_F32)
    int fail_skip = 0, fail_allocs = 0;     // test hook: allocations to let through, then to fail
};

// Test hook (qg_test_fail_allocations): true when this allocation is to be
// reported as failed without calling HIP.
inline bool qg_alloc_injected(qg_ctx *ctx)
{
    if (!ctx || ctx->fail_allocs <= 0) return false;
    if (ctx->fail_skip > 0) {
        ctx->fail_skip--;
        return false;
    }
    ctx->fail_allocs--;
    return true;
}

// check_mat of the C ABI: ctx valid and mat one of its live matrices.
int qg_check_mat(qg_ctx *ctx, const qg_mat *mat);

// The matrix in the GGUF layout: *out = mat->d (*temp = false), or a new
// device allocation (nbytes + kTailPad, *temp = true, the caller frees it)
// rebuilt from the repacked copy.  Synchronous.
int qg_mat_gguf(qg_ctx *ctx, const qg_mat *mat, uint8_t **out, bool *temp);
// Keep a GGUF-layout copy (rebuilt from the repacked copy if d is NULL).
int qg_mat_keep_gguf(qg_ctx *ctx, qg_mat *mat);
// Drop the repacked copy of a matrix that keeps its GGUF layout (the kernels
// of the GGUF layout serve it from then on).
int qg_mat_drop_repacked(qg_ctx *ctx, qg_mat *mat);

// The model-owned or shared matrix `mat` is no longer used by a model slot.
int qg_mat_release(qg_ctx *ctx, qg_mat *mat, bool owned);

struct qg_model;
// Frees every decode-step engine of the context (qg_model.hip); qg_destroy
// calls it before freeing the context's matrices.
void qg_models_free_all(qg_ctx *ctx);

// y = W · (rmsnorm(xa + xb) * nw), sum_out (may be NULL) = xa + xb (xb may be
// NULL: then xa alone).  The stream kernel does the norm in its prologue when
// the plan and the pointers allow; otherwise a one-workgroup RMSNorm kernel
// writes `scratch` (cols floats) and the mat-vec reads it.  Asynchronous.
int qg_norm_matvec(qg_ctx *ctx, const qg_mat *mat, const float *xa, const float *xb, const float *nw,
                   float eps, float *sum_out, float *y, float *scratch, hipStream_t stream);

// y = W · (silu(g) * u): the product inside the stream kernel's prologue, or
// a separate kernel into `scratch` (cols floats) when that does not apply.
int qg_silu_matvec(qg_ctx *ctx, const qg_mat *mat, const float *g, const float *u, float *y, float *scratch,
                   hipStream_t stream);

// h = silu(gate · x) * (up · x), x = rmsnorm(xa + xb) * nw, for the stacked
// gu = [gate; up] (rows = 2 * rows(h)): one stream kernel that pairs the rows
// when the plan and pointers allow; otherwise the norm mat-vec of gu into
// gu_out (rows floats; its norm scratch is `scratch`, cols floats) and a
// silu * up kernel.  Asynchronous.
int qg_norm_glu_matvec(qg_ctx *ctx, const qg_mat *gu, const float *xa, const float *xb, const float *nw,
                       float eps, float *sum_out, float *h, float *gu_out, float *scratch, hipStream_t stream);

// y1 = W1 · x, y2 = W2 · x with x = rmsnorm(xa + xb) * nw (same cols): one
// launch when the pair is supported and the pointers are 16-byte aligned;
// otherwise two qg_norm_matvec calls (scratch: cols floats).  sum_out (may be
// NULL) = xa + xb.  Asynchronous.
int qg_norm_pair_matvec(qg_ctx *ctx, const qg_mat *m1, const qg_mat *m2, const float *xa, const float *xb,
                        const float *nw, float eps, float *sum_out, float *y1, float *y2, float *scratch,
                        hipStream_t stream);

// One owned matrix whose rows are the rows of parts[0], parts[1], ... (same
// type and cols; every part but the last a whole number of blocks): device
// copies of the parts' blocks, one after the other.  Synchronous.
int qg_stack_mats(qg_ctx *ctx, qg_mat *const *parts, int n, qg_mat **out);

// The same stacked matrix without a second copy of the parts: parts that
// hold only a repacked copy (not a view), all with one row-group layout
// (same g, ni, group_bytes; whole groups), are copied into one allocation
// -- the repacked layout of stacked rows is the parts' repacked bytes one
// after the other -- and become views into it (rp_view; their own copies
// are freed).  QG_ERR_SHAPE (nothing changed) when the parts do not qualify.
// Synchronous.
int qg_stack_views(qg_ctx *ctx, qg_mat *const *parts, int n, qg_mat **out);
// A view part gets its own repacked copy again (before its stack is freed).
int qg_mat_unview(qg_ctx *ctx, qg_mat *mat);

// lm_head = the model's token_embd device matrix (a tied output, model.rs:224-226).
int qg_model_tie_lm_head(qg_model *m);

// Records `what` (and the HIP error text) as the context's last error; returns `status`.
int qg_fail(qg_ctx *ctx, int status, const char *what, hipError_t e = hipSuccess);
