// qgemv_api.cpp -- the C ABI of include/qgemv.h on HIP.
//
// Replaces yudono/rust-inference's GpuContext (src/gpu_backend.rs:14-18,
// 315-567).  Where the reference creates five wgpu buffers and re-uploads the
// whole weight matrix on every call (gpu_backend.rs:468-514) and then blocks
// on a staging readback (525-540), this keeps each matrix resident in HBM
// from upload on, and stages host vectors through pinned buffers allocated
// once per context.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <new>
#include <set>
#include <string>
#include <tuple>
#include <vector>

#include "qg_common.h"
#include "qg_internal.h"
#include "qgemv.h"

int qg_fail(qg_ctx *ctx, int status, const char *what, hipError_t e)
{
    if (ctx) {
        char buf[256];
        if (e != hipSuccess)
            snprintf(buf, sizeof buf, "%s: %s", what, hipGetErrorString(e));
        else
            snprintf(buf, sizeof buf, "%s", what);
        ctx->err = buf;
    }
    return status;
}

namespace {

int fail(qg_ctx *ctx, int status, const char *what, hipError_t e = hipSuccess)
{
    return qg_fail(ctx, status, what, e);
}

#define QG_HIP(ctx, call)                                                   \
    do {                                                                    \
        hipError_t e_ = (call);                                             \
        if (e_ != hipSuccess) return fail((ctx), QG_ERR_HIP, #call, e_);    \
    } while (0)

bool mul_overflows(size_t a, size_t b, size_t *out)
{
    if (a != 0 && b > SIZE_MAX / a) return true;
    *out = a * b;
    return false;
}

// Bytes a rows x cols matrix of `type` occupies: ceil(rows*cols/bs)*bb.
int required_bytes(uint32_t type, size_t rows, size_t cols, size_t *need)
{
    if (!qg::type_supported(type)) return QG_ERR_UNSUPPORTED_TYPE;
    size_t n;
    if (mul_overflows(rows, cols, &n)) return QG_ERR_SHAPE;
    const size_t bs = qg::block_elems(type), bb = qg::block_bytes(type);
    size_t nb = n / bs + (n % bs != 0);
    if (mul_overflows(nb, bb, need)) return QG_ERR_SHAPE;
    return QG_OK;
}

hipStream_t pick(qg_ctx *ctx, void *stream)
{
    return stream ? (hipStream_t)stream : ctx->stream;
}

int grow_pinned(qg_ctx *ctx, float **p, size_t *cap, size_t n)
{
    if (*cap >= n) return QG_OK;
    if (qg_alloc_injected(ctx)) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipHostMalloc (injected failure)");
    if (*p) (void)hipHostFree(*p);
    *p = nullptr;
    *cap = 0;
    hipError_t e = hipHostMalloc((void **)p, (n ? n : 1) * sizeof(float), hipHostMallocDefault);
    if (e != hipSuccess) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipHostMalloc", e);
    *cap = n;
    return QG_OK;
}

int grow_device(qg_ctx *ctx, float **p, size_t *cap, size_t n)
{
    if (*cap >= n) return QG_OK;
    if (qg_alloc_injected(ctx)) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipMalloc staging (injected failure)");
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    hipError_t e = hipMalloc((void **)p, (n ? n : 1) * sizeof(float));
    if (e != hipSuccess) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipMalloc staging", e);
    *cap = n;
    return QG_OK;
}

int new_mat(qg_ctx *ctx, uint8_t *d, size_t nbytes, uint32_t type, size_t rows, size_t cols,
            bool owned, qg_mat **out)
{
    qg_mat *m = new (std::nothrow) qg_mat;
    if (!m) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "host allocation");
    m->ctx = ctx;
    m->d = d;
    m->nbytes = nbytes;
    m->type = type;
    m->rows = rows;
    m->cols = cols;
    m->owned = owned;
    m->d_rp = nullptr;
    if (qg::make_plan(type, rows, cols, ctx->n_cu, &m->plan) != 0) {
        delete m;
        return fail(ctx, QG_ERR_UNSUPPORTED_TYPE, "no kernel for type");
    }
    // Owned Q8_0 / Q4_K / Q5_K / Q6_K matrices are kept in the repacked layout
    // the stream kernels read with contiguous loads (the same bytes -- for
    // Q5_K the same bits -- rearranged), and only in it: d is freed, and the
    // dequant kernels get the GGUF layout back from qg_mat_gguf.  Bytes
    // wrapped from caller memory keep the GGUF-layout kernels.
    if (owned && qg::repack_eligible(type, m->plan, rows)) {
        uint8_t *r = nullptr;
        hipError_t e = qg_alloc_injected(ctx) ? hipErrorOutOfMemory : hipMalloc((void **)&r, nbytes + qg::kTailPad);
        if (e != hipSuccess) {
            delete m;
            return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipMalloc repacked matrix", e);
        }
        qg::Plan rp_plan;
        int lr = qg::launch_repack(type, m->plan, d, r, (ihipStream_t *)ctx->stream);
        if (lr == 0) e = hipMemsetAsync(r + nbytes, 0, qg::kTailPad, ctx->stream);
        if (lr == 0 && e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (lr != 0 || e != hipSuccess || qg::make_plan(type, rows, cols, ctx->n_cu, &rp_plan, true) != 0 ||
            !rp_plan.rp) {
            (void)hipFree(r);
            delete m;
            return fail(ctx, QG_ERR_HIP, "repacking the matrix", e != hipSuccess ? e : hipGetLastError());
        }
        m->d_rp = r;
        m->plan = rp_plan;
        // one device copy: the kernels that need the GGUF layout rebuild it
        // (qg_mat_gguf)
        (void)hipFree(d);
        m->d = nullptr;
    }
    ctx->mats.insert(m);
    *out = m;
    return QG_OK;
}

void drop_mat(qg_ctx *ctx, qg_mat *m)
{
    if (m->owned && m->d) (void)hipFree(m->d);
    if (m->d_rp && !m->rp_view) (void)hipFree(m->d_rp);
    ctx->mats.erase(m);
    for (auto it = ctx->keyed.begin(); it != ctx->keyed.end();) {
        if (it->second.mat == m)
            it = ctx->keyed.erase(it);
        else
            ++it;
    }
    delete m;
}

// A handle is valid while its context lists it: the set is consulted before
// the handle is read, so a freed or foreign handle is an error, not a read of
// freed memory.
int check_mat(qg_ctx *ctx, const qg_mat *mat)
{
    if (!ctx) return QG_ERR_INVALID_ARG;
    if (!mat || !ctx->mats.count(const_cast<qg_mat *>(mat)))
        return fail(ctx, QG_ERR_INVALID_ARG, "matrix not of this context (or already freed)");
    return QG_OK;
}

// Fingerprint of a host weight buffer for qg_gpu_mat_vec_mul's cache: 64
// bytes at each of 16 evenly spaced offsets (the first and the last 64 bytes
// among them), or the whole buffer when it is shorter than 1 KiB.
std::vector<uint8_t> fingerprint(const uint8_t *p, size_t n)
{
    constexpr size_t kWin = 64, kN = 16;
    if (n <= kWin * kN) return std::vector<uint8_t>(p, p + n);
    std::vector<uint8_t> fp(kWin * kN);
    for (size_t i = 0; i < kN; i++) {
        const size_t off = (n - kWin) / (kN - 1) * i + (i == kN - 1 ? (n - kWin) % (kN - 1) : 0);
        memcpy(fp.data() + i * kWin, p + off, kWin);
    }
    return fp;
}

}  // namespace

int qg_check_mat(qg_ctx *ctx, const qg_mat *mat) { return check_mat(ctx, mat); }

int qg_mat_gguf(qg_ctx *ctx, const qg_mat *mat, uint8_t **out, bool *temp)
{
    *out = nullptr;
    *temp = false;
    if (mat->d) {
        *out = mat->d;
        return QG_OK;
    }
    if (!mat->d_rp || !mat->plan.rp) return fail(ctx, QG_ERR_INVALID_ARG, "matrix holds no device copy");
    QG_HIP(ctx, hipSetDevice(ctx->device));
    uint8_t *d = nullptr;
    hipError_t e = qg_alloc_injected(ctx) ? hipErrorOutOfMemory : hipMalloc((void **)&d, mat->nbytes + qg::kTailPad);
    if (e != hipSuccess) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipMalloc GGUF-layout copy", e);
    const int lr = qg::launch_unrepack(mat->type, mat->plan, mat->d_rp, d, (ihipStream_t *)ctx->stream);
    if (lr == 0) e = hipMemsetAsync(d + mat->nbytes, 0, qg::kTailPad, ctx->stream);
    if (lr == 0 && e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (lr != 0 || e != hipSuccess) {
        (void)hipFree(d);
        return fail(ctx, QG_ERR_HIP, "rebuilding the GGUF layout", e != hipSuccess ? e : hipGetLastError());
    }
    *out = d;
    *temp = true;
    return QG_OK;
}

int qg_mat_keep_gguf(qg_ctx *ctx, qg_mat *mat)
{
    if (mat->d) return QG_OK;
    bool temp = false;
    uint8_t *d = nullptr;
    const int rc = qg_mat_gguf(ctx, mat, &d, &temp);
    if (rc) return rc;
    mat->d = d;                      // owned (the matrix was uploaded)
    return QG_OK;
}

int qg_mat_drop_repacked(qg_ctx *ctx, qg_mat *mat)
{
    if (!mat->d_rp) return QG_OK;
    if (!mat->d) return fail(ctx, QG_ERR_INVALID_ARG, "the repacked copy is the only one");
    qg::Plan p;
    if (qg::make_plan(mat->type, mat->rows, mat->cols, ctx->n_cu, &p) != 0)
        return fail(ctx, QG_ERR_UNSUPPORTED_TYPE, "no kernel for type");
    QG_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (!mat->rp_view) (void)hipFree(mat->d_rp);
    mat->d_rp = nullptr;
    mat->rp_view = false;
    mat->plan = p;
    return QG_OK;
}

int qg_stack_views(qg_ctx *ctx, qg_mat *const *parts, int n, qg_mat **out)
{
    *out = nullptr;
    if (!ctx || n < 1) return QG_ERR_INVALID_ARG;
    const qg_mat *p0 = parts[0];
    size_t rows = 0, total = 0;
    for (int i = 0; i < n; i++) {
        const qg_mat *p = parts[i];
        if (p->type != p0->type || p->cols != p0->cols || !p->d_rp || p->rp_view || p->d || !p->plan.rp ||
            p->plan.g != p0->plan.g || p->plan.ni != p0->plan.ni || p->plan.group_bytes != p0->plan.group_bytes ||
            p->rows % p->plan.g != 0 || p->nbytes != (p->rows / p->plan.g) * p->plan.group_bytes)
            return QG_ERR_SHAPE;
        rows += p->rows;
        total += p->nbytes;
    }
    qg::Plan plan;
    if (qg::make_plan(p0->type, rows, p0->cols, ctx->n_cu, &plan, true) != 0 || !plan.rp || plan.g != p0->plan.g ||
        plan.ni != p0->plan.ni || plan.group_bytes != p0->plan.group_bytes)
        return QG_ERR_SHAPE;
    QG_HIP(ctx, hipSetDevice(ctx->device));
    uint8_t *r = nullptr;
    hipError_t e = qg_alloc_injected(ctx) ? hipErrorOutOfMemory : hipMalloc((void **)&r, total + qg::kTailPad);
    if (e != hipSuccess) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipMalloc stacked matrix", e);
    size_t off = 0;
    for (int i = 0; i < n && e == hipSuccess; i++) {
        e = hipMemcpyAsync(r + off, parts[i]->d_rp, parts[i]->nbytes, hipMemcpyDeviceToDevice, ctx->stream);
        off += parts[i]->nbytes;
    }
    if (e == hipSuccess) e = hipMemsetAsync(r + total, 0, qg::kTailPad, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    qg_mat *s = e == hipSuccess ? new (std::nothrow) qg_mat : nullptr;
    if (!s) {
        (void)hipFree(r);
        return e != hipSuccess ? fail(ctx, QG_ERR_HIP, "stacking copies", e)
                               : fail(ctx, QG_ERR_OUT_OF_MEMORY, "host allocation");
    }
    s->ctx = ctx;
    s->d = nullptr;
    s->d_rp = r;
    s->nbytes = total;
    s->type = p0->type;
    s->rows = rows;
    s->cols = p0->cols;
    s->owned = true;
    s->plan = plan;
    ctx->mats.insert(s);
    off = 0;
    for (int i = 0; i < n; i++) {
        (void)hipFree(parts[i]->d_rp);
        parts[i]->d_rp = r + off;
        parts[i]->rp_view = true;
        off += parts[i]->nbytes;
    }
    *out = s;
    return QG_OK;
}

int qg_mat_unview(qg_ctx *ctx, qg_mat *mat)
{
    if (!mat->rp_view) return QG_OK;
    QG_HIP(ctx, hipSetDevice(ctx->device));
    uint8_t *r = nullptr;
    hipError_t e = qg_alloc_injected(ctx) ? hipErrorOutOfMemory : hipMalloc((void **)&r, mat->nbytes + qg::kTailPad);
    if (e != hipSuccess) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipMalloc matrix copy", e);
    e = hipMemcpyAsync(r, mat->d_rp, mat->nbytes, hipMemcpyDeviceToDevice, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(r + mat->nbytes, 0, qg::kTailPad, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(r);
        return fail(ctx, QG_ERR_HIP, "copying a stacked part out", e);
    }
    mat->d_rp = r;
    mat->rp_view = false;
    return QG_OK;
}

int qg_mat_release(qg_ctx *ctx, qg_mat *mat, bool owned)
{
    if (!mat) return QG_OK;
    if (owned) return qg_mat_free(ctx, mat);
    if (mat->shares > 0) mat->shares--;
    return QG_OK;
}

int qg_norm_matvec(qg_ctx *ctx, const qg_mat *mat, const float *xa, const float *xb, const float *nw,
                   float eps, float *sum_out, float *y, float *scratch, hipStream_t st)
{
    ihipStream_t *sti = (ihipStream_t *)st;
    const size_t cols = mat->cols;
    auto a16 = [](const void *p) { return ((uintptr_t)p & 15u) == 0; };
    int lr = -1;
    if (cols == 0) {                                   // empty x: out.fill(0.0), quant.rs:189
        lr = qg::launch_fill(y, mat->rows, 0.0f, sti);
        return lr ? fail(ctx, QG_ERR_HIP, "kernel launch", hipGetLastError()) : QG_OK;
    }
    if (xb && a16(xa) && a16(xb) && a16(nw) && (!sum_out || a16(sum_out)))
        lr = qg::launch_gemv_norm(mat->plan, qg_gemv_bytes(mat), mat->nbytes, mat->rows, cols, xa, xb, nw, eps, sum_out,
                                  y, sti);
    if (lr == -1) {
        // two kernels: RMSNorm into scratch, then the mat-vec
        lr = qg::launch_rmsnorm(xa, xb, sum_out, nw, scratch, cols, eps, sti);
        if (lr == 0) {
            if (mat->plan.kind == 1 && (a16(scratch) || !mat->d))
                lr = qg::launch_gemv(mat->type, mat->plan, qg_gemv_bytes(mat), mat->nbytes, mat->rows, cols, scratch, y, sti);
            else
                lr = qg::launch_gemv_generic(mat->type, mat->d, mat->rows, cols, scratch, y, sti);
        }
    }
    return lr ? fail(ctx, QG_ERR_HIP, "kernel launch", hipGetLastError()) : QG_OK;
}

int qg_silu_matvec(qg_ctx *ctx, const qg_mat *mat, const float *g, const float *u, float *y, float *scratch,
                   hipStream_t st)
{
    ihipStream_t *sti = (ihipStream_t *)st;
    const size_t cols = mat->cols;
    auto a16 = [](const void *p) { return ((uintptr_t)p & 15u) == 0; };
    int lr = -1;
    if (cols == 0) {                                   // empty x: out.fill(0.0), quant.rs:189
        lr = qg::launch_fill(y, mat->rows, 0.0f, sti);
        return lr ? fail(ctx, QG_ERR_HIP, "kernel launch", hipGetLastError()) : QG_OK;
    }
    // every workgroup of the fused kernel forms the whole product itself:
    // cheaper than a second kernel for short rows only
    constexpr size_t kFuseMaxCols = 8192;
    if (cols <= kFuseMaxCols && a16(g) && a16(u))
        lr = qg::launch_gemv_silu(mat->plan, qg_gemv_bytes(mat), mat->nbytes, mat->rows, cols, g, u, y, sti);
    if (lr == -1) {
        lr = qg::launch_silu_mul(g, u, scratch, cols, sti);
        if (lr == 0) {
            if (mat->plan.kind == 1 && (a16(scratch) || !mat->d))
                lr = qg::launch_gemv(mat->type, mat->plan, qg_gemv_bytes(mat), mat->nbytes, mat->rows, cols, scratch, y, sti);
            else
                lr = qg::launch_gemv_generic(mat->type, mat->d, mat->rows, cols, scratch, y, sti);
        }
    }
    return lr ? fail(ctx, QG_ERR_HIP, "kernel launch", hipGetLastError()) : QG_OK;
}

int qg_norm_glu_matvec(qg_ctx *ctx, const qg_mat *gu, const float *xa, const float *xb, const float *nw,
                       float eps, float *sum_out, float *h, float *gu_out, float *scratch, hipStream_t st)
{
    ihipStream_t *sti = (ihipStream_t *)st;
    const size_t half = gu->rows / 2;
    auto a16 = [](const void *p) { return ((uintptr_t)p & 15u) == 0; };
    int lr = -1;
    if (gu->cols > 0 && xb && a16(xa) && a16(xb) && a16(nw) && (!sum_out || a16(sum_out)))
        lr = qg::launch_gemv_norm_glu(gu->plan, qg_gemv_bytes(gu), gu->nbytes, gu->rows, gu->cols, xa, xb, nw, eps, sum_out,
                                      h, sti);
    if (lr == -1) {
        int rc = qg_norm_matvec(ctx, gu, xa, xb, nw, eps, sum_out, gu_out, scratch, st);
        if (rc) return rc;
        lr = qg::launch_silu_mul(gu_out, gu_out + half, h, half, sti);
    }
    return lr ? fail(ctx, QG_ERR_HIP, "kernel launch", hipGetLastError()) : QG_OK;
}

int qg_norm_pair_matvec(qg_ctx *ctx, const qg_mat *m1, const qg_mat *m2, const float *xa, const float *xb,
                        const float *nw, float eps, float *sum_out, float *y1, float *y2, float *scratch,
                        hipStream_t st)
{
    auto a16 = [](const void *p) { return ((uintptr_t)p & 15u) == 0; };
    int lr = -1;
    if (m1->cols == m2->cols && m1->cols > 0 && xb && a16(xa) && a16(xb) && a16(nw) && (!sum_out || a16(sum_out)))
        lr = qg::launch_gemv_norm_pair(m1->type, m1->plan, qg_gemv_bytes(m1), m1->nbytes, m1->rows, y1, m2->type, m2->plan,
                                       qg_gemv_bytes(m2), m2->nbytes, m2->rows, y2, m1->cols, xa, xb, nw, eps, sum_out,
                                       ctx->n_cu, (ihipStream_t *)st);
    if (lr == 0) return QG_OK;
    if (lr != -1) return fail(ctx, QG_ERR_HIP, "kernel launch", hipGetLastError());
    int rc = qg_norm_matvec(ctx, m1, xa, xb, nw, eps, sum_out, y1, scratch, st);
    return rc ? rc : qg_norm_matvec(ctx, m2, xa, xb, nw, eps, nullptr, y2, scratch, st);
}

int qg_stack_mats(qg_ctx *ctx, qg_mat *const *parts, int n, qg_mat **out)
{
    *out = nullptr;
    if (!ctx || n < 1) return QG_ERR_INVALID_ARG;
    const uint32_t type = parts[0]->type;
    const size_t cols = parts[0]->cols;
    size_t rows = 0, total = 0;
    std::vector<size_t> need(n);
    for (int i = 0; i < n; i++) {
        const qg_mat *p = parts[i];
        if (p->type != type || p->cols != cols) return fail(ctx, QG_ERR_SHAPE, "stacked parts differ");
        if (required_bytes(type, p->rows, cols, &need[i]) != QG_OK)
            return fail(ctx, QG_ERR_SHAPE, "stacked part shape");
        // every part but the last ends on a block boundary, so the stacked
        // blocks are the blocks of the stacked matrix
        if (i + 1 < n && (p->rows * cols) % qg::block_elems(type) != 0)
            return fail(ctx, QG_ERR_SHAPE, "stacked part does not end on a block");
        rows += p->rows;
        total += need[i];
    }
    QG_HIP(ctx, hipSetDevice(ctx->device));
    uint8_t *d = nullptr;
    hipError_t e = qg_alloc_injected(ctx) ? hipErrorOutOfMemory : hipMalloc((void **)&d, total + qg::kTailPad);
    if (e != hipSuccess) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipMalloc", e);
    size_t off = 0;
    for (int i = 0; i < n && e == hipSuccess; i++) {
        if (parts[i]->d) {
            e = hipMemcpyAsync(d + off, parts[i]->d, need[i], hipMemcpyDeviceToDevice, ctx->stream);
        } else if (qg::launch_unrepack(type, parts[i]->plan, parts[i]->d_rp, d + off, (ihipStream_t *)ctx->stream)) {
            e = hipGetLastError();
            if (e == hipSuccess) e = hipErrorLaunchFailure;
        }
        off += need[i];
    }
    if (e == hipSuccess) e = hipMemsetAsync(d + total, 0, qg::kTailPad, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return fail(ctx, QG_ERR_HIP, "stacking copies", e);
    }
    int rc = new_mat(ctx, d, total, type, rows, cols, true, out);
    if (rc) (void)hipFree(d);
    return rc;
}

extern "C" {

const char *qg_status_string(int s)
{
    switch (s) {
    case QG_OK: return "ok";
    case QG_ERR_INVALID_ARG: return "invalid argument";
    case QG_ERR_UNSUPPORTED_TYPE: return "unsupported GGML type";
    case QG_ERR_SHORT_DATA: return "raw data shorter than the matrix needs";
    case QG_ERR_NO_DEVICE: return "no HIP device";
    case QG_ERR_HIP: return "HIP runtime error";
    case QG_ERR_OUT_OF_MEMORY: return "out of memory";
    case QG_ERR_SHAPE: return "shape mismatch";
    default: return "unknown status";
    }
}

const char *qg_last_error(const qg_ctx *ctx) { return ctx ? ctx->err.c_str() : ""; }

int qg_init(int device, qg_ctx **out)
{
    if (!out) return QG_ERR_INVALID_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return QG_ERR_NO_DEVICE;
    if (device < 0 || device >= n) return QG_ERR_INVALID_ARG;
    if (hipSetDevice(device) != hipSuccess) return QG_ERR_HIP;
    qg_ctx *ctx = new (std::nothrow) qg_ctx;
    if (!ctx) return QG_ERR_OUT_OF_MEMORY;
    ctx->device = device;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        delete ctx;
        return QG_ERR_HIP;
    }
    ctx->n_cu = prop.multiProcessorCount;
    // the static scratch array's address on this device (each GPU holds its
    // own copy at its own address); a failure only disables the no-allocation
    // entry point
    if (qg::scratch_address(device, &ctx->d_static_scratch) != 0) {
        ctx->d_static_scratch = nullptr;
        (void)hipGetLastError();
    }
    // default-priority stream (hipStreamCreateWithFlags keeps the default priority)
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return QG_ERR_HIP;
    }
    *out = ctx;
    return QG_OK;
}

int qg_destroy(qg_ctx *ctx)
{
    if (ctx) qg_models_free_all(ctx);
    if (!ctx) return QG_ERR_INVALID_ARG;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    while (!ctx->mats.empty()) drop_mat(ctx, *ctx->mats.begin());
    if (ctx->h_x) (void)hipHostFree(ctx->h_x);
    if (ctx->h_y) (void)hipHostFree(ctx->h_y);
    if (ctx->d_x) (void)hipFree(ctx->d_x);
    if (ctx->d_y) (void)hipFree(ctx->d_y);
    if (ctx->d_norm) (void)hipFree(ctx->d_norm);
    if (ctx->d_glu) (void)hipFree(ctx->d_glu);
    if (ctx->d_xal) (void)hipFree(ctx->d_xal);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return QG_OK;
}

int qg_upload(qg_ctx *ctx, const void *raw, size_t nbytes, uint32_t type, size_t rows,
              size_t cols, qg_mat **out)
{
    if (!ctx || !out) return QG_ERR_INVALID_ARG;
    *out = nullptr;
    size_t need = 0;
    int rc = required_bytes(type, rows, cols, &need);
    if (rc != QG_OK) return fail(ctx, rc, rc == QG_ERR_SHAPE ? "rows*cols overflows" : "unsupported type");
    if (nbytes < need) return fail(ctx, QG_ERR_SHORT_DATA, "raw data shorter than the matrix needs");
    if (need > 0 && !raw) return fail(ctx, QG_ERR_INVALID_ARG, "raw == NULL");
    QG_HIP(ctx, hipSetDevice(ctx->device));
    uint8_t *d = nullptr;
    hipError_t e = qg_alloc_injected(ctx) ? hipErrorOutOfMemory : hipMalloc((void **)&d, need + qg::kTailPad);
    if (e != hipSuccess) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipMalloc matrix", e);
    e = hipMemcpy(d, raw, need, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(d + need, 0, qg::kTailPad);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return fail(ctx, QG_ERR_HIP, "upload", e);
    }
    rc = new_mat(ctx, d, need, type, rows, cols, true, out);
    if (rc != QG_OK) (void)hipFree(d);
    return rc;
}

int qg_wrap_device(qg_ctx *ctx, const void *d_raw, size_t nbytes, uint32_t type, size_t rows,
                   size_t cols, qg_mat **out)
{
    if (!ctx || !out) return QG_ERR_INVALID_ARG;
    *out = nullptr;
    size_t need = 0;
    int rc = required_bytes(type, rows, cols, &need);
    if (rc != QG_OK) return fail(ctx, rc, "unsupported type or shape");
    if (nbytes < need) return fail(ctx, QG_ERR_SHORT_DATA, "raw data shorter than the matrix needs");
    if (!d_raw || ((uintptr_t)d_raw & 15u)) return fail(ctx, QG_ERR_INVALID_ARG, "device pointer NULL or not 16-byte aligned");
    // the kernels read whole 16-byte pieces up to kTailPad bytes past the
    // data: the allocation that holds d_raw must extend that far
    (void)hipSetDevice(ctx->device);
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)d_raw) != hipSuccess) {
        (void)hipGetLastError();                             // leave no sticky error for the caller's next launch
        return fail(ctx, QG_ERR_INVALID_ARG, "d_raw is not in a device allocation of this HIP runtime");
    }
    const uintptr_t end = (uintptr_t)base + size, p = (uintptr_t)d_raw;
    if (p < (uintptr_t)base || end - p < need || end - p - need < qg::kTailPad)
        return fail(ctx, QG_ERR_INVALID_ARG, "the allocation ends less than 512 bytes after the matrix data");
    return new_mat(ctx, (uint8_t *)d_raw, need, type, rows, cols, false, out);
}

int qg_mat_free(qg_ctx *ctx, qg_mat *mat)
{
    int rc = check_mat(ctx, mat);
    if (rc) return rc;
    if (mat->shares > 0)
        return fail(ctx, QG_ERR_INVALID_ARG, "matrix is in use by a decode-step model (qg_model_share_matrix)");
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    drop_mat(ctx, mat);
    return QG_OK;
}

int qg_mat_info(const qg_mat *mat, uint32_t *type, size_t *rows, size_t *cols, size_t *nbytes)
{
    if (!mat) return QG_ERR_INVALID_ARG;
    if (type) *type = mat->type;
    if (rows) *rows = mat->rows;
    if (cols) *cols = mat->cols;
    if (nbytes) *nbytes = mat->nbytes;
    return QG_OK;
}

int qg_mat_kernel_kind(const qg_mat *mat)
{
    if (!mat) return -1;
    if (mat->plan.kind == 1 && mat->plan.fn_wave) return 3;
    return mat->plan.kind == 1 && mat->plan.fn_ring ? 2 : mat->plan.kind;
}

int qg_matvec_dev(qg_ctx *ctx, const qg_mat *mat, const float *d_x, float *d_y, void *stream)
{
    int rc = check_mat(ctx, mat);
    if (rc) return rc;
    if (mat->rows == 0) return QG_OK;
    if (!d_y || (mat->cols > 0 && !d_x)) return fail(ctx, QG_ERR_INVALID_ARG, "x or y is NULL");
    if (((uintptr_t)d_x & 3u) || ((uintptr_t)d_y & 3u)) return fail(ctx, QG_ERR_INVALID_ARG, "x/y not 4-byte aligned");
    QG_HIP(ctx, hipSetDevice(ctx->device));
    hipStream_t st = pick(ctx, stream);
    int lr;
    if (mat->cols == 0)                                   // out.fill(0.0), quant.rs:189
        lr = qg::launch_fill(d_y, mat->rows, 0.0f, (ihipStream_t *)st);
    else if (ctx->prec_f32) {
        const uint8_t *w = qg_gemv_bytes(mat);
        if (!w) return fail(ctx, QG_ERR_INVALID_ARG, "matrix holds no bytes for the f32 path");
        lr = qg::launch_gemv_f32(mat->type, mat->plan, w, mat->nbytes, mat->rows, mat->cols, d_x, d_y,
                                 (ihipStream_t *)st);
    } else if (mat->plan.kind == 1 && ((uintptr_t)d_x & 15u) == 0)
        lr = qg::launch_gemv(mat->type, mat->plan, qg_gemv_bytes(mat), mat->nbytes, mat->rows, mat->cols, d_x,
                             d_y, (ihipStream_t *)st);
    else if (!mat->d) {
        // the repacked copy only: the stream kernel on an aligned copy of x
        if ((rc = grow_device(ctx, &ctx->d_xal, &ctx->d_xal_cap, mat->cols))) return rc;
        QG_HIP(ctx, hipMemcpyAsync(ctx->d_xal, d_x, mat->cols * sizeof(float), hipMemcpyDeviceToDevice, st));
        lr = qg::launch_gemv(mat->type, mat->plan, qg_gemv_bytes(mat), mat->nbytes, mat->rows, mat->cols, ctx->d_xal,
                             d_y, (ihipStream_t *)st);
    } else
        lr = qg::launch_gemv_generic(mat->type, mat->d, mat->rows, mat->cols, d_x, d_y,
                                     (ihipStream_t *)st);
    if (lr != 0) return fail(ctx, QG_ERR_HIP, "kernel launch", hipGetLastError());
    return QG_OK;
}

int qg_matvec_norm_dev(qg_ctx *ctx, const qg_mat *mat, const float *d_xa, const float *d_xb,
                       const float *d_nw, float eps, float *d_sum_out, float *d_y, void *stream)
{
    int rc = check_mat(ctx, mat);
    if (rc) return rc;
    if (mat->rows == 0 && !d_sum_out) return QG_OK;
    const size_t n = mat->cols;
    if (!d_y || (n > 0 && (!d_xa || !d_nw))) return fail(ctx, QG_ERR_INVALID_ARG, "xa, nw or y is NULL");
    auto a4 = [](const void *p) { return ((uintptr_t)p & 3u) == 0; };
    if (!a4(d_xa) || !a4(d_xb) || !a4(d_nw) || !a4(d_sum_out) || !a4(d_y))
        return fail(ctx, QG_ERR_INVALID_ARG, "vectors not 4-byte aligned");
    // sum_out is written while xa and xb are still being read
    auto overlap = [n](const float *p, const float *q) { return p && q && p < q + n && q < p + n; };
    if (overlap(d_sum_out, d_xa) || overlap(d_sum_out, d_xb))
        return fail(ctx, QG_ERR_INVALID_ARG, "sum_out overlaps xa or xb");
    QG_HIP(ctx, hipSetDevice(ctx->device));
    if ((rc = grow_device(ctx, &ctx->d_norm, &ctx->d_norm_cap, n))) return rc;
    return qg_norm_matvec(ctx, mat, d_xa, d_xb, d_nw, eps, d_sum_out, d_y, ctx->d_norm, pick(ctx, stream));
}

int qg_matvec_norm_glu_dev(qg_ctx *ctx, const qg_mat *gu, const float *d_xa, const float *d_xb,
                           const float *d_nw, float eps, float *d_sum_out, float *d_h, void *stream)
{
    int rc = check_mat(ctx, gu);
    if (rc) return rc;
    if (gu->rows % 2 != 0) return fail(ctx, QG_ERR_SHAPE, "[gate; up] matrix with an odd row count");
    if (gu->rows == 0 && !d_sum_out) return QG_OK;
    const size_t n = gu->cols;
    if (!d_h || (n > 0 && (!d_xa || !d_nw))) return fail(ctx, QG_ERR_INVALID_ARG, "xa, nw or h is NULL");
    auto a4 = [](const void *p) { return ((uintptr_t)p & 3u) == 0; };
    if (!a4(d_xa) || !a4(d_xb) || !a4(d_nw) || !a4(d_sum_out) || !a4(d_h))
        return fail(ctx, QG_ERR_INVALID_ARG, "vectors not 4-byte aligned");
    auto overlap = [n](const float *p, const float *q) { return p && q && p < q + n && q < p + n; };
    if (overlap(d_sum_out, d_xa) || overlap(d_sum_out, d_xb))
        return fail(ctx, QG_ERR_INVALID_ARG, "sum_out overlaps xa or xb");
    QG_HIP(ctx, hipSetDevice(ctx->device));
    if ((rc = grow_device(ctx, &ctx->d_norm, &ctx->d_norm_cap, n)) ||
        (rc = grow_device(ctx, &ctx->d_glu, &ctx->d_glu_cap, gu->rows)))
        return rc;
    return qg_norm_glu_matvec(ctx, gu, d_xa, d_xb, d_nw, eps, d_sum_out, d_h, ctx->d_glu, ctx->d_norm,
                              pick(ctx, stream));
}

int qg_mat_stack(qg_ctx *ctx, qg_mat *const *parts, int n_parts, qg_mat **out)
{
    if (!out) return fail(ctx, QG_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (!ctx || !parts || n_parts < 1) return fail(ctx, QG_ERR_INVALID_ARG, "no parts");
    for (int i = 0; i < n_parts; i++) {
        int rc = check_mat(ctx, parts[i]);
        if (rc) return rc;
    }
    return qg_stack_mats(ctx, parts, n_parts, out);
}

int qg_matvec_norm_glu_dev_noalloc(qg_ctx *ctx, const qg_mat *gu, const float *d_xa, const float *d_xb,
                                   const float *d_nw, float eps, float *d_sum_out, float *d_h, void *stream)
{
    int rc = check_mat(ctx, gu);
    if (rc) return rc;
    if (gu->rows % 2 != 0) return fail(ctx, QG_ERR_SHAPE, "[gate; up] matrix with an odd row count");
    if (gu->rows == 0 && !d_sum_out) return QG_OK;
    const size_t n = gu->cols;
    if (!d_h || (n > 0 && (!d_xa || !d_nw))) return fail(ctx, QG_ERR_INVALID_ARG, "xa, nw or h is NULL");
    auto a4 = [](const void *p) { return ((uintptr_t)p & 3u) == 0; };
    if (!a4(d_xa) || !a4(d_xb) || !a4(d_nw) || !a4(d_sum_out) || !a4(d_h))
        return fail(ctx, QG_ERR_INVALID_ARG, "vectors not 4-byte aligned");
    auto overlap = [n](const float *p, const float *q) { return p && q && p < q + n && q < p + n; };
    if (overlap(d_sum_out, d_xa) || overlap(d_sum_out, d_xb))
        return fail(ctx, QG_ERR_INVALID_ARG, "sum_out overlaps xa or xb");
    // the normalised x (cols floats, rounded up to 64 so the [gate; up]
    // outputs start 256-byte aligned), then the [gate; up] outputs (rows floats)
    const size_t xn = (n + 63) / 64 * 64;
    if (xn + gu->rows > qg::kNoAllocScratchFloats)
        return fail(ctx, QG_ERR_SHAPE, "cols + rows exceed the no-allocation scratch (262144 floats, 1 MiB)");
    if (!ctx->d_static_scratch) return fail(ctx, QG_ERR_HIP, "static scratch address not resolved at qg_init");
    QG_HIP(ctx, hipSetDevice(ctx->device));
    float *s = ctx->d_static_scratch;
    return qg_norm_glu_matvec(ctx, gu, d_xa, d_xb, d_nw, eps, d_sum_out, d_h, s + xn, s, pick(ctx, stream));
}

int qg_matvec_silu_dev(qg_ctx *ctx, const qg_mat *mat, const float *d_g, const float *d_u, float *d_y,
                       void *stream)
{
    int rc = check_mat(ctx, mat);
    if (rc) return rc;
    if (mat->rows == 0) return QG_OK;
    const size_t n = mat->cols;
    if (!d_y || (n > 0 && (!d_g || !d_u))) return fail(ctx, QG_ERR_INVALID_ARG, "g, u or y is NULL");
    auto a4 = [](const void *p) { return ((uintptr_t)p & 3u) == 0; };
    if (!a4(d_g) || !a4(d_u) || !a4(d_y)) return fail(ctx, QG_ERR_INVALID_ARG, "vectors not 4-byte aligned");
    QG_HIP(ctx, hipSetDevice(ctx->device));
    if ((rc = grow_device(ctx, &ctx->d_norm, &ctx->d_norm_cap, n))) return rc;
    return qg_silu_matvec(ctx, mat, d_g, d_u, d_y, ctx->d_norm, pick(ctx, stream));
}

int qg_matvec_host(qg_ctx *ctx, const qg_mat *mat, const float *x, float *y)
{
    int rc = check_mat(ctx, mat);
    if (rc) return rc;
    if (mat->rows == 0) return QG_OK;
    if (!y || (mat->cols > 0 && !x)) return fail(ctx, QG_ERR_INVALID_ARG, "x or y is NULL");
    QG_HIP(ctx, hipSetDevice(ctx->device));
    if ((rc = grow_pinned(ctx, &ctx->h_x, &ctx->h_x_cap, mat->cols)) ||
        (rc = grow_pinned(ctx, &ctx->h_y, &ctx->h_y_cap, mat->rows)) ||
        (rc = grow_device(ctx, &ctx->d_x, &ctx->d_x_cap, mat->cols)) ||
        (rc = grow_device(ctx, &ctx->d_y, &ctx->d_y_cap, mat->rows)))
        return rc;
    if (mat->cols) memcpy(ctx->h_x, x, mat->cols * sizeof(float));
    if (mat->cols)
        QG_HIP(ctx, hipMemcpyAsync(ctx->d_x, ctx->h_x, mat->cols * sizeof(float),
                                   hipMemcpyHostToDevice, ctx->stream));
    rc = qg_matvec_dev(ctx, mat, ctx->d_x, ctx->d_y, ctx->stream);
    if (rc) return rc;
    QG_HIP(ctx, hipMemcpyAsync(ctx->h_y, ctx->d_y, mat->rows * sizeof(float), hipMemcpyDeviceToHost,
                               ctx->stream));
    QG_HIP(ctx, hipStreamSynchronize(ctx->stream));
    memcpy(y, ctx->h_y, mat->rows * sizeof(float));
    return QG_OK;
}

int qg_gpu_mat_vec_mul(qg_ctx *ctx, const void *weight_data, size_t nbytes, uint32_t dtype,
                       const float *x, float *out, size_t rows, size_t cols)
{
    if (!ctx) return QG_ERR_INVALID_ARG;
    auto key = std::make_tuple((uintptr_t)weight_data, nbytes, dtype, rows, cols);
    size_t need = 0;
    int rc = required_bytes(dtype, rows, cols, &need);
    if (rc != QG_OK) return fail(ctx, rc, "unsupported type or shape");
    if (nbytes < need) return fail(ctx, QG_ERR_SHORT_DATA, "raw data shorter than the matrix needs");
    if (need > 0 && !weight_data) return fail(ctx, QG_ERR_INVALID_ARG, "weight_data == NULL");
    const bool exact = ctx->fresh_exact;
    const uint8_t *wb = (const uint8_t *)weight_data;
    std::vector<uint8_t> fp;
    if (!exact) fp = fingerprint(wb, need);
    qg_mat *m = nullptr;
    auto it = ctx->keyed.find(key);
    bool hit = false;
    if (it != ctx->keyed.end() && it->second.exact == exact) {
        const std::vector<uint8_t> &had = it->second.fp;
        hit = exact ? had.size() == need && (need == 0 || memcmp(had.data(), wb, need) == 0) : had == fp;
    }
    if (hit) {
        m = it->second.mat;
    } else {
        // first sight, or the bytes at this address changed since the copy
        // was made (weights edited in place, or a freed buffer's address
        // reused): upload the current bytes
        if (it != ctx->keyed.end()) {
            QG_HIP(ctx, hipSetDevice(ctx->device));
            (void)hipStreamSynchronize(ctx->stream);
            drop_mat(ctx, it->second.mat);
        }
        if (exact) {
            try {
                fp.assign(wb, wb + need);                // the bytes the copy is made from
            } catch (const std::bad_alloc &) {
                return fail(ctx, QG_ERR_OUT_OF_MEMORY, "host copy of the weight bytes");
            }
        }
        if ((rc = qg_upload(ctx, weight_data, nbytes, dtype, rows, cols, &m))) return rc;
        ctx->keyed[key] = qg_ctx::Keyed{m, std::move(fp), exact};
    }
    return qg_matvec_host(ctx, m, x, out);
}

int qg_set_precision(qg_ctx *ctx, int mode)
{
    if (!ctx || (mode != QG_PRECISION_FIXED22 && mode != QG_PRECISION_F32)) return QG_ERR_INVALID_ARG;
    ctx->prec_f32 = mode == QG_PRECISION_F32;
    return QG_OK;
}

int qg_gpu_set_freshness(qg_ctx *ctx, int mode)
{
    if (!ctx || (mode != QG_FRESH_SAMPLED && mode != QG_FRESH_EXACT)) return QG_ERR_INVALID_ARG;
    ctx->fresh_exact = mode == QG_FRESH_EXACT;
    return QG_OK;
}

int qg_gpu_invalidate(qg_ctx *ctx, const void *weight_data)
{
    if (!ctx) return QG_ERR_INVALID_ARG;
    QG_HIP(ctx, hipSetDevice(ctx->device));
    (void)hipStreamSynchronize(ctx->stream);
    std::vector<qg_mat *> gone;
    for (auto &kv : ctx->keyed)
        if (std::get<0>(kv.first) == (uintptr_t)weight_data) gone.push_back(kv.second.mat);
    for (qg_mat *m : gone) drop_mat(ctx, m);
    return QG_OK;
}

int qg_test_fail_allocations(qg_ctx *ctx, int skip, int n)
{
    if (!ctx || skip < 0 || n < 0) return QG_ERR_INVALID_ARG;
    ctx->fail_skip = skip;
    ctx->fail_allocs = n;
    return QG_OK;
}

int qg_dequant_dev(qg_ctx *ctx, const qg_mat *mat, float *d_out, void *stream)
{
    int rc = check_mat(ctx, mat);
    if (rc) return rc;
    size_t n = mat->rows * mat->cols;
    if (n == 0) return QG_OK;
    if (!d_out) return fail(ctx, QG_ERR_INVALID_ARG, "out is NULL");
    QG_HIP(ctx, hipSetDevice(ctx->device));
    uint8_t *w = nullptr;
    bool temp = false;
    if ((rc = qg_mat_gguf(ctx, mat, &w, &temp))) return rc;
    hipStream_t st = pick(ctx, stream);
    if (qg::launch_dequant(mat->type, w, n, d_out, (ihipStream_t *)st)) {
        if (temp) (void)hipFree(w);
        return fail(ctx, QG_ERR_HIP, "dequant launch", hipGetLastError());
    }
    if (temp) {                                          // the rebuilt copy lives until the kernel ends
        const hipError_t e = hipStreamSynchronize(st);
        (void)hipFree(w);
        if (e != hipSuccess) return fail(ctx, QG_ERR_HIP, "dequant", e);
    }
    return QG_OK;
}

int qg_dequant_host(qg_ctx *ctx, const qg_mat *mat, float *out)
{
    int rc = check_mat(ctx, mat);
    if (rc) return rc;
    size_t n = mat->rows * mat->cols;
    if (n == 0) return QG_OK;
    if (!out) return fail(ctx, QG_ERR_INVALID_ARG, "out is NULL");
    QG_HIP(ctx, hipSetDevice(ctx->device));
    float *d = nullptr;
    hipError_t e = hipMalloc((void **)&d, n * sizeof(float));
    if (e != hipSuccess) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipMalloc dequant", e);
    rc = qg_dequant_dev(ctx, mat, d, ctx->stream);
    if (rc == QG_OK) {
        e = hipMemcpyAsync(out, d, n * sizeof(float), hipMemcpyDeviceToHost, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) rc = fail(ctx, QG_ERR_HIP, "dequant readback", e);
    }
    (void)hipFree(d);
    return rc;
}

int qg_dequantize_row_dev(qg_ctx *ctx, const qg_mat *mat, size_t row, float *d_out, void *stream)
{
    int rc = check_mat(ctx, mat);
    if (rc) return rc;
    if (row >= mat->rows) return fail(ctx, QG_ERR_SHAPE, "row out of range");   // quant.rs:153
    if (!d_out) return fail(ctx, QG_ERR_INVALID_ARG, "out is NULL");
    QG_HIP(ctx, hipSetDevice(ctx->device));
    hipStream_t st = pick(ctx, stream);
    if (mat->d) {
        if (qg::launch_dequantize_row(mat->type, mat->d, mat->rows, mat->cols, row, d_out, (ihipStream_t *)st))
            return fail(ctx, QG_ERR_HIP, "dequantize_row launch", hipGetLastError());
        return QG_OK;
    }
    // repacked only: the row's row group (whole blocks) in the GGUF layout,
    // as a matrix of g rows
    const qg::Plan &p = mat->plan;
    const size_t grp = row / p.g;
    uint8_t *t = nullptr;
    hipError_t e = qg_alloc_injected(ctx) ? hipErrorOutOfMemory : hipMalloc((void **)&t, p.group_bytes + qg::kTailPad);
    if (e != hipSuccess) return fail(ctx, QG_ERR_OUT_OF_MEMORY, "hipMalloc row group", e);
    qg::Plan one = p;
    one.n_groups = 1;
    int lr = qg::launch_unrepack(mat->type, one, mat->d_rp + grp * p.group_bytes, t, (ihipStream_t *)st);
    if (lr == 0) e = hipMemsetAsync(t + p.group_bytes, 0, qg::kTailPad, st);
    if (lr == 0 && e == hipSuccess)
        lr = qg::launch_dequantize_row(mat->type, t, p.g, mat->cols, row % p.g, d_out, (ihipStream_t *)st);
    if (lr == 0 && e == hipSuccess) e = hipStreamSynchronize(st);
    (void)hipFree(t);
    if (lr != 0 || e != hipSuccess)
        return fail(ctx, QG_ERR_HIP, "dequantize_row", e != hipSuccess ? e : hipGetLastError());
    return QG_OK;
}

int qg_matvec_dev_repeat(qg_ctx *ctx, const qg_mat *const *mats, size_t n_mats, const float *d_x, float *d_y,
                         size_t n_launches, void *stream)
{
    if (!ctx || (n_launches && (!mats || n_mats == 0))) return QG_ERR_INVALID_ARG;
    for (size_t i = 0; i < n_launches; i++) {
        const int rc = qg_matvec_dev(ctx, mats[i % n_mats], d_x, d_y, stream);
        if (rc) return rc;
    }
    return QG_OK;
}

int qg_synchronize(qg_ctx *ctx)
{
    if (!ctx) return QG_ERR_INVALID_ARG;
    QG_HIP(ctx, hipSetDevice(ctx->device));
    QG_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return QG_OK;
}

void *qg_stream(qg_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int qg_device_cu_count(const qg_ctx *ctx) { return ctx ? ctx->n_cu : 0; }

}  // extern "C"
