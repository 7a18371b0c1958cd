// qg_model.hip -- the decode step of yudono/rust-inference on device
// (include/qgmodel.h).
//
// Every tensor stays in HBM for the whole generation: the quantized weights
// (raw GGUF blocks, mat-vec'd by the library's GEMV), norms and biases, the
// f32 KV caches, the activations and the logits.  Per token the host only
// enqueues kernels; the one device->host transfer is the sampled token id.
//
// Kernels (all f32, -ffp-contract=off: every product and sum is rounded where
// the reference rounds it, except that block reductions add in tree order):
//   rmsnorm_k        math.rs:237-273 (RmsNorm::forward), optionally fused
//                    with the residual add of transformer.rs:31-46
//   qkv_post_k       attention.rs:68-90: bias add, RoPE on q and k
//                    (rope.rs:88-96, pairs 2i/2i+1), KV append (kv_cache.rs:52-73)
//   attention_k      attention.rs:92-121: scores, softmax (math.rs:104-118),
//                    weighted sum of v, one workgroup per query head
//   silu_mul_k       mlp.rs:36-41, silu as math.rs:137-146
//   sample_greedy_k  sampler.rs:109-127 then math.rs:328-339
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "qg_common.h"
#include "qg_internal.h"
#include "qgmodel.h"

namespace qgm {

constexpr int kBlock = 1024;

// Sum over the workgroup (every thread gets the total).
__device__ float block_sum(float v, float *red)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// Max over the workgroup ignoring NaN (f32::max), every thread gets it.
__device__ float block_max(float v, float *red)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int i = 0; i < nw; i++) t = fmaxf(t, red[i]);
    return t;
}

// One thread per (2i, 2i+1) pair of q (q_dim/2 pairs) and of k/v (kv_dim/2).
__global__ void __launch_bounds__(256) qkv_post_k(float *__restrict__ q, const float *__restrict__ k,
                                                  const float *__restrict__ v, const float *__restrict__ bq,
                                                  const float *__restrict__ bk, const float *__restrict__ bv,
                                                  float *__restrict__ kc, float *__restrict__ vc,
                                                  const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                                                  uint32_t q_dim, uint32_t kv_dim, uint32_t hd, uint32_t pos,
                                                  uint32_t slot)
{
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x, half = hd / 2;
    const uint32_t i0 = 2 * t;
    if (i0 < q_dim) {
        const uint32_t j = (i0 % hd) / 2;
        const float c = cos_t[pos * half + j], s = sin_t[pos * half + j];
        const float x0 = q[i0] + bq[i0], x1 = q[i0 + 1] + bq[i0 + 1];
        q[i0] = x0 * c - x1 * s;
        q[i0 + 1] = x0 * s + x1 * c;
    }
    if (i0 < kv_dim) {
        const uint32_t j = (i0 % hd) / 2;
        const float c = cos_t[pos * half + j], s = sin_t[pos * half + j];
        const float x0 = k[i0] + bk[i0], x1 = k[i0 + 1] + bk[i0 + 1];
        float *kr = kc + (size_t)slot * kv_dim, *vr = vc + (size_t)slot * kv_dim;
        kr[i0] = x0 * c - x1 * s;
        kr[i0 + 1] = x0 * s + x1 * c;
        vr[i0] = v[i0] + bv[i0];
        vr[i0 + 1] = v[i0 + 1] + bv[i0 + 1];
    }
}

// One workgroup per query head; LDS: hd floats of q, seq floats of scores.
__global__ void __launch_bounds__(256) attention_k(const float *__restrict__ q, const float *__restrict__ kc,
                                                   const float *__restrict__ vc, float *__restrict__ out,
                                                   uint32_t seq, uint32_t hd, uint32_t kv_dim, uint32_t n_rep,
                                                   float scale)
{
    extern __shared__ float sm[];
    __shared__ float red[4];
    float *qs = sm, *sc = sm + hd;
    const uint32_t h = blockIdx.x, kvh = (h / n_rep) * hd;
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) qs[d] = q[h * hd + d];
    __syncthreads();
    float mx = -INFINITY;
    for (uint32_t j = threadIdx.x; j < seq; j += blockDim.x) {
        const float *kr = kc + (size_t)j * kv_dim + kvh;
        float s = 0.f;
        for (uint32_t d = 0; d < hd; d++) s += qs[d] * kr[d];             // math.rs:63-70
        s = s * scale;
        sc[j] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_max(mx, red);
    float sum = 0.f;
    for (uint32_t j = threadIdx.x; j < seq; j += blockDim.x) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    sum = block_sum(sum, red);
    const float inv = 1.0f / sum;
    for (uint32_t j = threadIdx.x; j < seq; j += blockDim.x) sc[j] *= inv;
    __syncthreads();
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
        float acc = 0.f;
        for (uint32_t j = 0; j < seq; j++) acc += sc[j] * vc[(size_t)j * kv_dim + kvh + d];
        out[h * hd + d] = acc;
    }
}

// Same result for head dimensions hd = 64 * E (E = 1, 2, 4): one workgroup of
// four waves per query head.  Wave w takes positions j = w, w + 4, ...; its
// lanes split the head dimension (lane owns d = lane + 64e), so every key and
// value row is one coalesced 4E-byte-per-lane read and each score is a wave
// reduction.  The four per-wave partial outputs are added through LDS.
template <int E>
__global__ void __launch_bounds__(256) attention_wave_k(const float *__restrict__ q, const float *__restrict__ kc,
                                                        const float *__restrict__ vc, float *__restrict__ out,
                                                        uint32_t seq, uint32_t kv_dim, uint32_t n_rep, float scale)
{
    constexpr uint32_t HD = 64 * E;
    extern __shared__ float sm[];                 // sc[seq], part[4][HD]
    __shared__ float red[4];
    float *sc = sm, *part = sm + seq;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t h = blockIdx.x, kvh = (h / n_rep) * HD;
    float qv[E];
#pragma unroll
    for (int e = 0; e < E; e++) qv[e] = q[h * HD + lane + 64 * e];
    float mx = -INFINITY;
    for (uint32_t j = wave; j < seq; j += 4) {
        const float *kr = kc + (size_t)j * kv_dim + kvh;
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < E; e++) s += qv[e] * kr[lane + 64 * e];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
        s = s * scale;
        if (lane == 0) sc[j] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_max(mx, red);                      // (barrier inside: sc complete)
    float sum = 0.f;
    for (uint32_t j = threadIdx.x; j < seq; j += blockDim.x) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    sum = block_sum(sum, red);
    const float inv = 1.0f / sum;
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] = 0.f;
    for (uint32_t j = wave; j < seq; j += 4) {
        const float p = sc[j] * inv;
        const float *vr = vc + (size_t)j * kv_dim + kvh;
#pragma unroll
        for (int e = 0; e < E; e++) acc[e] += p * vr[lane + 64 * e];
    }
#pragma unroll
    for (int e = 0; e < E; e++) part[wave * HD + lane + 64 * e] = acc[e];
    __syncthreads();
    for (uint32_t d = threadIdx.x; d < HD; d += blockDim.x)
        out[h * HD + d] = (part[d] + part[HD + d]) + (part[2 * HD + d] + part[3 * HD + d]);
}

__device__ __forceinline__ float silu1(float x)
{
    if (x >= 0.0f) {
        const float e = expf(-x);
        return x / (1.0f + e);
    }
    const float e = expf(x);
    return x * e / (1.0f + e);
}

__global__ void __launch_bounds__(256) silu_mul_k(const float *__restrict__ g, const float *__restrict__ u,
                                                  float *__restrict__ h, uint32_t n)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = silu1(g[i]) * u[i];
}

// Repetition penalty over recent[0..n_recent) in order, then the first index
// of the maximum (NaN never wins; a NaN at index 0 returns 0, as the
// reference's strict ">" scan does).
__global__ void __launch_bounds__(kBlock) sample_greedy_k(float *__restrict__ logits, uint32_t n,
                                                          const uint32_t *__restrict__ recent,
                                                          uint32_t n_recent, float penalty,
                                                          uint32_t *__restrict__ token)
{
    __shared__ float bv[kBlock / 64];
    __shared__ uint32_t bi[kBlock / 64];
    if (threadIdx.x == 0 && penalty != 1.0f) {
        for (uint32_t r = 0; r < n_recent; r++) {
            const uint32_t t = recent[r];
            if (t < n) {
                const float l = logits[t];
                logits[t] = l > 0.0f ? l / penalty : l * penalty;
            }
        }
    }
    __syncthreads();
    float best = -INFINITY;
    uint32_t idx = 0xFFFFFFFFu;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = logits[i];
        if (v > best || (idx == 0xFFFFFFFFu && v == best)) { best = v; idx = i; }
    }
    // (value, index) max with the smaller index on ties
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const uint32_t oi = __shfl_xor(idx, o, 64);
        if (oi != 0xFFFFFFFFu && (idx == 0xFFFFFFFFu || ov > best || (ov == best && oi < idx))) {
            best = ov; idx = oi;
        }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { bv[w] = best; bi[w] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = -INFINITY;
        uint32_t id = 0xFFFFFFFFu;
        for (int i = 0; i < (int)(blockDim.x >> 6); i++) {
            if (bi[i] == 0xFFFFFFFFu) continue;
            if (id == 0xFFFFFFFFu || bv[i] > b || (bv[i] == b && bi[i] < id)) { b = bv[i]; id = bi[i]; }
        }
        const float l0 = logits[0];
        *token = (l0 != l0 || id == 0xFFFFFFFFu) ? 0u : id;
    }
}

}  // namespace qgm

// ----------------------------------------------------------------- engine

namespace {
constexpr int kSlots = 7;                 // WQ .. DOWN
constexpr size_t kRecentMax = 64;         // model.rs:370-374 passes the last 64 tokens
}

struct qg_model {
    qg_ctx *ctx = nullptr;
    qg_model_config cfg{};
    uint32_t hd = 0, q_dim = 0, kv_dim = 0, n_rep = 0;
    qg_mat *tok = nullptr, *lm = nullptr;
    bool tok_owned = false, lm_owned = false;
    std::vector<qg_mat *> w[kSlots];
    std::vector<bool> owned[kSlots];
    float *final_norm = nullptr;
    std::vector<float *> vec[6];          // per layer: attn_norm, ffn_norm, bq, bk, bv (slot 0 unused)
    float *kc = nullptr, *vc = nullptr;   // [n_layers][max_seq_len][kv_dim]
    size_t seq = 0;
    float *cos_t = nullptr, *sin_t = nullptr;
    float *h0 = nullptr, *h1 = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
    float *ao = nullptr, *ao2 = nullptr, *g = nullptr, *u = nullptr, *hb = nullptr, *fo = nullptr;
    float *logits = nullptr;
    float *zeros = nullptr;               // the residual addend of the first layer
    uint32_t *d_recent = nullptr, *d_token = nullptr;
    uint32_t *h_recent = nullptr, *h_token = nullptr;   // pinned
    std::vector<void *> allocs;
};

namespace {

int mfail(qg_model *m, int st, const char *what, hipError_t e = hipSuccess)
{
    return qg_fail(m ? m->ctx : nullptr, st, what, e);
}

#define QGM_HIP(m, call)                                                      \
    do {                                                                      \
        hipError_t e_ = (call);                                               \
        if (e_ != hipSuccess) return mfail((m), QG_ERR_HIP, #call, e_);       \
    } while (0)

template <class T> int dalloc(qg_model *m, T **p, size_t n)
{
    void *d = nullptr;
    hipError_t e = hipMalloc(&d, (n ? n : 1) * sizeof(T));
    if (e != hipSuccess) return mfail(m, QG_ERR_OUT_OF_MEMORY, "hipMalloc", e);
    e = hipMemset(d, 0, (n ? n : 1) * sizeof(T));
    if (e != hipSuccess) { (void)hipFree(d); return mfail(m, QG_ERR_HIP, "hipMemset", e); }
    m->allocs.push_back(d);
    *p = (T *)d;
    return QG_OK;
}

void free_model(qg_model *m)
{
    m->ctx->models.erase(m);
    for (int s = 0; s < kSlots; s++)
        for (size_t l = 0; l < m->w[s].size(); l++)
            if (m->w[s][l] && m->owned[s][l]) qg_mat_free(m->ctx, m->w[s][l]);
    if (m->tok && m->tok_owned) qg_mat_free(m->ctx, m->tok);
    if (m->lm && m->lm_owned) qg_mat_free(m->ctx, m->lm);
    for (void *p : m->allocs) (void)hipFree(p);
    if (m->h_recent) (void)hipHostFree(m->h_recent);
    if (m->h_token) (void)hipHostFree(m->h_token);
    delete m;
}

// expected (rows, cols) of a slot
void slot_shape(const qg_model *m, uint32_t which, size_t *rows, size_t *cols)
{
    const size_t E = m->cfg.embed_dim, H = m->cfg.hidden_dim, V = m->cfg.vocab_size;
    switch (which) {
    case QG_M_TOKEN_EMBD: case QG_M_LM_HEAD: *rows = V; *cols = E; break;
    case QG_M_WQ: *rows = m->q_dim; *cols = E; break;
    case QG_M_WK: case QG_M_WV: *rows = m->kv_dim; *cols = E; break;
    case QG_M_WO: *rows = E; *cols = m->q_dim; break;
    case QG_M_GATE: case QG_M_UP: *rows = H; *cols = E; break;
    case QG_M_DOWN: *rows = E; *cols = H; break;
    default: *rows = *cols = 0;
    }
}

int gemv(qg_model *m, const qg_mat *a, const float *x, float *y)
{
    if (qg::launch_gemv(a->type, a->plan, a->d, a->nbytes, a->rows, a->cols, x, y,
                        (ihipStream_t *)m->ctx->stream) != 0)
        return mfail(m, QG_ERR_HIP, "GEMV launch", hipGetLastError());
    return QG_OK;
}

// y = A · (rmsnorm(xa + xb) * nw); sum_out (may be NULL) receives xa + xb.
// The GEMV's own prologue does the norm when the matrix runs on the stream
// kernel; otherwise a separate RMSNorm kernel writes m->xn first.
int gemv_norm(qg_model *m, const qg_mat *A, const float *xa, const float *xb, const float *nw,
              float *sum_out, float *y)
{
    return qg_norm_matvec(m->ctx, A, xa, xb, nw, m->cfg.norm_eps, sum_out, y, m->xn, m->ctx->stream);
}

int launched(qg_model *m, const char *what)
{
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? QG_OK : mfail(m, QG_ERR_HIP, what, e);
}

bool complete(const qg_model *m)
{
    if (!m->tok || !m->lm || !m->final_norm) return false;
    for (int s = 0; s < kSlots; s++)
        for (qg_mat *p : m->w[s])
            if (!p) return false;
    return true;
}

}  // namespace

extern "C" {

int qg_model_create(qg_ctx *ctx, const qg_model_config *cfg, qg_model **out)
{
    if (!ctx || !cfg || !out) return QG_ERR_INVALID_ARG;
    *out = nullptr;
    const qg_model_config c = *cfg;
    if (c.embed_dim == 0 || c.n_layers == 0 || c.n_heads == 0 || c.hidden_dim == 0 ||
        c.vocab_size == 0 || c.max_seq_len == 0 || c.embed_dim % c.n_heads != 0)
        return qg_fail(ctx, QG_ERR_SHAPE, "model config");
    const uint32_t n_kv = c.n_kv_heads ? c.n_kv_heads : c.n_heads;   // model.rs:100
    const uint32_t hd = c.embed_dim / c.n_heads;
    if (hd % 2 != 0 || c.n_heads % n_kv != 0) return qg_fail(ctx, QG_ERR_SHAPE, "model config");
    qg_model *m = new (std::nothrow) qg_model;
    if (!m) return qg_fail(ctx, QG_ERR_OUT_OF_MEMORY, "host allocation");
    m->ctx = ctx;
    m->cfg = c;
    m->cfg.n_kv_heads = n_kv;
    m->hd = hd;
    m->q_dim = c.n_heads * hd;
    m->kv_dim = n_kv * hd;
    m->n_rep = c.n_heads / n_kv;
    const size_t L = c.n_layers, E = c.embed_dim, H = c.hidden_dim;
    for (int s = 0; s < kSlots; s++) { m->w[s].assign(L, nullptr); m->owned[s].assign(L, false); }
    int rc;
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) { free_model(m); return qg_fail(ctx, QG_ERR_HIP, "hipSetDevice", e); }
    const size_t kvn = L * (size_t)c.max_seq_len * m->kv_dim;
    if ((rc = dalloc(m, &m->final_norm, E)) || (rc = dalloc(m, &m->kc, kvn)) ||
        (rc = dalloc(m, &m->vc, kvn)) || (rc = dalloc(m, &m->h0, E)) || (rc = dalloc(m, &m->h1, E)) ||
        (rc = dalloc(m, &m->xn, E > H ? E : H)) || (rc = dalloc(m, &m->q, m->q_dim)) ||
        (rc = dalloc(m, &m->k, m->kv_dim)) || (rc = dalloc(m, &m->v, m->kv_dim)) ||
        (rc = dalloc(m, &m->ao, m->q_dim)) || (rc = dalloc(m, &m->ao2, E)) ||
        (rc = dalloc(m, &m->g, H)) || (rc = dalloc(m, &m->u, H)) || (rc = dalloc(m, &m->hb, H)) ||
        (rc = dalloc(m, &m->fo, E)) || (rc = dalloc(m, &m->logits, c.vocab_size)) ||
        (rc = dalloc(m, &m->zeros, E > H ? E : H)) ||
        (rc = dalloc(m, &m->d_recent, kRecentMax)) || (rc = dalloc(m, &m->d_token, 1))) {
        free_model(m);
        return rc;
    }
    for (int s = 1; s < 6; s++) {
        m->vec[s].assign(L, nullptr);
        const size_t n = s <= 2 ? E : s == 3 ? m->q_dim : m->kv_dim;
        for (size_t l = 0; l < L; l++)
            if ((rc = dalloc(m, &m->vec[s][l], n))) { free_model(m); return rc; }
    }
    // RoPE tables (rope.rs:42-58): f32 powf / cos / sin, as the reference
    const size_t half = hd / 2, np = (size_t)c.max_seq_len * half;
    std::vector<float> ct(np), st(np);
    for (size_t pos = 0; pos < c.max_seq_len; pos++)
        for (size_t i = 0; i < half; i++) {
            const float exponent = (float)(2 * i) / (float)hd;
            const float theta = 1.0f / powf(c.rope_base, exponent);
            const float angle = (float)pos * theta;
            ct[pos * half + i] = cosf(angle);
            st[pos * half + i] = sinf(angle);
        }
    if ((rc = dalloc(m, &m->cos_t, np)) || (rc = dalloc(m, &m->sin_t, np))) { free_model(m); return rc; }
    if ((e = hipMemcpy(m->cos_t, ct.data(), np * sizeof(float), hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(m->sin_t, st.data(), np * sizeof(float), hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipHostMalloc((void **)&m->h_recent, kRecentMax * sizeof(uint32_t), hipHostMallocDefault)) != hipSuccess ||
        (e = hipHostMalloc((void **)&m->h_token, sizeof(uint32_t), hipHostMallocDefault)) != hipSuccess) {
        free_model(m);
        return qg_fail(ctx, QG_ERR_HIP, "model set-up", e);
    }
    ctx->models.insert(m);
    *out = m;
    return QG_OK;
}

int qg_model_destroy(qg_model *m)
{
    if (!m) return QG_ERR_INVALID_ARG;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    free_model(m);
    return QG_OK;
}

int qg_model_set_matrix(qg_model *m, uint32_t which, uint32_t layer, const void *raw, size_t nbytes,
                        uint32_t ggml_type, size_t rows, size_t cols)
{
    if (!m || !raw) return QG_ERR_INVALID_ARG;
    size_t er, ec;
    slot_shape(m, which, &er, &ec);
    if (er == 0) return mfail(m, QG_ERR_INVALID_ARG, "matrix slot");
    if (rows != er || cols != ec) return mfail(m, QG_ERR_SHAPE, "matrix shape does not match the config");
    const bool per_layer = which >= QG_M_WQ;
    if (per_layer && layer >= m->cfg.n_layers) return mfail(m, QG_ERR_INVALID_ARG, "layer");
    qg_mat *mat = nullptr;
    int rc = qg_upload(m->ctx, raw, nbytes, ggml_type, rows, cols, &mat);
    if (rc) return rc;
    qg_mat **dst;
    bool *own;
    if (which == QG_M_TOKEN_EMBD) { dst = &m->tok; own = &m->tok_owned; }
    else if (which == QG_M_LM_HEAD) { dst = &m->lm; own = &m->lm_owned; }
    else {
        const int s = (int)which - QG_M_WQ;
        if (m->w[s][layer] && m->owned[s][layer]) qg_mat_free(m->ctx, m->w[s][layer]);
        m->w[s][layer] = mat;
        m->owned[s][layer] = true;
        return QG_OK;
    }
    if (*dst && *own) qg_mat_free(m->ctx, *dst);
    *dst = mat;
    *own = true;
    return QG_OK;
}

int qg_model_share_matrix(qg_model *m, uint32_t which, uint32_t layer, const qg_mat *mat)
{
    if (!m || !mat) return QG_ERR_INVALID_ARG;
    size_t er, ec;
    slot_shape(m, which, &er, &ec);
    if (er == 0) return mfail(m, QG_ERR_INVALID_ARG, "matrix slot");
    if (mat->rows != er || mat->cols != ec || mat->ctx != m->ctx)
        return mfail(m, QG_ERR_SHAPE, "matrix shape does not match the config");
    qg_mat *mm = const_cast<qg_mat *>(mat);
    if (which == QG_M_TOKEN_EMBD) {
        if (m->tok && m->tok_owned) qg_mat_free(m->ctx, m->tok);
        m->tok = mm; m->tok_owned = false;
    } else if (which == QG_M_LM_HEAD) {
        if (m->lm && m->lm_owned) qg_mat_free(m->ctx, m->lm);
        m->lm = mm; m->lm_owned = false;
    } else {
        if (layer >= m->cfg.n_layers) return mfail(m, QG_ERR_INVALID_ARG, "layer");
        const int s = (int)which - QG_M_WQ;
        if (m->w[s][layer] && m->owned[s][layer]) qg_mat_free(m->ctx, m->w[s][layer]);
        m->w[s][layer] = mm;
        m->owned[s][layer] = false;
    }
    return QG_OK;
}

int qg_model_set_vector(qg_model *m, uint32_t which, uint32_t layer, const float *v, size_t n)
{
    if (!m || !v) return QG_ERR_INVALID_ARG;
    float *dst;
    size_t want;
    if (which == QG_V_FINAL_NORM) { dst = m->final_norm; want = m->cfg.embed_dim; }
    else if (which <= QG_V_BV) {
        if (layer >= m->cfg.n_layers) return mfail(m, QG_ERR_INVALID_ARG, "layer");
        dst = m->vec[which][layer];
        want = which <= QG_V_FFN_NORM ? m->cfg.embed_dim : which == QG_V_BQ ? m->q_dim : m->kv_dim;
    } else {
        return mfail(m, QG_ERR_INVALID_ARG, "vector slot");
    }
    if (n != want) return mfail(m, QG_ERR_SHAPE, "vector length does not match the config");
    QGM_HIP(m, hipSetDevice(m->ctx->device));
    QGM_HIP(m, hipMemcpy(dst, v, n * sizeof(float), hipMemcpyHostToDevice));
    return QG_OK;
}

int qg_model_reset(qg_model *m)
{
    if (!m) return QG_ERR_INVALID_ARG;
    m->seq = 0;
    return QG_OK;
}

int qg_model_seq_len(const qg_model *m, size_t *len)
{
    if (!m || !len) return QG_ERR_INVALID_ARG;
    *len = m->seq;
    return QG_OK;
}

int qg_model_forward(qg_model *m, uint32_t token, uint32_t pos, float *logits)
{
    if (!m) return QG_ERR_INVALID_ARG;
    if (!complete(m)) return mfail(m, QG_ERR_INVALID_ARG, "model matrices / final norm not all set");
    const qg_model_config &c = m->cfg;
    if (token >= c.vocab_size) return mfail(m, QG_ERR_SHAPE, "token id >= vocab_size");
    if (m->seq >= c.max_seq_len || pos >= c.max_seq_len)
        return mfail(m, QG_ERR_SHAPE, "KV cache full (max_seq_len)");   // kv_cache.rs:54-59
    QGM_HIP(m, hipSetDevice(m->ctx->device));
    hipStream_t st = m->ctx->stream;
    ihipStream_t *sti = (ihipStream_t *)st;
    const uint32_t E = c.embed_dim, H = c.hidden_dim;
    int rc;
    // embedding row into a zeroed buffer (transformer.rs:74-75, quant.rs:152-174)
    if (qg::launch_fill(m->h0, E, 0.0f, sti) || qg::launch_dequantize_row(m->tok->type, m->tok->d, m->tok->rows,
                                                                           m->tok->cols, token, m->h0, sti))
        return mfail(m, QG_ERR_HIP, "embedding", hipGetLastError());
    const uint32_t slot = (uint32_t)m->seq;
    const size_t kv_layer = (size_t)c.max_seq_len * m->kv_dim;
    const float scale = 1.0f / sqrtf((float)m->hd);                      // attention.rs:99
    const size_t att_lds = (m->hd + slot + 1) * sizeof(float);
    for (uint32_t l = 0; l < c.n_layers; l++) {
        // the residual stream entering the layer is h0 (layer 0: the
        // embedding) or h1 + fo, which the Q GEMV also stores to h0
        const float *na = l == 0 ? m->h0 : m->h1, *nb = l == 0 ? m->zeros : m->fo;
        const float *anorm = m->vec[QG_V_ATTN_NORM][l];
        if ((rc = gemv_norm(m, m->w[QG_M_WQ - 2][l], na, nb, anorm, l == 0 ? nullptr : m->h0, m->q)) ||
            (rc = gemv_norm(m, m->w[QG_M_WK - 2][l], na, nb, anorm, nullptr, m->k)) ||
            (rc = gemv_norm(m, m->w[QG_M_WV - 2][l], na, nb, anorm, nullptr, m->v)))
            return rc;
        float *kc = m->kc + l * kv_layer, *vc = m->vc + l * kv_layer;
        const uint32_t pairs = (m->q_dim > m->kv_dim ? m->q_dim : m->kv_dim) / 2;
        hipLaunchKernelGGL(qgm::qkv_post_k, dim3((pairs + 255) / 256), dim3(256), 0, st, m->q, m->k, m->v,
                           m->vec[QG_V_BQ][l], m->vec[QG_V_BK][l], m->vec[QG_V_BV][l], kc, vc, m->cos_t,
                           m->sin_t, m->q_dim, m->kv_dim, m->hd, pos, slot);
        const size_t wlds = (slot + 1 + 4 * (size_t)m->hd) * sizeof(float);
        if (m->hd == 64)
            hipLaunchKernelGGL(qgm::attention_wave_k<1>, dim3(c.n_heads), dim3(256), wlds, st, m->q, kc, vc,
                               m->ao, slot + 1, m->kv_dim, m->n_rep, scale);
        else if (m->hd == 128)
            hipLaunchKernelGGL(qgm::attention_wave_k<2>, dim3(c.n_heads), dim3(256), wlds, st, m->q, kc, vc,
                               m->ao, slot + 1, m->kv_dim, m->n_rep, scale);
        else if (m->hd == 256)
            hipLaunchKernelGGL(qgm::attention_wave_k<4>, dim3(c.n_heads), dim3(256), wlds, st, m->q, kc, vc,
                               m->ao, slot + 1, m->kv_dim, m->n_rep, scale);
        else
            hipLaunchKernelGGL(qgm::attention_k, dim3(c.n_heads), dim3(256), att_lds, st, m->q, kc, vc, m->ao,
                               slot + 1, m->hd, m->kv_dim, m->n_rep, scale);
        if ((rc = launched(m, "attention"))) return rc;
        if ((rc = gemv(m, m->w[QG_M_WO - 2][l], m->ao, m->ao2))) return rc;
        // h1 = h0 + attention output (stored by the gate GEMV); MLP input = ffn_norm(h1)
        const float *fnorm = m->vec[QG_V_FFN_NORM][l];
        if ((rc = gemv_norm(m, m->w[QG_M_GATE - 2][l], m->h0, m->ao2, fnorm, m->h1, m->g)) ||
            (rc = gemv_norm(m, m->w[QG_M_UP - 2][l], m->h0, m->ao2, fnorm, nullptr, m->u)))
            return rc;
        hipLaunchKernelGGL(qgm::silu_mul_k, dim3((H + 255) / 256), dim3(256), 0, st, m->g, m->u, m->hb, H);
        if ((rc = launched(m, "silu*up"))) return rc;
        if ((rc = gemv(m, m->w[QG_M_DOWN - 2][l], m->hb, m->fo))) return rc;
    }
    // final norm of h1 + fo (transformer.rs:87-97) inside the lm_head GEMV
    if ((rc = gemv_norm(m, m->lm, m->h1, m->fo, m->final_norm, nullptr, m->logits))) return rc;
    m->seq += 1;
    if (logits) {
        QGM_HIP(m, hipMemcpyAsync(logits, m->logits, (size_t)c.vocab_size * sizeof(float),
                                  hipMemcpyDeviceToHost, st));
        QGM_HIP(m, hipStreamSynchronize(st));
    }
    return QG_OK;
}

int qg_model_sample_greedy(qg_model *m, const uint32_t *recent, size_t n_recent, float penalty, size_t window,
                           uint32_t *token)
{
    if (!m || !token || (n_recent && !recent)) return QG_ERR_INVALID_ARG;
    // sampler.rs:109-116: the last `window` of the recent tokens
    size_t start = n_recent > window ? n_recent - window : 0;
    size_t n = n_recent - start;
    if (n > kRecentMax) { start += n - kRecentMax; n = kRecentMax; }
    hipStream_t st = m->ctx->stream;
    QGM_HIP(m, hipSetDevice(m->ctx->device));
    if (n) {
        std::memcpy(m->h_recent, recent + start, n * sizeof(uint32_t));
        QGM_HIP(m, hipMemcpyAsync(m->d_recent, m->h_recent, n * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    }
    // sampler.rs:76-78: no penalty pass without recent tokens or with penalty 1
    hipLaunchKernelGGL(qgm::sample_greedy_k, dim3(1), dim3(qgm::kBlock), 0, st, m->logits, m->cfg.vocab_size,
                       m->d_recent, (uint32_t)n, n ? penalty : 1.0f, m->d_token);
    int rc = launched(m, "sample");
    if (rc) return rc;
    QGM_HIP(m, hipMemcpyAsync(m->h_token, m->d_token, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    QGM_HIP(m, hipStreamSynchronize(st));
    *token = *m->h_token;
    return QG_OK;
}

int qg_model_generate(qg_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_new, float penalty,
                      size_t window, uint32_t *out_tokens, double *prefill_s, double *decode_s)
{
    if (!m || (n_prompt && !prompt) || (n_new && !out_tokens)) return QG_ERR_INVALID_ARG;
    if (n_prompt == 0 && n_new > 0) return mfail(m, QG_ERR_INVALID_ARG, "generation needs a prompt");
    using clk = std::chrono::steady_clock;
    std::vector<uint32_t> all(prompt, prompt + n_prompt);
    m->seq = 0;                                                     // fresh caches (model.rs:341-346)
    auto t0 = clk::now();
    int rc;
    for (size_t p = 0; p < n_prompt; p++)
        if ((rc = qg_model_forward(m, prompt[p], (uint32_t)p, nullptr))) return rc;
    QGM_HIP(m, hipStreamSynchronize(m->ctx->stream));
    auto t1 = clk::now();
    size_t pos = n_prompt;
    for (size_t s = 0; s < n_new; s++) {
        const size_t nr = all.size() > kRecentMax ? kRecentMax : all.size();   // model.rs:370-374
        uint32_t tok;
        if ((rc = qg_model_sample_greedy(m, all.data() + all.size() - nr, nr, penalty, window, &tok))) return rc;
        out_tokens[s] = tok;
        if ((rc = qg_model_forward(m, tok, (uint32_t)pos, nullptr))) return rc;
        all.push_back(tok);
        pos++;
    }
    QGM_HIP(m, hipStreamSynchronize(m->ctx->stream));
    auto t2 = clk::now();
    if (prefill_s) *prefill_s = std::chrono::duration<double>(t1 - t0).count();
    if (decode_s) *decode_s = std::chrono::duration<double>(t2 - t1).count();
    return QG_OK;
}

}  // extern "C"

void qg_models_free_all(qg_ctx *ctx)
{
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    while (!ctx->models.empty()) free_model(*ctx->models.begin());
}
