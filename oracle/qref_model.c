/*
 * oracle/qref_model.c -- CPU restatement of one decode step of
 * yudono/rust-inference (transformer.rs, attention.rs, mlp.rs, rmsnorm.rs,
 * rope.rs, kv_cache.rs) on top of qref.c's quantized mat-vec.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the on-device decode step.
 *
 * qref_mat_vec_mul_rows() is the quant.rs:188-205 loop reordered by row:
 * for a fixed output row the reference adds w*x terms in increasing column
 * order starting from 0.0 (flat index order), and so does this loop, so the
 * two produce bit-identical results (checked by tests/test_oracle.py); the
 * reordering only removes the per-element div/mod and lets rows run on
 * several threads so that multi-token parity runs finish in seconds.
 */
#include "qref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    const uint8_t *data;
    size_t nbytes;
    uint32_t dtype;
    size_t rows, cols;
} qref_mat;

/* Row-ordered, optionally multi-threaded equivalent of qref_mat_vec_mul. */
void qref_mat_vec_mul_rows(const uint8_t *data, size_t nbytes, uint32_t dtype,
                           size_t rows, size_t cols, const float *x, float *out)
{
    size_t bs = qref_block_size(dtype);
    if (bs == 0) { for (size_t r = 0; r < rows; r++) out[r] = 0.0f; return; }
    long long nr = (long long)rows;
#pragma omp parallel for schedule(static)
    for (long long rr = 0; rr < nr; rr++) {
        size_t r = (size_t)rr;
        float buf[256];
        memset(buf, 0, sizeof buf);
        size_t f0 = r * cols, f1 = f0 + cols;
        float sum = 0.0f;
        size_t f = f0;
        while (f < f1) {
            size_t b = f / bs;
            qref_dequantize_block(data, nbytes, dtype, b, buf);
            size_t bend = (b + 1) * bs < f1 ? (b + 1) * bs : f1;
            for (; f < bend; f++) sum += buf[f - b * bs] * x[f - f0];
        }
        out[r] = sum;
    }
}

typedef struct {
    size_t embed_dim, n_layers, n_heads, n_kv_heads, hidden_dim, vocab_size, max_seq_len;
    float rope_base, norm_eps;
    qref_mat token_embd, lm_head;
    const float *final_norm;
    qref_mat *wq, *wk, *wv, *wo, *gate, *up, *down;   /* [n_layers] */
    const float **attn_norm, **ffn_norm, **bq, **bk, **bv;
    /* state */
    float *kcache, *vcache;     /* [n_layers][max_seq_len][kv_dim] */
    size_t *seq_len;            /* [n_layers] */
    float *cos_t, *sin_t;       /* [max_seq_len][head_dim/2] */
} qref_model;

enum { QM_TOKEN_EMBD = 0, QM_LM_HEAD, QM_WQ, QM_WK, QM_WV, QM_WO, QM_GATE, QM_UP, QM_DOWN };
enum { QV_FINAL_NORM = 0, QV_ATTN_NORM, QV_FFN_NORM, QV_BQ, QV_BK, QV_BV };

qref_model *qref_model_create(size_t embed_dim, size_t n_layers, size_t n_heads,
                              size_t n_kv_heads, size_t hidden_dim, size_t vocab_size,
                              size_t max_seq_len, float rope_base, float norm_eps)
{
    qref_model *m = (qref_model *)calloc(1, sizeof *m);
    if (!m) return NULL;
    m->embed_dim = embed_dim; m->n_layers = n_layers; m->n_heads = n_heads;
    m->n_kv_heads = n_kv_heads; m->hidden_dim = hidden_dim; m->vocab_size = vocab_size;
    m->max_seq_len = max_seq_len; m->rope_base = rope_base; m->norm_eps = norm_eps;
    size_t L = n_layers;
    m->wq = calloc(L, sizeof(qref_mat)); m->wk = calloc(L, sizeof(qref_mat));
    m->wv = calloc(L, sizeof(qref_mat)); m->wo = calloc(L, sizeof(qref_mat));
    m->gate = calloc(L, sizeof(qref_mat)); m->up = calloc(L, sizeof(qref_mat));
    m->down = calloc(L, sizeof(qref_mat));
    m->attn_norm = calloc(L, sizeof(float *)); m->ffn_norm = calloc(L, sizeof(float *));
    m->bq = calloc(L, sizeof(float *)); m->bk = calloc(L, sizeof(float *));
    m->bv = calloc(L, sizeof(float *));
    size_t head_dim = embed_dim / n_heads;                       /* model.rs:153 */
    size_t kv_dim = n_kv_heads * head_dim;
    m->kcache = calloc(L * max_seq_len * kv_dim + 1, sizeof(float));
    m->vcache = calloc(L * max_seq_len * kv_dim + 1, sizeof(float));
    m->seq_len = calloc(L, sizeof(size_t));
    m->cos_t = calloc(max_seq_len * (head_dim / 2) + 1, sizeof(float));
    m->sin_t = calloc(max_seq_len * (head_dim / 2) + 1, sizeof(float));
    qref_rope_tables(head_dim, rope_base, max_seq_len, m->cos_t, m->sin_t);
    return m;
}

void qref_model_destroy(qref_model *m)
{
    if (!m) return;
    free(m->wq); free(m->wk); free(m->wv); free(m->wo); free(m->gate); free(m->up);
    free(m->down); free(m->attn_norm); free(m->ffn_norm); free(m->bq); free(m->bk);
    free(m->bv); free(m->kcache); free(m->vcache); free(m->seq_len); free(m->cos_t);
    free(m->sin_t); free(m);
}

/* The caller keeps the bytes alive; the oracle only borrows them. */
int qref_model_set_mat(qref_model *m, int which, size_t layer, const uint8_t *data,
                       size_t nbytes, uint32_t dtype, size_t rows, size_t cols)
{
    qref_mat q = { data, nbytes, dtype, rows, cols };
    if (which != QM_TOKEN_EMBD && which != QM_LM_HEAD && layer >= m->n_layers) return -1;
    switch (which) {
    case QM_TOKEN_EMBD: m->token_embd = q; break;
    case QM_LM_HEAD: m->lm_head = q; break;
    case QM_WQ: m->wq[layer] = q; break;
    case QM_WK: m->wk[layer] = q; break;
    case QM_WV: m->wv[layer] = q; break;
    case QM_WO: m->wo[layer] = q; break;
    case QM_GATE: m->gate[layer] = q; break;
    case QM_UP: m->up[layer] = q; break;
    case QM_DOWN: m->down[layer] = q; break;
    default: return -1;
    }
    return 0;
}

int qref_model_set_vec(qref_model *m, int which, size_t layer, const float *v)
{
    if (which != QV_FINAL_NORM && layer >= m->n_layers) return -1;
    switch (which) {
    case QV_FINAL_NORM: m->final_norm = v; break;
    case QV_ATTN_NORM: m->attn_norm[layer] = v; break;
    case QV_FFN_NORM: m->ffn_norm[layer] = v; break;
    case QV_BQ: m->bq[layer] = v; break;
    case QV_BK: m->bk[layer] = v; break;
    case QV_BV: m->bv[layer] = v; break;
    default: return -1;
    }
    return 0;
}

void qref_model_reset(qref_model *m)
{
    for (size_t l = 0; l < m->n_layers; l++) m->seq_len[l] = 0;      /* kv_cache.rs:232 */
}

static void mv(const qref_mat *q, const float *x, float *out)
{
    qref_mat_vec_mul_rows(q->data, q->nbytes, q->dtype, q->rows, q->cols, x, out);
}

static float dotp(const float *a, const float *b, size_t n)    /* math.rs:63-70 */
{
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* attention.rs:54-124 */
static int attention(qref_model *m, size_t l, const float *x, size_t pos, float *output)
{
    size_t hd = m->embed_dim / m->n_heads, kv_dim = m->n_kv_heads * hd;
    size_t q_dim = m->n_heads * hd, n_rep = m->n_heads / m->n_kv_heads;
    float *q = calloc(q_dim, sizeof(float)), *k = calloc(kv_dim, sizeof(float));
    float *v = calloc(kv_dim, sizeof(float)), *ao = calloc(q_dim, sizeof(float));
    if (m->seq_len[l] >= m->max_seq_len) { free(q); free(k); free(v); free(ao); return -1; }
    mv(&m->wq[l], x, q);
    if (m->bq[l]) for (size_t i = 0; i < q_dim; i++) q[i] += m->bq[l][i];
    mv(&m->wk[l], x, k);
    if (m->bk[l]) for (size_t i = 0; i < kv_dim; i++) k[i] += m->bk[l][i];
    mv(&m->wv[l], x, v);
    if (m->bv[l]) for (size_t i = 0; i < kv_dim; i++) v[i] += m->bv[l][i];
    for (size_t h = 0; h < m->n_heads; h++)
        qref_rope_apply(q + h * hd, hd, pos, m->cos_t, m->sin_t, m->max_seq_len);
    for (size_t h = 0; h < m->n_kv_heads; h++)
        qref_rope_apply(k + h * hd, hd, pos, m->cos_t, m->sin_t, m->max_seq_len);
    float *kc = m->kcache + l * m->max_seq_len * kv_dim;
    float *vc = m->vcache + l * m->max_seq_len * kv_dim;
    memcpy(kc + m->seq_len[l] * kv_dim, k, kv_dim * sizeof(float));  /* kv_cache.rs:52-73 */
    memcpy(vc + m->seq_len[l] * kv_dim, v, kv_dim * sizeof(float));
    m->seq_len[l] += 1;
    size_t seq = m->seq_len[l];
    float *scores = malloc(seq * sizeof(float));
    float scale = 1.0f / sqrtf((float)hd);                         /* attention.rs:99 */
    for (size_t h = 0; h < m->n_heads; h++) {
        size_t qs = h * hd, kvh = (h / n_rep) * hd;
        for (size_t j = 0; j < seq; j++) scores[j] = dotp(q + qs, kc + j * kv_dim + kvh, hd) * scale;
        qref_softmax_inplace(scores, seq);
        for (size_t j = 0; j < seq; j++) {
            const float *vv = vc + j * kv_dim + kvh;
            for (size_t d = 0; d < hd; d++) ao[qs + d] += scores[j] * vv[d];
        }
    }
    mv(&m->wo[l], ao, output);
    free(scores); free(q); free(k); free(v); free(ao);
    return 0;
}

/* mlp.rs:31-46 */
static void mlp(qref_model *m, size_t l, const float *x, float *output)
{
    size_t H = m->hidden_dim;
    float *g = malloc(H * sizeof(float)), *u = malloc(H * sizeof(float));
    float *hbuf = malloc(H * sizeof(float));
    mv(&m->gate[l], x, g);
    for (size_t i = 0; i < H; i++) g[i] = qref_silu(g[i]);
    mv(&m->up[l], x, u);
    for (size_t i = 0; i < H; i++) hbuf[i] = g[i] * u[i];
    mv(&m->down[l], hbuf, output);
    free(g); free(u); free(hbuf);
}

/* transformer.rs:63-98 with TransformerLayer::forward (transformer.rs:20-48).
 * Returns 0, or -1 on KV overflow (kv_cache.rs:54-59 panics). */
int qref_model_forward(qref_model *m, size_t token_id, size_t pos, float *logits)
{
    size_t E = m->embed_dim;
    float *hidden = calloc(E, sizeof(float)), *out = calloc(E, sizeof(float));
    float *xn = calloc(E, sizeof(float)), *ao = calloc(E, sizeof(float));
    float *xn2 = calloc(E, sizeof(float)), *fo = calloc(E, sizeof(float));
    int rc = 0;
    qref_dequantize_row(m->token_embd.data, m->token_embd.nbytes, m->token_embd.dtype,
                        m->token_embd.rows, m->token_embd.cols, token_id, hidden);
    for (size_t l = 0; l < m->n_layers && rc == 0; l++) {
        qref_rmsnorm(hidden, m->attn_norm[l], xn, E, m->norm_eps);
        memset(ao, 0, E * sizeof(float));
        rc = attention(m, l, xn, pos, ao);
        if (rc) break;
        for (size_t i = 0; i < E; i++) out[i] = hidden[i] + ao[i];
        qref_rmsnorm(out, m->ffn_norm[l], xn2, E, m->norm_eps);
        mlp(m, l, xn2, fo);
        for (size_t i = 0; i < E; i++) out[i] += fo[i];
        float *t = hidden; hidden = out; out = t;                  /* transformer.rs:87 */
    }
    if (rc == 0) {
        qref_rmsnorm_inplace(hidden, m->final_norm, E, m->norm_eps);
        mv(&m->lm_head, hidden, logits);
    }
    free(hidden); free(out); free(xn); free(ao); free(xn2); free(fo);
    return rc;
}
