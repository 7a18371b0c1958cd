/*
 * qgmodel.h -- C ABI of the on-device decode step built on libqgemv.
 *
 * One decode step of yudono/rust-inference with every tensor resident in HBM:
 * Transformer::forward (src/transformer.rs:63-98, TransformerLayer::forward
 * 20-48), Attention::forward (src/attention.rs:54-124), Mlp::forward
 * (src/mlp.rs:31-46), RmsNorm (src/rmsnorm.rs:14-29, src/math.rs:237-273),
 * RoPE (src/rope.rs:42-96), KVCache (src/kv_cache.rs:40-90), and the greedy
 * path of Sampler::sample with its repetition penalty (src/sampler.rs:72-83,
 * 109-127) inside Model::generate's token loop (src/model.rs:330-440, without
 * the tokenizer).  Activations, the KV cache and the logits stay on device;
 * every mat-vec is the library's GEMV on the raw GGUF blocks.
 *
 * Status codes are qg_status values (qgemv.h).  A model belongs to one
 * context and is not thread safe.
 */
#ifndef QGMODEL_H
#define QGMODEL_H

#include <stddef.h>
#include <stdint.h>

#include "qgemv.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qg_model qg_model;

/* ModelConfig (src/model.rs:34-46); head_dim = embed_dim / n_heads (model.rs:153). */
typedef struct qg_model_config {
    uint32_t embed_dim, n_layers, n_heads, n_kv_heads, hidden_dim, vocab_size, max_seq_len;
    float rope_base, norm_eps;
} qg_model_config;

/* Matrix slots, named after the GGUF tensors the reference loads
 * (src/model.rs:197-298).  Shapes (rows x cols): TOKEN_EMBD vocab x embed,
 * LM_HEAD vocab x embed, WQ q_dim x embed, WK / WV kv_dim x embed,
 * WO embed x q_dim, GATE / UP hidden x embed, DOWN embed x hidden. */
enum {
    QG_M_TOKEN_EMBD = 0, QG_M_LM_HEAD = 1, QG_M_WQ = 2, QG_M_WK = 3, QG_M_WV = 4,
    QG_M_WO = 5, QG_M_GATE = 6, QG_M_UP = 7, QG_M_DOWN = 8
};
/* f32 vector slots: norms (embed) and attention biases (q_dim / kv_dim);
 * a bias never set is zero, as model.rs:251-281 defaults it. */
enum {
    QG_V_FINAL_NORM = 0, QG_V_ATTN_NORM = 1, QG_V_FFN_NORM = 2, QG_V_BQ = 3, QG_V_BK = 4,
    QG_V_BV = 5
};

/* Model::load's allocation of the decode state (src/model.rs:136-160, 340-346):
 * KV caches of max_seq_len positions per layer, RoPE tables, activations. */
int qg_model_create(qg_ctx *ctx, const qg_model_config *cfg, qg_model **out);
int qg_model_destroy(qg_model *m);

/* load_mat! (src/model.rs:197-203): uploads raw GGUF bytes for slot `which`
 * of layer `layer` (ignored for TOKEN_EMBD / LM_HEAD).  The shape is checked
 * against the configuration. */
int qg_model_set_matrix(qg_model *m, uint32_t which, uint32_t layer, const void *raw,
                        size_t nbytes, uint32_t ggml_type, size_t rows, size_t cols);
/* Uses an already uploaded matrix (e.g. a tied lm_head = token_embd,
 * src/model.rs:221-226) without copying; the model does not free it, and
 * qg_mat_free refuses it while any model slot still uses it (the slot is
 * released when the model is destroyed or the slot gets another matrix).
 * QG_ERR_INVALID_ARG for a handle that is not a live matrix of the model's
 * context; QG_ERR_SHAPE for a shape that does not match the slot. */
int qg_model_share_matrix(qg_model *m, uint32_t which, uint32_t layer, const qg_mat *mat);
int qg_model_set_vector(qg_model *m, uint32_t which, uint32_t layer, const float *v, size_t n);

/* No counterpart in the reference: replay each forward pass (and generate's
 * sample + forward step) from a HIP graph captured on first use (enable != 0,
 * the default), or enqueue the kernels one by one (enable == 0).  Both run the
 * same kernels on the same data and give bit-identical results. */
int qg_model_use_graphs(qg_model *m, int enable);

/* KVCache::clear for every layer (src/kv_cache.rs:232). */
int qg_model_reset(qg_model *m);
/* Number of positions currently in the caches. */
int qg_model_seq_len(const qg_model *m, size_t *len);

/* Transformer::forward(token, pos, ...) (src/transformer.rs:63-98): appends
 * one position to every cache and leaves the logits on device.  `logits`,
 * if not NULL, receives vocab_size floats (host memory).  QG_ERR_SHAPE when
 * the caches are full (kv_cache.rs:54-59 panics there) or token >= vocab. */
int qg_model_forward(qg_model *m, uint32_t token, uint32_t pos, float *logits);

/* The prompt loop of Model::generate (src/model.rs:361-365): n forward passes
 * of tokens[0..n) at positions seq, seq + 1, ... (seq = the positions already
 * cached), leaving the caches and the device logits as those n calls of
 * qg_model_forward would -- the logits are the last token's.  Chunks of up to
 * 64 tokens go through each layer together, every projection one f16 MFMA
 * GEMM over the tokens' x split into two f16 pieces under a power-of-two
 * scale per 256 elements (batched prefill, exact products, f32
 * accumulation) and the attention on f32 MFMAs, when every layer matrix is
 * Q4_K, Q5_K, Q6_K or Q8_0 with cols % 128 == 0 and head_dim is 64, 128 or
 * 256; otherwise, or after qg_model_use_batched_prefill(m, 0), one forward
 * pass per token.  `logits`,
 * if not NULL, receives vocab_size floats (host memory).  QG_ERR_SHAPE when
 * the tokens would not fit the caches or a token >= vocab. */
int qg_model_prefill(qg_model *m, const uint32_t *tokens, size_t n, float *logits);
/* No counterpart in the reference: batched prefill in qg_model_prefill and
 * qg_model_generate where it applies (enable != 0, the default), or one
 * forward pass per prompt token (enable == 0). */
int qg_model_use_batched_prefill(qg_model *m, int enable);
/* No counterpart in the reference (tuning and tests): the decode step's
 * attention for head_dim 64, 128 and 256 -- path 0 (the default) by length:
 * up to 512 cached positions each query head in two workgroups (even and odd
 * positions) merged in the output projection's input where every wo matrix
 * allows it (a fixed-point type with whole blocks per row), else in one
 * workgroup; split over position ranges and merged beyond.  1 always one
 * workgroup per head; 2 always split; 3 always two workgroups per head where
 * allowed.  All compute attention.rs:93-121; they differ in summation order
 * only. */
int qg_model_set_attention_path(qg_model *m, int path);
/* No counterpart in the reference (memory accounting): device bytes the
 * model reads.  weights: every distinct matrix it uses (token_embd, lm_head,
 * layer matrices, the stacked [Q;K;V] / [gate; up] matrices the decode step
 * builds), each counted with the copies it holds (tail pads included);
 * file_bytes: the quantized bytes of its slots (what a GGUF file holds for
 * them); total: weights plus the norms, biases, KV caches, RoPE tables and
 * activation buffers.  Uploaded Q8_0/Q4_K/Q5_K/Q6_K matrices are held once,
 * in the repacked layout; layer parts the model owns are views into their
 * stacked matrix; token_embd is held in the GGUF layout (and repacked too
 * only when it is also the lm_head).  Any output may be NULL. */
int qg_model_resident_bytes(qg_model *m, size_t *weights, size_t *file_bytes, size_t *total);

/* Greedy Sampler::sample on the device logits of the last forward:
 * repetition penalty over `recent` (the last `window` entries, applied in
 * order, sampler.rs:109-127) then argmax (math.rs:328-339).  Modifies the
 * device logits as the reference modifies its slice. */
int qg_model_sample_greedy(qg_model *m, const uint32_t *recent, size_t n_recent, float penalty,
                           size_t window, uint32_t *token);

/* Model::generate's loop (src/model.rs:357-440) without the tokenizer and
 * without stop tokens: the prompt as in qg_model_prefill, then n_new times sample
 * (over the last 64 tokens, as model.rs:370-374 passes them) + forward.
 * out_tokens receives the n_new sampled tokens.  *prefill_s / *decode_s (if
 * not NULL) receive the wall seconds of the two phases. */
int qg_model_generate(qg_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_new,
                      float penalty, size_t window, uint32_t *out_tokens, double *prefill_s,
                      double *decode_s);

#ifdef __cplusplus
}
#endif

#endif /* QGMODEL_H */
