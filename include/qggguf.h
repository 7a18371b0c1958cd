/*
 * qggguf.h -- GGUF v3 reader and the upload-once model loader of libqgemv.
 *
 * Replaces GgufFile::load / parse (src/gguf.rs:255-341), the metadata
 * accessors (gguf.rs:160-213), ModelConfig::from_metadata (src/model.rs:49-117)
 * and the weight part of Model::load (src/model.rs:136-329).  The file is
 * memory-mapped; tensor bytes are never copied on the host, and the loader
 * uploads each GGUF tensor to HBM once (a tied lm_head shares token_embd's
 * device copy instead of the reference's clone, model.rs:225).
 *
 * Status codes are qg_status values (qgemv.h); qg_gguf_last_error gives the
 * reason of the last failure of a handle, qg_gguf_open_error the reason an
 * open failed.
 */
#ifndef QGGGUF_H
#define QGGGUF_H

#include <stddef.h>
#include <stdint.h>

#include "qgemv.h"
#include "qgmodel.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qg_gguf qg_gguf;

/* Metadata value types (gguf.rs:15-17). */
enum {
    QG_GGUF_U8 = 0, QG_GGUF_I8 = 1, QG_GGUF_U16 = 2, QG_GGUF_I16 = 3, QG_GGUF_U32 = 4,
    QG_GGUF_I32 = 5, QG_GGUF_F32 = 6, QG_GGUF_BOOL = 7, QG_GGUF_STRING = 8, QG_GGUF_ARRAY = 9,
    QG_GGUF_U64 = 10, QG_GGUF_I64 = 11, QG_GGUF_F64 = 12
};

/* GgufFile::load (gguf.rs:255-341): magic "GGUF", version 3 only, the
 * metadata key/value pairs, the tensor descriptors (unknown tensor type ids
 * fail the whole file, as gguf.rs:312-318), data section at the next multiple
 * of 32 bytes after the descriptors (gguf.rs:330-331; general.alignment is not
 * consulted).  Also fails if a tensor's bytes lie past the end of the file. */
int qg_gguf_open(const char *path, qg_gguf **out);
int qg_gguf_close(qg_gguf *g);
const char *qg_gguf_last_error(const qg_gguf *g);
/* Reason of the last failed qg_gguf_open on this thread. */
const char *qg_gguf_open_error(void);

int qg_gguf_version(const qg_gguf *g, uint32_t *version);
int qg_gguf_data_offset(const qg_gguf *g, uint64_t *offset);

/* Metadata.  The numeric getters follow MetadataValue::to_u64 / to_f32
 * (gguf.rs:160-184): u64 accepts UINT64, INT64 and UINT32 values; f32
 * accepts FLOAT32 and FLOAT64.  QG_ERR_SHAPE when the key is missing or of
 * another type.  qg_gguf_get_string copies at most cap-1 bytes plus a NUL
 * and reports the full length.  Arrays: element type and count. */
int qg_gguf_metadata_count(const qg_gguf *g, size_t *n);
int qg_gguf_metadata_type(const qg_gguf *g, const char *key, uint32_t *type);
int qg_gguf_get_u64(const qg_gguf *g, const char *key, uint64_t *value);
int qg_gguf_get_f32(const qg_gguf *g, const char *key, float *value);
int qg_gguf_get_string(const qg_gguf *g, const char *key, char *buf, size_t cap, size_t *len);
int qg_gguf_get_array_info(const qg_gguf *g, const char *key, uint32_t *elem_type, uint64_t *count);

/* Tensor descriptors (TensorInfo, gguf.rs:218-240).  dims: up to 4 values,
 * ne0 first.  nbytes = the byte size Model::load reads for the type
 * (model.rs:176-187: ceil(n_elements / block) * block_bytes; 0 for the types
 * it skips).  offset is relative to the data section. */
int qg_gguf_tensor_count(const qg_gguf *g, size_t *n);
int qg_gguf_find_tensor(const qg_gguf *g, const char *name, size_t *index);
int qg_gguf_tensor_info(const qg_gguf *g, size_t index, const char **name, uint32_t *ggml_type,
                        uint32_t *n_dims, uint64_t dims[4], uint64_t *offset, size_t *nbytes);
/* The tensor's bytes inside the mapping (valid until qg_gguf_close). */
int qg_gguf_tensor_data(const qg_gguf *g, size_t index, const void **data, size_t *nbytes);

/* ModelConfig::from_metadata (model.rs:49-117): keys "<arch>.embedding_length",
 * "block_count", "attention.head_count", "attention.head_count_kv",
 * "feed_forward_length", "vocab_size", "context_length", "rope.freq_base",
 * "attention.layer_norm_rms_epsilon" (else "attention.layer_norm_epsilon",
 * else 1e-5) with arch = general.architecture (default "llama"), and the
 * reference's per-architecture defaults for missing or zero values.
 * max_seq_len != 0 replaces context_length, as Model::load's argument does
 * (model.rs:141-143). */
int qg_gguf_model_config(const qg_gguf *g, uint32_t max_seq_len, qg_model_config *cfg);

/* Model::load's weights (model.rs:136-329) into a new decode-step engine:
 * token_embd (vocab x embed), output_norm, output.weight (rows ne1, cols ne0)
 * or, when absent, token_embd shared on device, and per layer attn_norm,
 * attn_q/k/v/output, the optional attn_q/k/v biases (zeros when absent),
 * ffn_norm, ffn_gate/up/down.  Norms and biases stored in a type other than
 * F32 load as zeros, as the reference does (model.rs:211-216).  A missing
 * tensor or a skipped type fails with QG_ERR_SHAPE naming it. */
int qg_model_load_gguf(qg_ctx *ctx, const char *path, uint32_t max_seq_len, qg_model **out);

#ifdef __cplusplus
}
#endif

#endif /* QGGGUF_H */
