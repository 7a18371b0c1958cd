// qg_gguf.cpp -- GGUF v3 reader and upload-once model loader (include/qggguf.h).
//
// Host code.  The file is memory-mapped read-only and parsed in place:
// GgufFile::parse (src/gguf.rs:261-341) with the value readers of
// gguf.rs:370-485, ModelConfig::from_metadata (src/model.rs:50-117) and the
// weight part of Model::load (src/model.rs:136-329).  Tensor bytes go from the
// mapping straight to HBM (qg_upload), once per tensor.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "qg_common.h"
#include "qg_internal.h"
#include "qggguf.h"
#include "qgmodel.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;     // "GGUF" little-endian (gguf.rs:33)
constexpr uint32_t kVersion = 3;             // gguf.rs:34
constexpr uint64_t kAlign = 32;              // gguf.rs:35

struct Value {
    uint32_t type = 0;
    uint64_t u = 0;          // integer / bool payload (sign-extended for signed types)
    double f = 0.0;          // float payload
    std::string s;           // string payload
    uint32_t elem_type = 0;  // arrays
    uint64_t count = 0;
};

struct Tensor {
    std::string name;
    uint32_t type = 0;
    std::vector<uint64_t> dims;
    uint64_t offset = 0;     // relative to the data section
};

thread_local std::string g_open_error;

}  // namespace

struct qg_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    std::unordered_map<std::string, Value> meta;
    std::vector<Tensor> tensors;
    uint64_t data_offset = 0;
    std::string err;
};

namespace {

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
    const uint8_t *p;
    size_t n, pos = 0;
    bool ok = true;
    bool take(size_t k, const uint8_t **out)
    {
        if (!ok || k > n - pos) { ok = false; return false; }
        *out = p + pos;
        pos += k;
        return true;
    }
    uint64_t le(size_t k)
    {
        const uint8_t *b;
        if (!take(k, &b)) return 0;
        uint64_t v = 0;
        for (size_t i = 0; i < k; i++) v |= (uint64_t)b[i] << (8 * i);
        return v;
    }
    std::string str()                                      // gguf.rs:422-428
    {
        const uint64_t len = le(8);
        const uint8_t *b;
        if (!ok || len > n - pos) { ok = false; return std::string(); }
        take((size_t)len, &b);
        return std::string((const char *)b, (size_t)len);
    }
};

// String::from_utf8's rule: well-formed UTF-8 (no overlong forms, no
// surrogates, nothing above U+10FFFF)
bool utf8_valid(const std::string &s)
{
    const unsigned char *p = (const unsigned char *)s.data();
    const size_t n = s.size();
    size_t i = 0;
    while (i < n) {
        const unsigned c = p[i];
        if (c < 0x80) { i++; continue; }
        size_t k;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) { k = 1; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { k = 2; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { k = 3; cp = c & 0x07; }
        else return false;
        if (k >= n - i) return false;                      // needs bytes i+1 .. i+k
        for (size_t j = 1; j <= k; j++) {
            if ((p[i + j] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (p[i + j] & 0x3F);
        }
        if ((k == 1 && cp < 0x80) || (k == 2 && cp < 0x800) || (k == 3 && cp < 0x10000) || cp > 0x10FFFF ||
            (cp >= 0xD800 && cp <= 0xDFFF))
            return false;
        i += k + 1;
    }
    return true;
}

// One value of a known type (read_metadata_value_by_type, gguf.rs:465-485);
// arrays only at the top level (read_metadata_value, gguf.rs:431-462).
bool read_value(Cursor &c, uint32_t type, bool top, Value *v, std::string *err)
{
    v->type = type;
    switch (type) {
    case QG_GGUF_U8: v->u = c.le(1); break;
    case QG_GGUF_I8: v->u = (uint64_t)(int64_t)(int8_t)c.le(1); break;
    case QG_GGUF_U16: v->u = c.le(2); break;
    case QG_GGUF_I16: v->u = (uint64_t)(int64_t)(int16_t)c.le(2); break;
    case QG_GGUF_U32: v->u = c.le(4); break;
    case QG_GGUF_I32: v->u = (uint64_t)(int64_t)(int32_t)c.le(4); break;
    case QG_GGUF_F32: {
        const uint32_t b = (uint32_t)c.le(4);
        float f;
        std::memcpy(&f, &b, 4);
        v->f = f;
        break;
    }
    case QG_GGUF_BOOL: v->u = c.le(1) != 0; break;
    case QG_GGUF_STRING:
        v->s = c.str();
        if (c.ok && !utf8_valid(v->s)) { *err = "invalid UTF-8 in a string"; return false; }
        break;
    case QG_GGUF_U64: v->u = c.le(8); break;
    case QG_GGUF_I64: v->u = c.le(8); break;
    case QG_GGUF_F64: {
        const uint64_t b = c.le(8);
        std::memcpy(&v->f, &b, 8);
        break;
    }
    case QG_GGUF_ARRAY: {
        if (!top) { *err = "unknown metadata array element type: 9"; return false; }
        v->elem_type = (uint32_t)c.le(4);
        v->count = c.le(8);
        Value e;
        for (uint64_t i = 0; i < v->count && c.ok; i++)
            if (!read_value(c, v->elem_type, false, &e, err)) return false;
        break;
    }
    default: {
        char b[64];
        snprintf(b, sizeof b, "unknown metadata value type: %u", type);
        *err = b;
        return false;
    }
    }
    if (!c.ok) { *err = "file ends inside the header"; return false; }
    return true;
}

// GgufDataType::from_u32 (gguf.rs:62-78): ids 0-3, 6-14
bool known_type(uint32_t t) { return t <= 3 || (t >= 6 && t <= 14); }

// Element count of a tensor (the product of its dims); false when the
// product does not fit in 64 bits (a crafted header), which no tensor of a
// real file reaches.
bool n_elements(const Tensor &t, uint64_t *n)
{
    uint64_t p = 1;
    for (uint64_t d : t.dims) {
        if (d != 0 && p > UINT64_MAX / d) return false;
        p *= d;
    }
    *n = p;
    return true;
}

// Bytes Model::load reads for a tensor (model.rs:166-180): *nb = 0 for a
// type the loader skips.  False when the tensor's element or byte count
// overflows 64 bits.
bool load_bytes(const Tensor &t, uint64_t *nb)
{
    uint64_t n;
    if (!n_elements(t, &n)) return false;
    const uint64_t bs = qg::block_elems(t.type), bb = qg::block_bytes(t.type);
    if (bb == 0) { *nb = 0; return true; }
    const uint64_t blocks = n / bs + (n % bs != 0);
    if (blocks > UINT64_MAX / bb) return false;
    *nb = blocks * bb;
    return true;
}

int gfail(qg_gguf *g, int st, const std::string &what)
{
    g->err = what;
    return st;
}

void unmap(qg_gguf *g)
{
    if (g->map) munmap((void *)g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    g->map = nullptr;
    g->fd = -1;
}

int parse(qg_gguf *g)
{
    Cursor c{g->map, g->size};
    const uint32_t magic = (uint32_t)c.le(4);
    if (!c.ok || magic != kMagic) return gfail(g, QG_ERR_INVALID_ARG, "invalid GGUF magic");
    g->version = (uint32_t)c.le(4);
    if (!c.ok || g->version != kVersion) return gfail(g, QG_ERR_INVALID_ARG, "unsupported GGUF version (only v3)");
    const uint64_t n_tensors = c.le(8), n_kv = c.le(8);
    if (!c.ok) return gfail(g, QG_ERR_SHORT_DATA, "file ends inside the header");
    std::string err;
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key = c.str();
        if (!c.ok) return gfail(g, QG_ERR_SHORT_DATA, "file ends inside the metadata");
        if (!utf8_valid(key)) return gfail(g, QG_ERR_INVALID_ARG, "invalid UTF-8 in a key");
        Value v;
        const uint32_t type = (uint32_t)c.le(4);
        if (!c.ok) return gfail(g, QG_ERR_SHORT_DATA, "file ends inside the metadata");
        if (!read_value(c, type, true, &v, &err)) return gfail(g, c.ok ? QG_ERR_INVALID_ARG : QG_ERR_SHORT_DATA, err);
        g->meta[key] = std::move(v);                       // HashMap::insert: the last one wins
    }
    // each descriptor takes at least 24 bytes: no reservation past the file's size
    if (n_tensors > g->size / 24) return gfail(g, QG_ERR_SHORT_DATA, "file ends inside the tensor descriptors");
    g->tensors.reserve((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        Tensor t;
        t.name = c.str();
        const uint32_t nd = (uint32_t)c.le(4);
        if (!c.ok || nd > (g->size - c.pos) / 8) return gfail(g, QG_ERR_SHORT_DATA, "file ends inside the tensor descriptors");
        if (!utf8_valid(t.name)) return gfail(g, QG_ERR_INVALID_ARG, "invalid UTF-8 in a tensor name");
        for (uint32_t d = 0; d < nd; d++) t.dims.push_back(c.le(8));
        t.type = (uint32_t)c.le(4);
        if (c.ok && !known_type(t.type)) {
            char b[64];
            snprintf(b, sizeof b, "unknown tensor data type: %u", t.type);
            return gfail(g, QG_ERR_UNSUPPORTED_TYPE, b);
        }
        t.offset = c.le(8);
        if (!c.ok) return gfail(g, QG_ERR_SHORT_DATA, "file ends inside the tensor descriptors");
        g->tensors.push_back(std::move(t));
    }
    g->data_offset = (c.pos + kAlign - 1) / kAlign * kAlign;   // gguf.rs:328-330
    return QG_OK;
}

const Value *find(const qg_gguf *g, const char *key)
{
    if (!g || !key) return nullptr;
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

// MetadataValue::to_u64 / to_f32 (gguf.rs:171-186)
bool to_u64(const Value *v, uint64_t *out)
{
    if (!v || (v->type != QG_GGUF_U64 && v->type != QG_GGUF_I64 && v->type != QG_GGUF_U32)) return false;
    *out = v->u;
    return true;
}

bool to_f32(const Value *v, float *out)
{
    if (!v || (v->type != QG_GGUF_F32 && v->type != QG_GGUF_F64)) return false;
    *out = (float)v->f;
    return true;
}

}  // namespace

extern "C" {

int qg_gguf_open(const char *path, qg_gguf **out)
{
    if (!path || !out) return QG_ERR_INVALID_ARG;
    *out = nullptr;
    qg_gguf *g = new (std::nothrow) qg_gguf;
    if (!g) return QG_ERR_OUT_OF_MEMORY;
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0) {
        g_open_error = std::string("cannot open ") + path;
        delete g;
        return QG_ERR_INVALID_ARG;
    }
    g->size = (size_t)st.st_size;
    if (g->size > 0) {
        void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
        if (m == MAP_FAILED) {
            g_open_error = std::string("cannot map ") + path;
            unmap(g);
            delete g;
            return QG_ERR_OUT_OF_MEMORY;
        }
        g->map = (const uint8_t *)m;
    }
    int rc;
    try {
        rc = parse(g);
    } catch (const std::bad_alloc &) {      // host memory for the metadata / descriptors
        g->err = "host allocation failed while parsing";
        rc = QG_ERR_OUT_OF_MEMORY;
    } catch (...) {
        g->err = "unexpected error while parsing";
        rc = QG_ERR_INVALID_ARG;
    }
    if (rc) {
        g_open_error = g->err;
        unmap(g);
        delete g;
        return rc;
    }
    *out = g;
    return QG_OK;
}

int qg_gguf_close(qg_gguf *g)
{
    if (!g) return QG_ERR_INVALID_ARG;
    unmap(g);
    delete g;
    return QG_OK;
}

const char *qg_gguf_last_error(const qg_gguf *g) { return g ? g->err.c_str() : ""; }
const char *qg_gguf_open_error(void) { return g_open_error.c_str(); }

int qg_gguf_version(const qg_gguf *g, uint32_t *version)
{
    if (!g || !version) return QG_ERR_INVALID_ARG;
    *version = g->version;
    return QG_OK;
}

int qg_gguf_data_offset(const qg_gguf *g, uint64_t *offset)
{
    if (!g || !offset) return QG_ERR_INVALID_ARG;
    *offset = g->data_offset;
    return QG_OK;
}

int qg_gguf_metadata_count(const qg_gguf *g, size_t *n)
{
    if (!g || !n) return QG_ERR_INVALID_ARG;
    *n = g->meta.size();
    return QG_OK;
}

int qg_gguf_metadata_type(const qg_gguf *g, const char *key, uint32_t *type)
{
    if (!g || !key || !type) return QG_ERR_INVALID_ARG;
    const Value *v = find(g, key);
    if (!v) return QG_ERR_SHAPE;
    *type = v->type;
    return QG_OK;
}

int qg_gguf_get_u64(const qg_gguf *g, const char *key, uint64_t *value)
{
    if (!g || !key || !value) return QG_ERR_INVALID_ARG;
    return to_u64(find(g, key), value) ? QG_OK : QG_ERR_SHAPE;
}

int qg_gguf_get_f32(const qg_gguf *g, const char *key, float *value)
{
    if (!g || !key || !value) return QG_ERR_INVALID_ARG;
    return to_f32(find(g, key), value) ? QG_OK : QG_ERR_SHAPE;
}

int qg_gguf_get_string(const qg_gguf *g, const char *key, char *buf, size_t cap, size_t *len)
{
    if (!g || !key) return QG_ERR_INVALID_ARG;
    const Value *v = find(g, key);
    if (!v || v->type != QG_GGUF_STRING) return QG_ERR_SHAPE;
    if (len) *len = v->s.size();
    if (buf && cap) {
        const size_t k = v->s.size() < cap - 1 ? v->s.size() : cap - 1;
        std::memcpy(buf, v->s.data(), k);
        buf[k] = 0;
    }
    return QG_OK;
}

int qg_gguf_get_array_info(const qg_gguf *g, const char *key, uint32_t *elem_type, uint64_t *count)
{
    if (!g || !key) return QG_ERR_INVALID_ARG;
    const Value *v = find(g, key);
    if (!v || v->type != QG_GGUF_ARRAY) return QG_ERR_SHAPE;
    if (elem_type) *elem_type = v->elem_type;
    if (count) *count = v->count;
    return QG_OK;
}

int qg_gguf_tensor_count(const qg_gguf *g, size_t *n)
{
    if (!g || !n) return QG_ERR_INVALID_ARG;
    *n = g->tensors.size();
    return QG_OK;
}

int qg_gguf_find_tensor(const qg_gguf *g, const char *name, size_t *index)
{
    if (!g || !name || !index) return QG_ERR_INVALID_ARG;
    for (size_t i = 0; i < g->tensors.size(); i++)            // get_tensor: the first match
        if (g->tensors[i].name == name) { *index = i; return QG_OK; }
    return QG_ERR_SHAPE;
}

int qg_gguf_tensor_info(const qg_gguf *g, size_t index, const char **name, uint32_t *ggml_type,
                        uint32_t *n_dims, uint64_t dims[4], uint64_t *offset, size_t *nbytes)
{
    if (!g || index >= g->tensors.size()) return QG_ERR_INVALID_ARG;
    const Tensor &t = g->tensors[index];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = t.type;
    if (n_dims) *n_dims = (uint32_t)t.dims.size();
    if (dims)
        for (int d = 0; d < 4; d++) dims[d] = d < (int)t.dims.size() ? t.dims[d] : 1;
    if (offset) *offset = t.offset;
    uint64_t nb = 0;
    const bool ok = load_bytes(t, &nb);
    if (nbytes) *nbytes = ok ? (size_t)nb : 0;
    return ok ? QG_OK : QG_ERR_SHAPE;
}

int qg_gguf_tensor_data(const qg_gguf *g, size_t index, const void **data, size_t *nbytes)
{
    if (!g || index >= g->tensors.size() || !data) return QG_ERR_INVALID_ARG;
    const Tensor &t = g->tensors[index];
    uint64_t nb = 0;
    if (!load_bytes(t, &nb)) return QG_ERR_SHAPE;             // dims overflow 64 bits
    if (nb == 0) return QG_ERR_UNSUPPORTED_TYPE;              // model.rs:176-179 skips it
    const uint64_t start = g->data_offset + t.offset;
    if (start < g->data_offset || start > g->size || nb > g->size - start) return QG_ERR_SHORT_DATA;
    *data = g->map + start;
    if (nbytes) *nbytes = (size_t)nb;
    return QG_OK;
}

int qg_gguf_model_config(const qg_gguf *g, uint32_t max_seq_len, qg_model_config *cfg)
{
    if (!g || !cfg) return QG_ERR_INVALID_ARG;
    const Value *a = find(g, "general.architecture");
    const std::string arch = a && a->type == QG_GGUF_STRING ? a->s : std::string("llama");
    const std::string p = arch + ".";
    auto u = [&](const char *k) -> uint64_t {
        uint64_t v = 0;
        return to_u64(find(g, (p + k).c_str()), &v) ? v : 0;
    };
    auto f = [&](const char *k) -> float {
        float v = 0.f;
        return to_f32(find(g, (p + k).c_str()), &v) ? v : 0.f;
    };
    uint64_t embed = u("embedding_length"), layers = u("block_count"), heads = u("attention.head_count");
    uint64_t kv = u("attention.head_count_kv"), hidden = u("feed_forward_length"), vocab = u("vocab_size");
    uint64_t ctx_len = u("context_length");
    float rope = f("rope.freq_base");
    // attention.layer_norm_rms_epsilon, else attention.layer_norm_epsilon, else 1e-5 (model.rs:82-86)
    float eps = 1e-5f;
    const Value *e = find(g, (p + "attention.layer_norm_rms_epsilon").c_str());
    if (!e) e = find(g, (p + "attention.layer_norm_epsilon").c_str());
    if (e && !to_f32(e, &eps)) eps = 1e-5f;
    // architecture defaults (model.rs:88-95)
    uint64_t d_embed = 4096, d_layers = 32, d_heads = 32, d_hidden = 11008, d_vocab = 32000;
    float d_rope = 10000.0f;
    if (arch == "qwen2") { d_embed = 3584; d_layers = 28; d_heads = 28; d_hidden = 18944; d_vocab = 151936; d_rope = 1000000.0f; }
    else if (arch == "mistral") { d_hidden = 14336; }
    if (!embed) embed = d_embed;
    if (!layers) layers = d_layers;
    if (!heads) heads = d_heads;
    if (!kv) kv = heads;
    if (!hidden) hidden = d_hidden;
    if (!vocab) vocab = d_vocab;
    if (!ctx_len) ctx_len = 32768;
    if (rope == 0.0f) rope = d_rope;
    if (max_seq_len) ctx_len = max_seq_len;
    const uint64_t lim = 0xFFFFFFFFull;
    if (embed > lim || layers > lim || heads > lim || kv > lim || hidden > lim || vocab > lim || ctx_len > lim)
        return QG_ERR_SHAPE;
    cfg->embed_dim = (uint32_t)embed;
    cfg->n_layers = (uint32_t)layers;
    cfg->n_heads = (uint32_t)heads;
    cfg->n_kv_heads = (uint32_t)kv;
    cfg->hidden_dim = (uint32_t)hidden;
    cfg->vocab_size = (uint32_t)vocab;
    cfg->max_seq_len = (uint32_t)ctx_len;
    cfg->rope_base = rope;
    cfg->norm_eps = eps;
    return QG_OK;
}

}  // extern "C"

namespace {

// the last tensor of that name, as Model::load's HashMap keeps it (model.rs:183-184)
const Tensor *last_tensor(const qg_gguf *g, const std::string &name, size_t *index)
{
    for (size_t i = g->tensors.size(); i-- > 0;)
        if (g->tensors[i].name == name) { *index = i; return &g->tensors[i]; }
    return nullptr;
}

struct Loader {
    qg_ctx *ctx;
    qg_gguf *g;
    qg_model *m = nullptr;
    std::string why;

    int missing(const std::string &name)
    {
        why = "missing " + name;
        return QG_ERR_SHAPE;
    }

    // load_mat! (model.rs:197-203): the raw bytes as a rows x cols matrix
    // (rows = 0: output.weight's own (ne1, ne0), model.rs:221-223)
    int mat(const std::string &name, uint32_t slot, uint32_t layer, size_t rows, size_t cols)
    {
        size_t i;
        const Tensor *t = last_tensor(g, name, &i);
        const void *data;
        size_t nb;
        if (!t) return missing(name);
        int rc = qg_gguf_tensor_data(g, i, &data, &nb);
        if (rc == QG_ERR_UNSUPPORTED_TYPE) return missing(name + " (type skipped by the loader)");
        if (rc) { why = "cannot read " + name; return rc; }
        if (rows == 0) {
            cols = t->dims.empty() ? 0 : (size_t)t->dims[0];
            rows = t->dims.size() > 1 ? (size_t)t->dims[1] : 1;
        }
        rc = qg_model_set_matrix(m, slot, layer, data, nb, t->type, rows, cols);
        if (rc) why = name + ": " + qg_last_error(ctx);
        return rc;
    }

    // an f32 vector: F32 tensors load their ne0 values, other types zeros
    // (model.rs:207-218, 232-279); a missing optional bias stays zero
    int vec(const std::string &name, uint32_t slot, uint32_t layer, bool required)
    {
        size_t i;
        const Tensor *t = last_tensor(g, name, &i);
        if (!t) return required ? missing(name) : QG_OK;
        const void *data;
        size_t nb;
        int rc = qg_gguf_tensor_data(g, i, &data, &nb);
        if (rc == QG_ERR_UNSUPPORTED_TYPE) return required ? missing(name + " (type skipped by the loader)") : QG_OK;
        if (rc) { why = "cannot read " + name; return rc; }
        const uint64_t n = t->dims.empty() ? 0 : t->dims[0];
        // every vector slot holds embed_dim, q_dim or kv_dim floats (u32
        // sizes): a longer ne0 cannot match the config, so it is refused
        // before anything is allocated for it
        if (n > 0xFFFFFFFFull) { why = name + ": length does not match the config"; return QG_ERR_SHAPE; }
        std::vector<float> v((size_t)n, 0.0f);
        if (t->type == 0 && n <= nb / 4) std::memcpy(v.data(), data, (size_t)n * 4);
        rc = qg_model_set_vector(m, slot, layer, v.data(), v.size());
        if (rc) why = name + ": " + qg_last_error(ctx);
        return rc;
    }
};

}  // namespace

namespace {

// Owners that release the mapping and a half-loaded model on every way out
// of load_gguf, exceptions included.
struct GgufGuard {
    qg_gguf *g = nullptr;
    ~GgufGuard() { if (g) qg_gguf_close(g); }
};
struct ModelGuard {
    qg_model *m = nullptr;
    ~ModelGuard() { if (m) qg_model_destroy(m); }
};

int load_gguf(qg_ctx *ctx, const char *path, uint32_t max_seq_len, qg_model **out)
{
    GgufGuard gg;
    int rc = qg_gguf_open(path, &gg.g);
    if (rc) return qg_fail(ctx, rc, (std::string("GGUF: ") + qg_gguf_open_error()).c_str());
    qg_gguf *g = gg.g;
    qg_model_config cfg;
    if ((rc = qg_gguf_model_config(g, max_seq_len, &cfg))) return qg_fail(ctx, rc, "GGUF: model config out of range");
    Loader L{ctx, g};
    ModelGuard mg;
    if ((rc = qg_model_create(ctx, &cfg, &mg.m))) return rc;
    L.m = mg.m;
    const std::string b = "blk.";
    auto blk = [&](uint32_t l, const char *s) { return b + std::to_string(l) + "." + s; };
    const size_t E = cfg.embed_dim, H = cfg.hidden_dim, V = cfg.vocab_size;
    const size_t q_dim = (size_t)cfg.n_heads * (E / cfg.n_heads), kv_dim = (size_t)cfg.n_kv_heads * (E / cfg.n_heads);
    rc = L.mat("token_embd.weight", QG_M_TOKEN_EMBD, 0, V, E);
    if (!rc) rc = L.vec("output_norm.weight", QG_V_FINAL_NORM, 0, true);
    if (!rc) {
        size_t i;
        if (last_tensor(g, "output.weight", &i))
            rc = L.mat("output.weight", QG_M_LM_HEAD, 0, 0, 0);
        else
            rc = qg_model_tie_lm_head(L.m);                         // model.rs:224-226
    }
    for (uint32_t l = 0; l < cfg.n_layers && !rc; l++) {
        if ((rc = L.vec(blk(l, "attn_norm.weight"), QG_V_ATTN_NORM, l, true)) ||
            (rc = L.mat(blk(l, "attn_q.weight"), QG_M_WQ, l, q_dim, E)) ||
            (rc = L.mat(blk(l, "attn_k.weight"), QG_M_WK, l, kv_dim, E)) ||
            (rc = L.mat(blk(l, "attn_v.weight"), QG_M_WV, l, kv_dim, E)) ||
            (rc = L.mat(blk(l, "attn_output.weight"), QG_M_WO, l, E, q_dim)) ||
            (rc = L.vec(blk(l, "attn_q.bias"), QG_V_BQ, l, false)) ||
            (rc = L.vec(blk(l, "attn_k.bias"), QG_V_BK, l, false)) ||
            (rc = L.vec(blk(l, "attn_v.bias"), QG_V_BV, l, false)) ||
            (rc = L.vec(blk(l, "ffn_norm.weight"), QG_V_FFN_NORM, l, true)) ||
            (rc = L.mat(blk(l, "ffn_gate.weight"), QG_M_GATE, l, H, E)) ||
            (rc = L.mat(blk(l, "ffn_up.weight"), QG_M_UP, l, H, E)) ||
            (rc = L.mat(blk(l, "ffn_down.weight"), QG_M_DOWN, l, E, H)))
            break;
    }
    if (rc) {
        const std::string why = L.why.empty() ? std::string(qg_last_error(ctx)) : L.why;
        return qg_fail(ctx, rc, ("GGUF: " + why).c_str());
    }
    *out = mg.m;
    mg.m = nullptr;
    return QG_OK;
}

}  // namespace

// Model::load (model.rs:136-329) from a GGUF file; no exception leaves the C ABI.
extern "C" int qg_model_load_gguf(qg_ctx *ctx, const char *path, uint32_t max_seq_len, qg_model **out)
{
    if (!ctx || !path || !out) return QG_ERR_INVALID_ARG;
    *out = nullptr;
    try {
        return load_gguf(ctx, path, max_seq_len, out);
    } catch (const std::bad_alloc &) {
        return qg_fail(ctx, QG_ERR_OUT_OF_MEMORY, "GGUF: host allocation failed");
    } catch (...) {
        return qg_fail(ctx, QG_ERR_INVALID_ARG, "GGUF: unexpected error while loading");
    }
}
