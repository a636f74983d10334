// gguf.hip — GGUF v3 reader and model loader (host code).
//
// lrs_gguf_open maps a file and parses what GgufFile::parse reads
// (crates/gguf/src/parse.rs:64-126): magic "GGUF", version 3, tensor and KV
// counts, the KV metadata (value types 0-12, arrays of non-array values), the
// tensor infos (name, dims, ggml type, offset), and the data section at the
// next multiple of general.alignment (default 32).  Tensor bytes are checked
// like GgufFile::tensor_data (file.rs:47-75): element count a multiple of the
// block size, [data + offset, + n_blocks * type_size) inside the file.
//
// lrs_model_load_gguf follows LlamaConfig::from_gguf (config.rs:81-187) for
// the architecture keys and GpuRawWeights / GpuAuxWeights::from_gguf
// (gpu.rs:128-600) for the tensor names, then builds a dense or hybrid model
// that owns the weights it uploaded.
#include "lrs_internal.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace {

struct GValue {
    uint32_t type = 0;  // GGUF value type; 9 = array
    uint64_t u = 0;     // unsigned / bool / signed (two's complement)
    double f = 0;       // float types
    std::string s;      // string
    uint32_t arr_type = 0;
    uint64_t arr_len = 0;
};

struct GTensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
};

struct Cursor {
    const uint8_t *p, *end;
    bool ok = true;
    template <typename T>
    T get() {
        T v{};
        if ((size_t)(end - p) < sizeof(T)) {
            ok = false;
            return v;
        }
        memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || (uint64_t)(end - p) < n) {
            ok = false;
            return {};
        }
        std::string s(reinterpret_cast<const char *>(p), (size_t)n);
        p += n;
        return s;
    }
    void skip(uint64_t n) {
        if ((uint64_t)(end - p) < n) ok = false;
        else p += n;
    }
};

// scalar sizes of value types 0-12 (8 = string, 9 = array: variable)
int64_t scalar_size(uint32_t t) {
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return -1;
    }
}

bool read_scalar(Cursor &c, uint32_t t, GValue &v) {
    v.type = t;
    switch (t) {
    case 0: v.u = c.get<uint8_t>(); break;
    case 1: v.u = (uint64_t)(int64_t)c.get<int8_t>(); break;
    case 2: v.u = c.get<uint16_t>(); break;
    case 3: v.u = (uint64_t)(int64_t)c.get<int16_t>(); break;
    case 4: v.u = c.get<uint32_t>(); break;
    case 5: v.u = (uint64_t)(int64_t)c.get<int32_t>(); break;
    case 6: v.f = c.get<float>(); break;
    case 7: v.u = c.get<uint8_t>(); break;
    case 8: v.s = c.str(); break;
    case 10: v.u = c.get<uint64_t>(); break;
    case 11: v.u = (uint64_t)c.get<int64_t>(); break;
    case 12: v.f = c.get<double>(); break;
    default: return false;
    }
    return c.ok;
}

}  // namespace

struct lrs_gguf {
    void *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    std::map<std::string, GValue> kv;
    std::vector<GTensor> tensors;
    size_t data_offset = 0;
};

using namespace lrs;

namespace {

int parse_gguf(lrs_gguf *g) {
    Cursor c{reinterpret_cast<const uint8_t *>(g->map), reinterpret_cast<const uint8_t *>(g->map) + g->size};
    const uint32_t magic = c.get<uint32_t>();
    if (!c.ok || memcmp(&magic, "GGUF", 4) != 0) return fail(LRS_E_ARG, "gguf: bad magic");
    g->version = c.get<uint32_t>();
    if (g->version != 3)
        return fail(LRS_E_UNSUPPORTED, "gguf: unsupported version " + std::to_string(g->version));
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (!c.ok) return fail(LRS_E_ARG, "gguf: truncated header");
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        if (!c.ok) return fail(LRS_E_ARG, "gguf: truncated metadata");
        GValue v;
        if (t == 9) {
            v.type = 9;
            v.arr_type = c.get<uint32_t>();
            v.arr_len = c.get<uint64_t>();
            if (v.arr_type == 9) return fail(LRS_E_ARG, "gguf: nested array in " + key);
            if (v.arr_type == 8) {
                for (uint64_t k = 0; k < v.arr_len && c.ok; k++) (void)c.str();
            } else {
                const int64_t sz = scalar_size(v.arr_type);
                if (sz < 0) return fail(LRS_E_ARG, "gguf: unknown array type in " + key);
                if (v.arr_len > (uint64_t)(c.end - c.p) / (uint64_t)sz) c.ok = false;
                else c.skip(v.arr_len * (uint64_t)sz);
            }
        } else if (!read_scalar(c, t, v)) {
            return fail(LRS_E_ARG, "gguf: bad value for " + key);
        }
        if (!c.ok) return fail(LRS_E_ARG, "gguf: truncated metadata");
        g->kv[key] = v;
    }
    for (uint64_t i = 0; i < n_tensors; i++) {
        GTensor t;
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (!c.ok || nd > 8) return fail(LRS_E_ARG, "gguf: bad tensor info");
        for (uint32_t d = 0; d < nd; d++) t.dims.push_back(c.get<uint64_t>());
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (!c.ok) return fail(LRS_E_ARG, "gguf: truncated tensor infos");
        g->tensors.push_back(t);
    }
    uint64_t align = 32;
    auto it = g->kv.find("general.alignment");
    if (it != g->kv.end()) {
        if (it->second.type != 4) return fail(LRS_E_ARG, "gguf: general.alignment is not u32");
        align = it->second.u;
    }
    size_t pos = (size_t)(c.p - reinterpret_cast<const uint8_t *>(g->map));
    if (align && pos % align) pos += align - pos % align;
    g->data_offset = pos;
    return LRS_OK;
}

const GTensor *find_tensor(const lrs_gguf *g, const char *name) {
    for (const GTensor &t : g->tensors)
        if (t.name == name) return &t;
    return nullptr;
}

// GgufFile::tensor_data (file.rs:47-75)
int tensor_bytes(const lrs_gguf *g, const GTensor &t, const uint8_t **data, size_t *len) {
    uint64_t n = 1;
    for (uint64_t d : t.dims) {
        if (d && n > UINT64_MAX / d) return fail(LRS_E_ARG, "gguf: element count overflow in " + t.name);
        n *= d;
    }
    const int64_t bs = block_elems(t.type), ts = block_bytes(t.type);
    if (bs <= 0 || n % (uint64_t)bs) return fail(LRS_E_ARG, "gguf: tensor " + t.name + " out of bounds");
    const uint64_t nb = (n / (uint64_t)bs) * (uint64_t)ts;
    const uint64_t start = (uint64_t)g->data_offset + t.offset;
    if (start < t.offset || start > g->size || nb > g->size - start)
        return fail(LRS_E_ARG, "gguf: tensor " + t.name + " out of bounds");
    *data = reinterpret_cast<const uint8_t *>(g->map) + start;
    *len = (size_t)nb;
    return LRS_OK;
}

bool get_u32(const lrs_gguf *g, const std::string &key, uint32_t *v) {
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return false;
    const GValue &x = it->second;
    if (x.type == 4 || x.type == 0 || x.type == 2 || x.type == 10 || x.type == 5 || x.type == 11) {
        *v = (uint32_t)x.u;
        return true;
    }
    return false;
}

float h2f_host(uint16_t h) {
    const uint32_t s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
    uint32_t b;
    if (e == 0) {
        if (m == 0) {
            b = s << 31;
        } else {  // subnormal: normalise
            int ex = -1;
            uint32_t mm = m;
            do {
                ex++;
                mm <<= 1;
            } while (!(mm & 1024));
            b = (s << 31) | ((uint32_t)(127 - 15 - ex) << 23) | ((mm & 1023) << 13);
        }
    } else if (e == 31) {
        b = (s << 31) | 0x7F800000u | (m << 13);
    } else {
        b = (s << 31) | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &b, 4);
    return f;
}

}  // namespace

extern "C" {

int lrs_gguf_open(const char *path, lrs_gguf **out) {
    if (!path || !out) return fail(LRS_E_ARG, "null argument");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(LRS_E_ARG, std::string("gguf: cannot open ") + path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return fail(LRS_E_ARG, std::string("gguf: cannot stat ") + path);
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return fail(LRS_E_ARG, std::string("gguf: cannot map ") + path);
    lrs_gguf *g = new lrs_gguf();
    g->map = m;
    g->size = (size_t)st.st_size;
    const int rc = parse_gguf(g);
    if (rc) {
        lrs_gguf_close(g);
        return rc;
    }
    *out = g;
    return LRS_OK;
}

void lrs_gguf_close(lrs_gguf *g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->size);
    delete g;
}

uint32_t lrs_gguf_version(const lrs_gguf *g) { return g ? g->version : 0; }
uint64_t lrs_gguf_n_tensors(const lrs_gguf *g) { return g ? g->tensors.size() : 0; }

int lrs_gguf_get_u32(const lrs_gguf *g, const char *key, uint32_t *v) {
    if (!g || !key || !v) return fail(LRS_E_ARG, "null argument");
    if (!get_u32(g, key, v)) return fail(LRS_E_ARG, std::string("gguf: missing or non-integer key ") + key);
    return LRS_OK;
}

int lrs_gguf_get_f32(const lrs_gguf *g, const char *key, float *v) {
    if (!g || !key || !v) return fail(LRS_E_ARG, "null argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end() || (it->second.type != 6 && it->second.type != 12))
        return fail(LRS_E_ARG, std::string("gguf: missing or non-float key ") + key);
    *v = (float)it->second.f;
    return LRS_OK;
}

int lrs_gguf_get_str(const lrs_gguf *g, const char *key, const char **s) {
    if (!g || !key || !s) return fail(LRS_E_ARG, "null argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 8)
        return fail(LRS_E_ARG, std::string("gguf: missing or non-string key ") + key);
    *s = it->second.s.c_str();
    return LRS_OK;
}

int lrs_gguf_array_len(const lrs_gguf *g, const char *key, uint64_t *n) {
    if (!g || !key || !n) return fail(LRS_E_ARG, "null argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 9)
        return fail(LRS_E_ARG, std::string("gguf: missing or non-array key ") + key);
    *n = it->second.arr_len;
    return LRS_OK;
}

int lrs_gguf_tensor(const lrs_gguf *g, const char *name, uint32_t *ggml_type, uint64_t *dims,
                    uint32_t *n_dims, const void **data, size_t *len) {
    if (!g || !name) return fail(LRS_E_ARG, "null argument");
    const GTensor *t = find_tensor(g, name);
    if (!t) return fail(LRS_E_ARG, std::string("gguf: tensor ") + name + " missing");
    const uint8_t *d = nullptr;
    size_t n = 0;
    int rc = tensor_bytes(g, *t, &d, &n);
    if (rc) return rc;
    if (ggml_type) *ggml_type = t->type;
    if (n_dims) *n_dims = (uint32_t)t->dims.size();
    if (dims)
        for (size_t i = 0; i < t->dims.size() && i < 4; i++) dims[i] = t->dims[i];
    if (data) *data = d;
    if (len) *len = n;
    return LRS_OK;
}

}  // extern "C"

// ---- model loader ----------------------------------------------------------
namespace {

struct Loader {
    lrs_ctx *ctx;
    const lrs_gguf *g;
    std::vector<lrs_weight *> owned;
    std::vector<std::vector<float>> vecs;

    ~Loader() {
        for (lrs_weight *w : owned) lrs_weight_free(w);
    }

    // a matrix [n_out][n_in] of any GGUF type, uploaded (gpu.rs:132-164)
    int weight(const std::string &name, uint32_t n_in, uint32_t n_out, const lrs_weight **out) {
        const GTensor *t = find_tensor(g, name.c_str());
        if (!t) return fail(LRS_E_ARG, "gguf: tensor " + name + " missing");
        const uint8_t *d;
        size_t n;
        int rc = tensor_bytes(g, *t, &d, &n);
        if (rc) return rc;
        lrs_weight *w = nullptr;
        if ((rc = lrs_weight_upload(ctx, t->type, d, n, n_in, n_out, &w)))
            return fail(rc, name + ": " + lrs_last_error());
        owned.push_back(w);
        *out = w;
        return LRS_OK;
    }

    // an f32 vector of `count` elements (F32 or F16 in the file), or null
    // when optional and absent (gpu.rs:474-492)
    int vec(const std::string &name, size_t count, const float **out, bool optional = false) {
        const GTensor *t = find_tensor(g, name.c_str());
        if (!t) {
            if (optional) {
                *out = nullptr;
                return LRS_OK;
            }
            return fail(LRS_E_ARG, "gguf: tensor " + name + " missing");
        }
        const uint8_t *d;
        size_t n;
        int rc = tensor_bytes(g, *t, &d, &n);
        if (rc) return rc;
        std::vector<float> v;
        if (t->type == T_F32) {
            v.resize(n / 4);
            memcpy(v.data(), d, n);
        } else if (t->type == T_F16) {
            v.resize(n / 2);
            for (size_t i = 0; i < v.size(); i++) {
                uint16_t h;
                memcpy(&h, d + 2 * i, 2);
                v[i] = h2f_host(h);
            }
        } else {
            return fail(LRS_E_UNSUPPORTED, "gguf: " + name + " must be F32 or F16");
        }
        if (v.size() != count)
            return fail(LRS_E_ARG, "gguf: tensor " + name + " has " + std::to_string(v.size()) +
                                       " floats, expected " + std::to_string(count));
        vecs.push_back(std::move(v));
        *out = vecs.back().data();
        return LRS_OK;
    }
};

}  // namespace

void lrs_model_adopt_weights(lrs_model *m, std::vector<lrs_weight *> &ws);

extern "C" int lrs_model_load_gguf(lrs_ctx *ctx, const lrs_gguf *g, uint32_t ctx_len,
                                   lrs_model **out) {
    if (!ctx || !g || !out) return fail(LRS_E_ARG, "null argument");
    // LlamaConfig::from_gguf (config.rs:81-187)
    std::string arch = "llama";
    auto ai = g->kv.find("general.architecture");
    if (ai != g->kv.end() && ai->second.type == 8) arch = ai->second.s;
    auto key = [&](const char *s) { return arch + "." + s; };
    uint32_t n_embd, n_head, n_head_kv, n_ff, n_layer_all, ctx_train;
    if (!get_u32(g, key("embedding_length"), &n_embd) ||
        !get_u32(g, key("attention.head_count"), &n_head) ||
        !get_u32(g, key("attention.head_count_kv"), &n_head_kv) ||
        !get_u32(g, key("feed_forward_length"), &n_ff) || !get_u32(g, key("block_count"), &n_layer_all) ||
        !get_u32(g, key("context_length"), &ctx_train))
        return fail(LRS_E_ARG, "gguf: missing " + arch + ".* model keys");
    if (n_head == 0) return fail(LRS_E_ARG, "gguf: n_head is zero");
    uint32_t head_dim;
    if (!get_u32(g, key("attention.key_length"), &head_dim)) {
        if (n_embd % n_head) return fail(LRS_E_ARG, "gguf: n_head does not divide n_embd and attention.key_length is absent");
        head_dim = n_embd / n_head;
    }
    uint32_t rope_dim = head_dim;
    (void)get_u32(g, key("rope.dimension_count"), &rope_dim);
    float freq_base = 10000.0f;
    {
        auto it = g->kv.find(key("rope.freq_base"));
        if (it != g->kv.end() && it->second.type == 6) freq_base = (float)it->second.f;
    }
    float rms_eps = 0.f;
    {
        auto it = g->kv.find(key("attention.layer_norm_rms_epsilon"));
        if (it == g->kv.end() || it->second.type != 6)
            return fail(LRS_E_ARG, "gguf: missing " + key("attention.layer_norm_rms_epsilon"));
        rms_eps = (float)it->second.f;
    }
    uint64_t vocab = 0;
    {
        auto it = g->kv.find("tokenizer.ggml.tokens");
        if (it == g->kv.end() || it->second.type != 9) return fail(LRS_E_ARG, "gguf: tokenizer.ggml.tokens is not an array");
        vocab = it->second.arr_len;
    }
    uint32_t nextn = 0;
    (void)get_u32(g, key("nextn_predict_layers"), &nextn);
    if (nextn >= n_layer_all) return fail(LRS_E_ARG, "gguf: nextn_predict_layers >= block_count");
    lrs_config c = {};
    c.n_layer = n_layer_all - nextn;
    c.n_embd = n_embd;
    c.n_head = n_head;
    c.n_head_kv = n_head_kv;
    c.head_dim = head_dim;
    c.n_ff = n_ff;
    c.vocab = (uint32_t)vocab;
    c.rope_dim = rope_dim;
    c.ctx = ctx_len ? ctx_len : ctx_train;
    c.rms_eps = rms_eps;
    c.freq_base = freq_base;

    Loader L{ctx, g, {}, {}};
    L.vecs.reserve(16 * (size_t)c.n_layer + 4);  // pointers into vecs stay valid
    const uint32_t qd = n_head * head_dim, kvd = n_head_kv * head_dim;
    const lrs_weight *embd = nullptr, *output = nullptr;
    const float *onorm = nullptr;
    int rc;
    if ((rc = L.weight("token_embd.weight", n_embd, c.vocab, &embd)) ||
        (rc = L.weight("output.weight", n_embd, c.vocab, &output)) ||
        (rc = L.vec("output_norm.weight", n_embd, &onorm)))
        return rc;
    auto blk = [](uint32_t l, const char *s) { return "blk." + std::to_string(l) + "." + s; };
    lrs_model *m = nullptr;
    uint32_t conv_kernel = 0;
    if (get_u32(g, key("ssm.conv_kernel"), &conv_kernel)) {
        // qwen35: gated attention every full_attention_interval-th layer,
        // gated delta net elsewhere (config.rs:126-141, gpu.rs:172-200, 495-538)
        lrs_hybrid_config hc = {};
        hc.base = c;
        hc.full_attn_interval = 4;
        (void)get_u32(g, key("full_attention_interval"), &hc.full_attn_interval);
        if (hc.full_attn_interval == 0) return fail(LRS_E_ARG, "gguf: full_attention_interval is zero");
        uint32_t d_inner;
        if (!get_u32(g, key("ssm.inner_size"), &d_inner) || !get_u32(g, key("ssm.state_size"), &hc.dn_state) ||
            !get_u32(g, key("ssm.time_step_rank"), &hc.dn_v_heads) ||
            !get_u32(g, key("ssm.group_count"), &hc.dn_k_heads))
            return fail(LRS_E_ARG, "gguf: missing ssm.* keys");
        hc.dn_conv = conv_kernel;
        if (hc.dn_v_heads == 0 || d_inner / hc.dn_v_heads != hc.dn_state)
            return fail(LRS_E_UNSUPPORTED, "gguf: value head width (ssm.inner_size / time_step_rank) must equal ssm.state_size");
        const uint32_t D = hc.dn_state, VD = hc.dn_v_heads * D, CD = 2 * hc.dn_k_heads * D + VD;
        std::vector<lrs_hybrid_layer> layers(c.n_layer);
        for (uint32_t l = 0; l < c.n_layer; l++) {
            lrs_hybrid_layer &H = layers[l];
            if ((rc = L.weight(blk(l, "ffn_gate.weight"), n_embd, n_ff, &H.ffn_gate)) ||
                (rc = L.weight(blk(l, "ffn_up.weight"), n_embd, n_ff, &H.ffn_up)) ||
                (rc = L.weight(blk(l, "ffn_down.weight"), n_ff, n_embd, &H.ffn_down)) ||
                (rc = L.vec(blk(l, "attn_norm.weight"), n_embd, &H.attn_norm)) ||
                (rc = L.vec(blk(l, "post_attention_norm.weight"), n_embd, &H.post_norm)))
                return rc;
            if ((l + 1) % hc.full_attn_interval == 0) {
                if ((rc = L.weight(blk(l, "attn_q.weight"), n_embd, 2 * qd, &H.attn_q)) ||
                    (rc = L.weight(blk(l, "attn_k.weight"), n_embd, kvd, &H.attn_k)) ||
                    (rc = L.weight(blk(l, "attn_v.weight"), n_embd, kvd, &H.attn_v)) ||
                    (rc = L.weight(blk(l, "attn_output.weight"), qd, n_embd, &H.attn_output)) ||
                    (rc = L.vec(blk(l, "attn_q_norm.weight"), head_dim, &H.q_norm)) ||
                    (rc = L.vec(blk(l, "attn_k_norm.weight"), head_dim, &H.k_norm)))
                    return rc;
            } else {
                if ((rc = L.weight(blk(l, "attn_qkv.weight"), n_embd, CD, &H.ssm_qkv)) ||
                    (rc = L.weight(blk(l, "attn_gate.weight"), n_embd, VD, &H.ssm_gate)) ||
                    (rc = L.weight(blk(l, "ssm_out.weight"), VD, n_embd, &H.ssm_out)) ||
                    (rc = L.vec(blk(l, "ssm_alpha.weight"), (size_t)n_embd * hc.dn_v_heads, &H.ssm_alpha)) ||
                    (rc = L.vec(blk(l, "ssm_beta.weight"), (size_t)n_embd * hc.dn_v_heads, &H.ssm_beta)) ||
                    (rc = L.vec(blk(l, "ssm_a"), hc.dn_v_heads, &H.ssm_a)) ||
                    (rc = L.vec(blk(l, "ssm_dt.bias"), hc.dn_v_heads, &H.ssm_dt)) ||
                    (rc = L.vec(blk(l, "ssm_conv1d.weight"), (size_t)CD * hc.dn_conv, &H.ssm_conv)) ||
                    (rc = L.vec(blk(l, "ssm_norm.weight"), D, &H.ssm_norm)))
                    return rc;
            }
        }
        if ((rc = lrs_hybrid_create(ctx, &hc, layers.data(), embd, onorm, output, &m))) return rc;
    } else {
        // dense Llama / Qwen2 (gpu.rs:200-206, model.rs:99-266), q/k/v biases when present
        std::vector<lrs_layer_weights> layers(c.n_layer);
        for (uint32_t l = 0; l < c.n_layer; l++) {
            lrs_layer_weights &W = layers[l];
            if ((rc = L.weight(blk(l, "attn_q.weight"), n_embd, qd, &W.attn_q)) ||
                (rc = L.weight(blk(l, "attn_k.weight"), n_embd, kvd, &W.attn_k)) ||
                (rc = L.weight(blk(l, "attn_v.weight"), n_embd, kvd, &W.attn_v)) ||
                (rc = L.weight(blk(l, "attn_output.weight"), qd, n_embd, &W.attn_output)) ||
                (rc = L.weight(blk(l, "ffn_gate.weight"), n_embd, n_ff, &W.ffn_gate)) ||
                (rc = L.weight(blk(l, "ffn_up.weight"), n_embd, n_ff, &W.ffn_up)) ||
                (rc = L.weight(blk(l, "ffn_down.weight"), n_ff, n_embd, &W.ffn_down)) ||
                (rc = L.vec(blk(l, "attn_norm.weight"), n_embd, &W.attn_norm)) ||
                (rc = L.vec(blk(l, "ffn_norm.weight"), n_embd, &W.ffn_norm)) ||
                (rc = L.vec(blk(l, "attn_q.bias"), qd, &W.bq, true)) ||
                (rc = L.vec(blk(l, "attn_k.bias"), kvd, &W.bk, true)) ||
                (rc = L.vec(blk(l, "attn_v.bias"), kvd, &W.bv, true)))
                return rc;
        }
        if ((rc = lrs_model_create(ctx, &c, layers.data(), embd, onorm, output, &m))) return rc;
    }
    // the model frees the weights it was built from
    lrs_model_adopt_weights(m, L.owned);
    *out = m;
    return LRS_OK;
}
