// GGUF reader and the MoE-layer loader of the C ABI (include/biv_hip.h).
//
// The container format follows biv's reader (engine/src/gguf.rs): header
// (magic "GGUF", version >= 2, tensor and key/value counts), key/values of
// the value types 0..12, the tensor table (name, dims in ggml order, type,
// offset from the aligned data start), data aligned to general.alignment
// (32 by default).  Split files are read together: the first file that holds
// a key keeps it, and each tensor's bytes stay in its own file.  Files are
// memory-mapped; the loader uploads straight from the mapping, as biv's
// Loader slices it (engine/src/model.rs:298-421).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdint>
#include <new>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "biv_hip.h"

int biv_hip_fail_ext(biv_hip_ctx *ctx, int code, const char *msg); // api.cpp

namespace {

thread_local std::string g_open_error;

struct Value {
    uint32_t ty = 0; // GGUF value type
    uint64_t u = 0;  // integers and bools (sign-extended for the signed types)
    double f = 0.0;  // F32 / F64
    std::string s;
    std::vector<Value> arr;
};

struct Shard {
    const uint8_t *p = nullptr;
    size_t n = 0;
};

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dims;
    int ty = 0;
    int shard = 0;
    uint64_t offset = 0; // absolute, in the shard
    size_t n_bytes = 0;
};

// (elements per block, bytes per block) of the types biv reads
// (GgmlType::block, engine/src/quant.rs:50-66); false for the others
bool type_block(uint32_t ty, size_t &be, size_t &bb)
{
    switch (ty) {
    case 0: be = 1, bb = 4; return true;     // F32
    case 1: be = 1, bb = 2; return true;     // F16
    case 2: be = 32, bb = 18; return true;   // Q4_0
    case 3: be = 32, bb = 20; return true;   // Q4_1
    case 6: be = 32, bb = 22; return true;   // Q5_0
    case 7: be = 32, bb = 24; return true;   // Q5_1
    case 8: be = 32, bb = 34; return true;   // Q8_0
    case 10: be = 256, bb = 84; return true; // Q2_K
    case 11: be = 256, bb = 110; return true; // Q3_K
    case 12: be = 256, bb = 144; return true; // Q4_K
    case 13: be = 256, bb = 176; return true; // Q5_K
    case 14: be = 256, bb = 210; return true; // Q6_K
    case 30: be = 1, bb = 2; return true;    // BF16
    default: return false;
    }
}

struct ParseError {
    int code;
    std::string msg;
};

struct Cursor {
    const uint8_t *buf;
    size_t n, pos = 0;
    const uint8_t *take(size_t k)
    {
        if (k > n - pos) throw ParseError{BIV_HIP_E_FORMAT, "gguf: unexpected end of data"};
        const uint8_t *p = buf + pos;
        pos += k;
        return p;
    }
    template <class T> T get()
    {
        T v;
        memcpy(&v, take(sizeof(T)), sizeof(T));
        return v;
    }
    std::string str()
    {
        const uint64_t len = get<uint64_t>();
        if (len > n - pos) throw ParseError{BIV_HIP_E_FORMAT, "gguf: unexpected end of data"};
        const uint8_t *p = take((size_t)len);
        return std::string(reinterpret_cast<const char *>(p), (size_t)len);
    }
    Value value(uint32_t ty)
    {
        Value v;
        v.ty = ty;
        switch (ty) {
        case 0: v.u = get<uint8_t>(); break;
        case 1: v.u = (uint64_t)(int64_t)get<int8_t>(); break;
        case 2: v.u = get<uint16_t>(); break;
        case 3: v.u = (uint64_t)(int64_t)get<int16_t>(); break;
        case 4: v.u = get<uint32_t>(); break;
        case 5: v.u = (uint64_t)(int64_t)get<int32_t>(); break;
        case 6: v.f = get<float>(); break;
        case 7: v.u = get<uint8_t>() != 0; break;
        case 8: v.s = str(); break;
        case 9: {
            const uint32_t et = get<uint32_t>();
            const uint64_t cnt = get<uint64_t>();
            if (cnt > n - pos) throw ParseError{BIV_HIP_E_FORMAT, "gguf: unexpected end of data"};
            v.arr.reserve((size_t)cnt);
            for (uint64_t i = 0; i < cnt; i++) v.arr.push_back(value(et));
            break;
        }
        case 10: v.u = get<uint64_t>(); break;
        case 11: v.u = (uint64_t)get<int64_t>(); break;
        case 12: v.f = get<double>(); break;
        default: throw ParseError{BIV_HIP_E_FORMAT, "gguf: unknown value type " + std::to_string(ty)};
        }
        return v;
    }
};

std::string fmt(const char *f, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

} // namespace

struct biv_gguf {
    std::vector<Shard> shards;
    std::vector<std::pair<std::string, Value>> kv; // file order, first holder of a key
    std::map<std::string, size_t> kv_index;
    std::vector<TensorInfo> tensors;               // file order
    std::map<std::string, size_t> tensor_index;
    std::string err;

    const Value *get(const std::string &key) const
    {
        auto it = kv_index.find(key);
        return it == kv_index.end() ? nullptr : &kv[it->second].second;
    }
    const TensorInfo *tensor(const std::string &name) const
    {
        auto it = tensor_index.find(name);
        return it == tensor_index.end() ? nullptr : &tensors[it->second];
    }
    int fail(int code, const std::string &msg)
    {
        err = msg;
        return code;
    }

    // Gguf::parse_shard (engine/src/gguf.rs:254-306)
    void parse(int shard)
    {
        Cursor c{shards[shard].p, shards[shard].n};
        if (c.get<uint32_t>() != 0x46554747u) throw ParseError{BIV_HIP_E_FORMAT, "gguf: bad magic, not a GGUF file"};
        const uint32_t version = c.get<uint32_t>();
        if (version < 2) throw ParseError{BIV_HIP_E_FORMAT, fmt("gguf: unsupported version %u", version)};
        const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
        for (uint64_t i = 0; i < n_kv; i++) {
            std::string key = c.str();
            const uint32_t ty = c.get<uint32_t>();
            Value v = c.value(ty);
            // split shards repeat split.* keys: the first holder keeps a key
            if (kv_index.count(key)) continue;
            kv_index[key] = kv.size();
            kv.emplace_back(std::move(key), std::move(v));
        }
        std::vector<TensorInfo> infos;
        for (uint64_t i = 0; i < n_tensors; i++) {
            TensorInfo t;
            t.name = c.str();
            const uint32_t n_dims = c.get<uint32_t>();
            if (n_dims > 4) throw ParseError{BIV_HIP_E_FORMAT, fmt("gguf: tensor %s has %u dims", t.name.c_str(), n_dims)};
            for (uint32_t d = 0; d < n_dims; d++) t.dims.push_back(c.get<uint64_t>());
            const uint32_t raw = c.get<uint32_t>();
            size_t be, bb;
            if (!type_block(raw, be, bb))
                throw ParseError{BIV_HIP_E_FORMAT, fmt("gguf: tensor %s has unknown type %u", t.name.c_str(), raw)};
            t.ty = (int)raw;
            t.shard = shard;
            t.offset = c.get<uint64_t>();
            uint64_t ne = 1;
            for (uint64_t d : t.dims)
                if (__builtin_mul_overflow(ne, d, &ne))
                    throw ParseError{BIV_HIP_E_FORMAT, fmt("gguf: tensor %s is too large", t.name.c_str())};
            if (ne % be)
                throw ParseError{BIV_HIP_E_FORMAT,
                                 fmt("gguf: tensor %s has %llu elements, not whole blocks of %zu", t.name.c_str(),
                                     (unsigned long long)ne, be)};
            uint64_t nb;
            if (__builtin_mul_overflow(ne / be, (uint64_t)bb, &nb) || nb > SIZE_MAX)
                throw ParseError{BIV_HIP_E_FORMAT, fmt("gguf: tensor %s is too large", t.name.c_str())};
            t.n_bytes = (size_t)nb;
            infos.push_back(std::move(t));
        }
        uint64_t alignment = 32;
        if (const Value *a = get("general.alignment"); a && a->ty <= 11 && a->ty != 6 && a->ty != 8 && a->ty != 9 && a->u)
            alignment = a->u;
        const uint64_t data_start = (c.pos + alignment - 1) / alignment * alignment;
        for (auto &t : infos) {
            t.offset += data_start;
            if (t.offset > shards[shard].n || t.n_bytes > shards[shard].n - t.offset)
                throw ParseError{BIV_HIP_E_FORMAT, "gguf: tensor " + t.name + " out of bounds"};
            tensor_index[t.name] = tensors.size();
            tensors.push_back(std::move(t));
        }
    }

    ~biv_gguf()
    {
        for (auto &s : shards)
            if (s.p) munmap(const_cast<uint8_t *>(s.p), s.n);
    }
};

extern "C" {

int biv_gguf_open(const char *const *paths, int n_paths, biv_gguf **out)
{
    if (!paths || n_paths < 1 || !out) {
        g_open_error = "biv_gguf_open: no files";
        return BIV_HIP_E_INVALID;
    }
    *out = nullptr;
    auto *g = new biv_gguf();
    for (int i = 0; i < n_paths; i++) {
        const int fd = open(paths[i], O_RDONLY);
        struct stat st;
        if (fd < 0 || fstat(fd, &st) != 0) {
            if (fd >= 0) close(fd);
            g_open_error = fmt("gguf: cannot open %s", paths[i]);
            delete g;
            return BIV_HIP_E_IO;
        }
        Shard s;
        s.n = (size_t)st.st_size;
        if (s.n) {
            void *p = mmap(nullptr, s.n, PROT_READ, MAP_PRIVATE, fd, 0);
            if (p == MAP_FAILED) {
                close(fd);
                g_open_error = fmt("gguf: cannot map %s", paths[i]);
                delete g;
                return BIV_HIP_E_IO;
            }
            s.p = static_cast<const uint8_t *>(p);
        }
        close(fd);
        g->shards.push_back(s);
        try {
            g->parse(i);
        } catch (const ParseError &e) {
            g_open_error = e.msg;
            delete g;
            return e.code;
        } catch (const std::bad_alloc &) {
            g_open_error = fmt("gguf: out of host memory reading %s", paths[i]);
            delete g;
            return BIV_HIP_E_NOMEM;
        }
    }
    *out = g;
    return 0;
}

void biv_gguf_close(biv_gguf *g) { delete g; }

const char *biv_gguf_last_error(const biv_gguf *g) { return g ? g->err.c_str() : g_open_error.c_str(); }

int biv_gguf_get_u64(biv_gguf *g, const char *key, uint64_t *out)
{
    if (!g || !key || !out) return BIV_HIP_E_INVALID;
    const Value *v = g->get(key);
    if (!v) return g->fail(BIV_HIP_E_MISSING, fmt("gguf: missing key %s", key));
    if (v->ty == 6 || v->ty == 8 || v->ty == 9 || v->ty == 12) return g->fail(BIV_HIP_E_FORMAT, fmt("gguf: %s is not an integer", key));
    *out = v->u; // Value::as_u64
    return 0;
}

int biv_gguf_get_f32(biv_gguf *g, const char *key, float *out)
{
    if (!g || !key || !out) return BIV_HIP_E_INVALID;
    const Value *v = g->get(key);
    if (!v) return g->fail(BIV_HIP_E_MISSING, fmt("gguf: missing key %s", key));
    if (v->ty == 6 || v->ty == 12) *out = (float)v->f; // Value::as_f32
    else if (v->ty == 8 || v->ty == 9) return g->fail(BIV_HIP_E_FORMAT, fmt("gguf: %s is not a number", key));
    else *out = (float)v->u;
    return 0;
}

int biv_gguf_get_str(biv_gguf *g, const char *key, char *buf, size_t len)
{
    if (!g || !key || !buf || !len) return BIV_HIP_E_INVALID;
    const Value *v = g->get(key);
    if (!v) return g->fail(BIV_HIP_E_MISSING, fmt("gguf: missing key %s", key));
    if (v->ty != 8) return g->fail(BIV_HIP_E_FORMAT, fmt("gguf: %s is not a string", key));
    if (v->s.size() + 1 > len) return g->fail(BIV_HIP_E_INVALID, fmt("gguf: %s needs %zu bytes", key, v->s.size() + 1));
    memcpy(buf, v->s.c_str(), v->s.size() + 1);
    return 0;
}

int biv_gguf_n_tensors(const biv_gguf *g) { return g ? (int)g->tensors.size() : 0; }

const char *biv_gguf_tensor_name(const biv_gguf *g, int i)
{
    return g && i >= 0 && i < (int)g->tensors.size() ? g->tensors[i].name.c_str() : nullptr;
}

int biv_gguf_tensor(biv_gguf *g, const char *name, int *ggml_type, int *n_dims, uint64_t dims[4], const void **data,
                    size_t *n_bytes)
{
    if (!g || !name) return BIV_HIP_E_INVALID;
    const TensorInfo *t = g->tensor(name);
    if (!t) return g->fail(BIV_HIP_E_MISSING, fmt("missing tensor %s", name));
    if (ggml_type) *ggml_type = t->ty;
    if (n_dims) *n_dims = (int)t->dims.size();
    if (dims)
        for (int d = 0; d < 4; d++) dims[d] = d < (int)t->dims.size() ? t->dims[d] : 1;
    if (data) *data = g->shards[t->shard].p + t->offset;
    if (n_bytes) *n_bytes = t->n_bytes;
    return 0;
}

// The MoE part of Config::from_gguf (engine/src/model.rs:70-120)
int biv_gguf_read_moe_config(biv_gguf *g, biv_gguf_moe_config *cfg)
{
    if (!g || !cfg) return BIV_HIP_E_INVALID;
    memset(cfg, 0, sizeof *cfg);
    int rc = biv_gguf_get_str(g, "general.architecture", cfg->arch, sizeof cfg->arch);
    if (rc) return rc;
    const std::string arch = cfg->arch;
    if (arch != "qwen35moe") return g->fail(BIV_HIP_E_TYPE, "unsupported architecture " + arch + ": the MoE loader takes qwen35moe");
    auto need = [&](const char *k, uint64_t &v) { return biv_gguf_get_u64(g, (arch + "." + k).c_str(), &v); };
    uint64_t block_count, nextn = 0, n_embd, n_expert, n_used, n_ff, n_ff_sh = 0;
    if ((rc = need("block_count", block_count)) || (rc = need("embedding_length", n_embd)) ||
        (rc = need("expert_count", n_expert)) || (rc = need("expert_used_count", n_used)) ||
        (rc = need("expert_feed_forward_length", n_ff)))
        return rc;
    (void)need("nextn_predict_layers", nextn);
    (void)need("expert_shared_feed_forward_length", n_ff_sh);
    g->err.clear();
    if (n_used == 0 || n_used > n_expert) return g->fail(BIV_HIP_E_INVALID, "expert_used_count not in 1..=expert_count");
    for (uint64_t v : {block_count, n_embd, n_expert, n_ff, n_ff_sh})
        if (v > INT32_MAX) return g->fail(BIV_HIP_E_INVALID, "a qwen35moe size is out of range");
    if (nextn > block_count) return g->fail(BIV_HIP_E_INVALID, "nextn_predict_layers > block_count");
    float eps = 0.0f;
    if ((rc = biv_gguf_get_f32(g, (arch + ".attention.layer_norm_rms_epsilon").c_str(), &eps))) return rc;
    cfg->n_layer = (int)(block_count - nextn);
    cfg->n_embd = (int)n_embd;
    cfg->n_expert = (int)n_expert;
    cfg->n_expert_used = (int)n_used;
    cfg->n_ff_exp = (int)n_ff;
    cfg->n_ff_shexp = (int)n_ff_sh;
    cfg->eps = eps;
    return 0;
}

int biv_gguf_read_dense_config(biv_gguf *g, biv_gguf_dense_config *cfg)
{
    if (!g || !cfg) return BIV_HIP_E_INVALID;
    memset(cfg, 0, sizeof *cfg);
    int rc = biv_gguf_get_str(g, "general.architecture", cfg->arch, sizeof cfg->arch);
    if (rc) return rc;
    const std::string arch = cfg->arch;
    if (arch != "qwen35") return g->fail(BIV_HIP_E_TYPE, "unsupported architecture " + arch + ": the dense loader takes qwen35");
    auto need = [&](const char *k, uint64_t &v) { return biv_gguf_get_u64(g, (arch + "." + k).c_str(), &v); };
    uint64_t block_count, nextn = 0, n_embd, n_ff;
    if ((rc = need("block_count", block_count)) || (rc = need("embedding_length", n_embd)) ||
        (rc = need("feed_forward_length", n_ff)))
        return rc;
    (void)need("nextn_predict_layers", nextn);
    g->err.clear();
    if (nextn > block_count) return g->fail(BIV_HIP_E_INVALID, "nextn_predict_layers > block_count");
    for (uint64_t v : {block_count, n_embd, n_ff})
        if (v > INT32_MAX) return g->fail(BIV_HIP_E_INVALID, "a qwen35 size is out of range");
    float eps = 0.0f;
    if ((rc = biv_gguf_get_f32(g, (arch + ".attention.layer_norm_rms_epsilon").c_str(), &eps))) return rc;
    cfg->n_layer = (int)(block_count - nextn);
    cfg->n_embd = (int)n_embd;
    cfg->n_ff = (int)n_ff;
    cfg->eps = eps;
    return 0;
}

} // extern "C"

// Loader::ffn for a dense layer (engine/src/model.rs:381-386): gate and up
// `[n_embd, n_ff]`, down `[n_ff, n_embd]`, shapes checked as Loader::weight.
extern "C" int biv_hip_dense_from_gguf(biv_hip_ctx *ctx, biv_gguf *g, int layer, biv_hip_dense **out)
{
    if (!ctx || !g || !out) return BIV_HIP_E_INVALID;
    biv_gguf_dense_config cfg;
    int rc = biv_gguf_read_dense_config(g, &cfg);
    if (rc) return biv_hip_fail_ext(ctx, rc, g->err.c_str());
    if (layer < 0 || layer >= cfg.n_layer)
        return biv_hip_fail_ext(ctx, BIV_HIP_E_INVALID, fmt("layer %d of %d", layer, cfg.n_layer).c_str());
    const size_t e = cfg.n_embd, ff = cfg.n_ff;
    const std::string blk = "blk." + std::to_string(layer) + ".";
    const TensorInfo *t[3];
    const char *names[3] = {"ffn_gate", "ffn_up", "ffn_down"};
    const std::vector<uint64_t> want[3] = {{e, ff}, {e, ff}, {ff, e}};
    biv_hip_weight *w[3];
    for (int i = 0; i < 3; i++) {
        const std::string name = blk + names[i] + ".weight";
        t[i] = g->tensor(name);
        if (!t[i]) return biv_hip_fail_ext(ctx, BIV_HIP_E_MISSING, ("missing tensor " + name).c_str());
        if (t[i]->dims != want[i]) {
            std::string d, wd;
            for (auto v : t[i]->dims) d += (d.empty() ? "" : ", ") + std::to_string(v);
            for (auto v : want[i]) wd += (wd.empty() ? "" : ", ") + std::to_string(v);
            return biv_hip_fail_ext(ctx, BIV_HIP_E_INVALID,
                                    ("tensor " + name + " has dims [" + d + "], expected [" + wd + "]").c_str());
        }
        const void *data = g->shards[t[i]->shard].p + t[i]->offset;
        if ((rc = biv_hip_upload_weight(ctx, t[i]->ty, want[i][0], want[i][1], data, &w[i]))) return rc;
    }
    return biv_hip_dense_create(ctx, w[0], w[1], w[2], out);
}

// Loader::ffn for a MoE layer (engine/src/model.rs:386-421), uploading each
// matrix: the router `[n_embd, n_expert]`, the experts `[cols, rows, n]` (or
// the fused gate_up `[n_embd, 2 ff, n]`, gate rows then up rows per expert),
// the shared expert and its gate vector.  Shapes are checked as
// Loader::weight / experts / row do (Error::TensorShape).
extern "C" int biv_hip_moe_from_gguf(biv_hip_ctx *ctx, biv_gguf *g, int layer, biv_hip_moe **out)
{
    if (!ctx || !g || !out) return BIV_HIP_E_INVALID;
    biv_gguf_moe_config cfg;
    int rc = biv_gguf_read_moe_config(g, &cfg);
    if (rc) return biv_hip_fail_ext(ctx, rc, g->err.c_str());
    if (layer < 0 || layer >= cfg.n_layer)
        return biv_hip_fail_ext(ctx, BIV_HIP_E_INVALID, fmt("layer %d of %d", layer, cfg.n_layer).c_str());
    const size_t e = cfg.n_embd, n = cfg.n_expert, ff = cfg.n_ff_exp, sff = cfg.n_ff_shexp;
    // the shapes the kernels take, checked before anything is uploaded
    // (biv_hip_moe_create checks them again on the uploaded parts)
    auto width_ok = [](size_t K) { return K == 512 || K == 1024 || K == 2048; };
    if (!width_ok(e) || !width_ok(ff) || n > 256 || cfg.n_expert_used > 16 || (sff && sff != ff))
        return biv_hip_fail_ext(ctx, BIV_HIP_E_INVALID,
                                fmt("n_embd %zu, n_ff %zu, %zu experts (%d used), shared n_ff %zu: the kernels take "
                                    "n_embd and n_ff of 512, 1024 or 2048, at most 256 experts, k <= 16 and a "
                                    "shared expert as wide as the routed ones",
                                    e, ff, n, cfg.n_expert_used, sff)
                                    .c_str());
    const std::string blk = "blk." + std::to_string(layer) + ".";
    auto find = [&](const std::string &name, std::vector<uint64_t> want, const TensorInfo *&t) -> int {
        t = g->tensor(name + ".weight");
        if (!t) return biv_hip_fail_ext(ctx, BIV_HIP_E_MISSING, ("missing tensor " + name + ".weight").c_str());
        if (t->dims != want) {
            std::string d, w;
            for (auto v : t->dims) d += (d.empty() ? "" : ", ") + std::to_string(v);
            for (auto v : want) w += (w.empty() ? "" : ", ") + std::to_string(v);
            return biv_hip_fail_ext(ctx, BIV_HIP_E_INVALID,
                                    ("tensor " + name + ".weight has dims [" + d + "], expected [" + w + "]").c_str());
        }
        return 0;
    };
    auto bytes = [&](const TensorInfo *t) { return static_cast<const void *>(g->shards[t->shard].p + t->offset); };
    auto row_bytes = [](const TensorInfo *t, size_t cols) {
        size_t be = 1, bb = 1;
        type_block((uint32_t)t->ty, be, bb);
        return cols / be * bb;
    };
    const TensorInfo *tr, *tg = nullptr, *tu = nullptr, *tgu = nullptr, *td;
    if ((rc = find(blk + "ffn_gate_inp", {e, n}, tr))) return rc;
    biv_hip_weight *router;
    if ((rc = biv_hip_upload_weight(ctx, tr->ty, e, n, bytes(tr), &router))) return rc;
    biv_hip_experts *gate, *up, *down;
    if (g->tensor(blk + "ffn_gate_up_exps.weight")) {
        // gate rows then up rows, per expert
        if ((rc = find(blk + "ffn_gate_up_exps", {e, 2 * ff, n}, tgu))) return rc;
        const size_t rb = row_bytes(tgu, e), stride = 2 * ff * rb;
        if ((rc = biv_hip_upload_experts(ctx, tgu->ty, e, ff, n, bytes(tgu), stride, 0, &gate)) ||
            (rc = biv_hip_upload_experts(ctx, tgu->ty, e, ff, n, bytes(tgu), stride, ff * rb, &up)))
            return rc;
    } else {
        if ((rc = find(blk + "ffn_gate_exps", {e, ff, n}, tg)) || (rc = find(blk + "ffn_up_exps", {e, ff, n}, tu)))
            return rc;
        if ((rc = biv_hip_upload_experts(ctx, tg->ty, e, ff, n, bytes(tg), ff * row_bytes(tg, e), 0, &gate)) ||
            (rc = biv_hip_upload_experts(ctx, tu->ty, e, ff, n, bytes(tu), ff * row_bytes(tu, e), 0, &up)))
            return rc;
    }
    if ((rc = find(blk + "ffn_down_exps", {ff, e, n}, td))) return rc;
    if ((rc = biv_hip_upload_experts(ctx, td->ty, ff, e, n, bytes(td), e * row_bytes(td, ff), 0, &down))) return rc;
    biv_hip_weight *sg = nullptr, *su = nullptr, *sd = nullptr, *gi = nullptr;
    if (sff) {
        const TensorInfo *t1, *t2, *t3, *t4;
        if ((rc = find(blk + "ffn_gate_shexp", {e, sff}, t1)) || (rc = find(blk + "ffn_up_shexp", {e, sff}, t2)) ||
            (rc = find(blk + "ffn_down_shexp", {sff, e}, t3)) || (rc = find(blk + "ffn_gate_inp_shexp", {e}, t4)))
            return rc;
        if ((rc = biv_hip_upload_weight(ctx, t1->ty, e, sff, bytes(t1), &sg)) ||
            (rc = biv_hip_upload_weight(ctx, t2->ty, e, sff, bytes(t2), &su)) ||
            (rc = biv_hip_upload_weight(ctx, t3->ty, sff, e, bytes(t3), &sd)) ||
            (rc = biv_hip_upload_weight(ctx, t4->ty, e, 1, bytes(t4), &gi)))
            return rc;
    }
    return biv_hip_moe_create(ctx, router, gate, up, down, sg, su, sd, gi, cfg.n_expert_used, out);
}
