// GGUF reader (gguf.rs:113-336) and the model description it yields
// (Config::from_gguf, model.rs:31-97; Model::load's tensor binding and
// checks, model.rs:487-601; Tokenizer::from_gguf's vocabulary size and
// end-of-generation ids, tokenizer.rs:41-109).  Host code only: the tensors
// stay in the read-only mapping and the descriptor points into it, so
// pi_hip_model_bind uploads them straight from the file.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/pocketinfer_hip.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;   // "GGUF"

enum KvType : uint32_t {
    KV_U8 = 0, KV_I8 = 1, KV_U16 = 2, KV_I16 = 3, KV_U32 = 4, KV_I32 = 5, KV_F32 = 6, KV_BOOL = 7,
    KV_STR = 8, KV_ARR = 9, KV_U64 = 10, KV_I64 = 11, KV_F64 = 12,
};

struct Kv {
    uint32_t type = 0;
    uint64_t u = 0;       // integer and bool values (sign-extended for signed types)
    double f = 0.0;       // F32 / F64
    size_t off = 0, len = 0;   // string: bytes; array: first element
    uint32_t etype = 0;   // array element type
    uint64_t count = 0;   // array length
};

struct TensorInfo {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t ne[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0;
};

// quant.rs:19-37: (elements, bytes) of a block.
bool type_block(uint32_t t, uint64_t *be, uint64_t *bb) {
    switch (t) {
    case 0: *be = 1; *bb = 4; return true;     // F32
    case 1: case 30: *be = 1; *bb = 2; return true;   // F16, BF16
    case 2: *be = 32; *bb = 18; return true;   // Q4_0
    case 3: *be = 32; *bb = 20; return true;   // Q4_1
    case 6: *be = 32; *bb = 22; return true;   // Q5_0
    case 7: *be = 32; *bb = 24; return true;   // Q5_1
    case 8: *be = 32; *bb = 34; return true;   // Q8_0
    case 9: *be = 32; *bb = 36; return true;   // Q8_1
    case 10: *be = 256; *bb = 84; return true;    // Q2_K
    case 11: *be = 256; *bb = 110; return true;   // Q3_K
    case 12: *be = 256; *bb = 144; return true;   // Q4_K
    case 13: *be = 256; *bb = 176; return true;   // Q5_K
    case 14: *be = 256; *bb = 210; return true;   // Q6_K
    case 15: *be = 256; *bb = 292; return true;   // Q8_K
    default: return false;
    }
}

// quant.rs:60-72: bytes of a tensor; false with a message on error.
bool tensor_nbytes(uint32_t t, const uint64_t *ne, uint32_t nd, uint64_t *out, std::string &err) {
    uint64_t be, bb;
    if (!type_block(t, &be, &bb)) { err = "unsupported tensor type " + std::to_string(t); return false; }
    uint64_t n = 1;
    for (uint32_t i = 0; i < nd; i++) {
        if (i == 0 && ne[i] % be) { err = "dim0 " + std::to_string(ne[i]) + " not divisible by block " + std::to_string(be); return false; }
        if (ne[i] && n > UINT64_MAX / ne[i]) { err = "tensor element count overflow"; return false; }
        n *= ne[i];
    }
    const uint64_t blocks = n / be;
    if (blocks && bb > UINT64_MAX / blocks) { err = "tensor byte size overflow"; return false; }
    *out = blocks * bb;
    return true;
}

struct Reader {
    const uint8_t *b;
    size_t n, o = 0;
    std::string err;
    bool need(size_t k) {
        if (k > n - std::min(o, n)) {
            if (err.empty()) err = "gguf truncated at offset " + std::to_string(o);
            return false;
        }
        return true;
    }
    bool u8(uint64_t &v) { if (!need(1)) return false; v = b[o]; o += 1; return true; }
    bool u16(uint64_t &v) { if (!need(2)) return false; v = (uint64_t)b[o] | ((uint64_t)b[o + 1] << 8); o += 2; return true; }
    bool u32(uint64_t &v) {
        if (!need(4)) return false;
        uint32_t x;
        memcpy(&x, b + o, 4);
        v = x;
        o += 4;
        return true;
    }
    bool u64(uint64_t &v) { if (!need(8)) return false; memcpy(&v, b + o, 8); o += 8; return true; }
    bool str(size_t &off, size_t &len) {
        uint64_t l;
        if (!u64(l)) return false;
        if (l > n || !need((size_t)l)) { if (err.empty()) err = "gguf truncated at offset " + std::to_string(o); return false; }
        off = o;
        len = (size_t)l;
        o += (size_t)l;
        return true;
    }
    // gguf.rs:338-366
    bool skip_array(uint32_t et, uint64_t count, int depth = 0) {
        if (depth > 8) { err = "gguf arrays nested too deeply"; return false; }
        uint64_t v;
        size_t so, sl;
        for (uint64_t i = 0; i < count; i++) {
            switch (et) {
            case KV_U8: case KV_I8: case KV_BOOL: if (!u8(v)) return false; break;
            case KV_U16: case KV_I16: if (!u16(v)) return false; break;
            case KV_U32: case KV_I32: case KV_F32: if (!u32(v)) return false; break;
            case KV_U64: case KV_I64: case KV_F64: if (!u64(v)) return false; break;
            case KV_STR: if (!str(so, sl)) return false; break;
            case KV_ARR: {
                uint64_t e2, c2;
                if (!u32(e2) || !u64(c2) || !skip_array((uint32_t)e2, c2, depth + 1)) return false;
                break;
            }
            default: err = "unknown array element type " + std::to_string(et); return false;
            }
        }
        return true;
    }
};

}  // namespace

struct pi_gguf {
    const uint8_t *bytes = nullptr;
    size_t len = 0;
    void *map = nullptr;     // mmap'd file (null for pi_gguf_parse)
    uint32_t version = 0;
    uint64_t data_offset = 0;
    std::vector<TensorInfo> tensors;
    std::unordered_map<std::string, Kv> kv;
    std::vector<std::string> order;
};

namespace {

int gfail(char *err, size_t n, const char *fmt, ...) {
    if (err && n) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, n, fmt, ap);
        va_end(ap);
    }
    return PI_E_INVALID;
}

// Gguf::parse (gguf.rs:113-192).
int parse(pi_gguf *g, char *err, size_t errn) {
    Reader r{g->bytes, g->len};
    uint64_t magic, version, n_tensors, n_kv;
    if (!r.u32(magic)) return gfail(err, errn, "%s", r.err.c_str());
    if (magic != kMagic) return gfail(err, errn, "not a GGUF file (magic %#llx)", (unsigned long long)magic);
    if (!r.u32(version)) return gfail(err, errn, "%s", r.err.c_str());
    if (version < 2 || version > 3) return gfail(err, errn, "unsupported GGUF version %llu", (unsigned long long)version);
    g->version = (uint32_t)version;
    if (!r.u64(n_tensors) || !r.u64(n_kv)) return gfail(err, errn, "%s", r.err.c_str());
    if (n_tensors > 1000000 || n_kv > 1000000) return gfail(err, errn, "implausible gguf header");
    g->tensors.reserve((size_t)n_tensors);
    for (uint64_t i = 0; i < n_kv; i++) {
        size_t ko, kl;
        uint64_t t;
        if (!r.str(ko, kl) || !r.u32(t)) return gfail(err, errn, "%s", r.err.c_str());
        std::string key(reinterpret_cast<const char *>(g->bytes + ko), kl);
        Kv v;
        v.type = (uint32_t)t;
        uint64_t x;
        bool ok = true;
        switch (t) {
        case KV_U8: ok = r.u8(x); v.u = x; break;
        case KV_I8: ok = r.u8(x); v.u = (uint64_t)(int64_t)(int8_t)x; break;
        case KV_U16: ok = r.u16(x); v.u = x; break;
        case KV_I16: ok = r.u16(x); v.u = (uint64_t)(int64_t)(int16_t)x; break;
        case KV_U32: ok = r.u32(x); v.u = x; break;
        case KV_I32: ok = r.u32(x); v.u = (uint64_t)(int64_t)(int32_t)x; break;
        case KV_F32: {
            ok = r.u32(x);
            float f;
            const uint32_t b32 = (uint32_t)x;
            memcpy(&f, &b32, 4);
            v.f = f;
            break;
        }
        case KV_BOOL: ok = r.u8(x); v.u = x != 0; break;
        case KV_STR: ok = r.str(v.off, v.len); break;
        case KV_ARR: {
            uint64_t et, cnt;
            ok = r.u32(et) && r.u64(cnt);
            if (ok) {
                v.etype = (uint32_t)et;
                v.count = cnt;
                v.off = r.o;
                ok = r.skip_array((uint32_t)et, cnt);
            }
            break;
        }
        case KV_U64: ok = r.u64(x); v.u = x; break;
        case KV_I64: ok = r.u64(x); v.u = x; break;
        case KV_F64: {
            ok = r.u64(x);
            double d;
            memcpy(&d, &x, 8);
            v.f = d;
            break;
        }
        default: return gfail(err, errn, "unknown gguf metadata type %llu for key %s", (unsigned long long)t, key.c_str());
        }
        if (!ok) return gfail(err, errn, "%s", r.err.c_str());
        g->order.push_back(key);
        g->kv[key] = v;
    }
    for (uint64_t i = 0; i < n_tensors; i++) {
        size_t no, nl;
        uint64_t nd;
        if (!r.str(no, nl) || !r.u32(nd)) return gfail(err, errn, "%s", r.err.c_str());
        TensorInfo ti;
        ti.name.assign(reinterpret_cast<const char *>(g->bytes + no), nl);
        if (nd > 4) return gfail(err, errn, "tensor %s has %llu dims", ti.name.c_str(), (unsigned long long)nd);
        ti.n_dims = (uint32_t)nd;
        for (uint32_t d = 0; d < nd; d++)
            if (!r.u64(ti.ne[d])) return gfail(err, errn, "%s", r.err.c_str());
        uint64_t tt;
        if (!r.u32(tt) || !r.u64(ti.offset)) return gfail(err, errn, "%s", r.err.c_str());
        ti.type = (uint32_t)tt;
        g->tensors.push_back(std::move(ti));
    }
    uint64_t alignment = 32;
    auto it = g->kv.find("general.alignment");
    if (it != g->kv.end() && (it->second.type == KV_U32 || it->second.type == KV_U64 || it->second.type == KV_I32))
        alignment = it->second.u;
    alignment = std::max<uint64_t>(alignment, 1);
    if (r.o > UINT64_MAX - (alignment - 1)) return gfail(err, errn, "invalid GGUF alignment");
    g->data_offset = (r.o + alignment - 1) / alignment * alignment;
    if (g->data_offset > g->len) return gfail(err, errn, "GGUF tensor data begins past the end of the file");
    return PI_OK;
}

const Kv *find_kv(const pi_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    auto it = g->kv.find(key);
    return it == g->kv.end() ? nullptr : &it->second;
}

// Gguf::get_u64 (gguf.rs:206-219): any integer type.
bool kv_u64(const Kv *v, uint64_t *out) {
    if (!v) return false;
    switch (v->type) {
    case KV_U8: case KV_U16: case KV_U32: case KV_U64: case KV_I8: case KV_I16: case KV_I32: case KV_I64:
        *out = v->u;
        return true;
    default: return false;
    }
}

// Gguf::get_f32 (gguf.rs:229-235).
bool kv_f32(const Kv *v, float *out) {
    if (!v) return false;
    if (v->type == KV_F32 || v->type == KV_F64) { *out = (float)v->f; return true; }
    uint64_t u;
    if (kv_u64(v, &u)) { *out = (float)u; return true; }
    return false;
}

}  // namespace

extern "C" {

int pi_gguf_parse(const void *bytes, size_t len, pi_gguf **out, char *err, size_t errn) {
    if (!out) return PI_E_INVALID;
    *out = nullptr;
    if (!bytes && len) return gfail(err, errn, "null GGUF bytes");
    pi_gguf *g = new pi_gguf();
    g->bytes = static_cast<const uint8_t *>(bytes);
    g->len = len;
    const int r = parse(g, err, errn);
    if (r) { delete g; return r; }
    *out = g;
    return PI_OK;
}

int pi_gguf_open(const char *path, pi_gguf **out, char *err, size_t errn) {
    if (!out || !path) return PI_E_INVALID;
    *out = nullptr;
    // MappedFile::open (util.rs:163-192): read-only, private mapping
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return gfail(err, errn, "open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return gfail(err, errn, "stat %s: %s", path, strerror(errno)); }
    const size_t len = (size_t)st.st_size;
    void *m = nullptr;
    if (len) {
        m = mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) { close(fd); return gfail(err, errn, "mmap %s: %s", path, strerror(errno)); }
    }
    close(fd);
    pi_gguf *g = new pi_gguf();
    g->bytes = static_cast<const uint8_t *>(m);
    g->len = len;
    g->map = m;
    const int r = parse(g, err, errn);
    if (r) {
        if (m) munmap(m, len);
        delete g;
        return r;
    }
    *out = g;
    return PI_OK;
}

void pi_gguf_close(pi_gguf *g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->len);
    delete g;
}

uint32_t pi_gguf_version(const pi_gguf *g) { return g ? g->version : 0; }
size_t pi_gguf_n_tensors(const pi_gguf *g) { return g ? g->tensors.size() : 0; }
size_t pi_gguf_n_kv(const pi_gguf *g) { return g ? g->order.size() : 0; }
uint64_t pi_gguf_data_offset(const pi_gguf *g) { return g ? g->data_offset : 0; }

const char *pi_gguf_key(const pi_gguf *g, size_t i) {
    return g && i < g->order.size() ? g->order[i].c_str() : nullptr;
}

int pi_gguf_kv_type(const pi_gguf *g, const char *key, uint32_t *type) {
    const Kv *v = find_kv(g, key);
    if (!v || !type) return PI_E_INVALID;
    *type = v->type;
    return PI_OK;
}

int pi_gguf_get_u64(const pi_gguf *g, const char *key, uint64_t *v) {
    return v && kv_u64(find_kv(g, key), v) ? PI_OK : PI_E_INVALID;
}

int pi_gguf_get_f32(const pi_gguf *g, const char *key, float *v) {
    return v && kv_f32(find_kv(g, key), v) ? PI_OK : PI_E_INVALID;
}

int pi_gguf_get_bool(const pi_gguf *g, const char *key, int *v) {
    const Kv *k = find_kv(g, key);
    if (!k || !v || (k->type != KV_BOOL && k->type != KV_U8)) return PI_E_INVALID;
    *v = k->u != 0;
    return PI_OK;
}

int pi_gguf_get_str(const pi_gguf *g, const char *key, const char **s, size_t *len) {
    const Kv *k = find_kv(g, key);
    if (!k || !s || !len || k->type != KV_STR) return PI_E_INVALID;
    *s = reinterpret_cast<const char *>(g->bytes + k->off);
    *len = k->len;
    return PI_OK;
}

int pi_gguf_array_info(const pi_gguf *g, const char *key, uint32_t *etype, uint64_t *count) {
    const Kv *k = find_kv(g, key);
    if (!k || !etype || !count || k->type != KV_ARR) return PI_E_INVALID;
    *etype = k->etype;
    *count = k->count;
    return PI_OK;
}

int pi_gguf_array_str(const pi_gguf *g, const char *key, uint64_t i, const char **s, size_t *len) {
    const Kv *k = find_kv(g, key);
    if (!k || !s || !len || k->type != KV_ARR || k->etype != KV_STR || i >= k->count) return PI_E_INVALID;
    Reader r{g->bytes, g->len};
    r.o = k->off;
    size_t o = 0, l = 0;
    for (uint64_t j = 0; j <= i; j++)
        if (!r.str(o, l)) return PI_E_INVALID;
    *s = reinterpret_cast<const char *>(g->bytes + o);
    *len = l;
    return PI_OK;
}

int pi_gguf_array_i32(const pi_gguf *g, const char *key, int32_t *out, size_t n) {
    const Kv *k = find_kv(g, key);
    if (!k || k->type != KV_ARR || k->etype != KV_I32 || (n && !out) || n > k->count) return PI_E_INVALID;
    memcpy(out, g->bytes + k->off, n * 4);
    return PI_OK;
}

int pi_gguf_array_f32(const pi_gguf *g, const char *key, float *out, size_t n) {
    const Kv *k = find_kv(g, key);
    if (!k || k->type != KV_ARR || k->etype != KV_F32 || (n && !out) || n > k->count) return PI_E_INVALID;
    memcpy(out, g->bytes + k->off, n * 4);
    return PI_OK;
}

int64_t pi_gguf_find_tensor(const pi_gguf *g, const char *name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->tensors.size(); i++)
        if (g->tensors[i].name == name) return (int64_t)i;
    return -1;
}

int pi_gguf_tensor_info(const pi_gguf *g, size_t i, const char **name, uint32_t *type, uint32_t *n_dims, uint64_t ne[4],
                        uint64_t *offset) {
    if (!g || i >= g->tensors.size()) return PI_E_INVALID;
    const TensorInfo &t = g->tensors[i];
    if (name) *name = t.name.c_str();
    if (type) *type = t.type;
    if (n_dims) *n_dims = t.n_dims;
    if (ne)
        for (int d = 0; d < 4; d++) ne[d] = t.ne[d];
    if (offset) *offset = t.offset;
    return PI_OK;
}

int pi_gguf_tensor_data(const pi_gguf *g, size_t i, const void **data, size_t *nbytes, char *err, size_t errn) {
    if (!g || i >= g->tensors.size() || !data || !nbytes) return PI_E_INVALID;
    const TensorInfo &t = g->tensors[i];
    if (t.offset > UINT64_MAX - g->data_offset) return gfail(err, errn, "tensor %s offset overflow", t.name.c_str());
    const uint64_t start = g->data_offset + t.offset;
    if (start > g->len) return gfail(err, errn, "tensor %s outside file", t.name.c_str());
    uint64_t n;
    std::string e;
    if (!tensor_nbytes(t.type, t.ne, t.n_dims, &n, e)) return gfail(err, errn, "%s", e.c_str());
    if (n > g->len - start) return gfail(err, errn, "tensor %s truncated (need %llu bytes)", t.name.c_str(), (unsigned long long)n);
    *data = g->bytes + start;
    *nbytes = (size_t)n;
    return PI_OK;
}

// Config::from_gguf (model.rs:31-97), Model::load / finish (487-601) and the
// tokenizer's vocabulary size and end-of-generation ids (tokenizer.rs:41-109).
int pi_gguf_model_desc(const pi_gguf *g, pi_model_desc *m, pi_layer_desc *layers, uint32_t max_layers, uint32_t *eos,
                       uint32_t max_eos, char *err, size_t errn) {
    if (!g || !m) return PI_E_INVALID;
    memset(m, 0, sizeof *m);
    std::string p = "llama";
    const Kv *arch = find_kv(g, "general.architecture");
    if (arch && arch->type == KV_STR && arch->len) p.assign(reinterpret_cast<const char *>(g->bytes + arch->off), arch->len);
    auto meta_u = [&](const char *key, uint64_t *v) { return kv_u64(find_kv(g, (p + "." + key).c_str()), v); };
    auto meta_f = [&](const char *key, float *v) { return kv_f32(find_kv(g, (p + "." + key).c_str()), v); };
    uint64_t n_layer, n_embd, n_ff, n_head;
    if (!meta_u("block_count", &n_layer)) return gfail(err, errn, "missing metadata %s.block_count", p.c_str());
    if (!meta_u("embedding_length", &n_embd)) return gfail(err, errn, "missing metadata %s.embedding_length", p.c_str());
    if (!meta_u("feed_forward_length", &n_ff)) return gfail(err, errn, "missing metadata %s.feed_forward_length", p.c_str());
    if (!meta_u("attention.head_count", &n_head)) return gfail(err, errn, "missing metadata %s.attention.head_count", p.c_str());
    if (n_layer == 0 || n_embd == 0 || n_ff == 0 || n_head == 0)
        return gfail(err, errn, "invalid model configuration: zero layer, hidden, FFN or head count");
    uint64_t n_kv = n_head, head_dim = n_embd / n_head, n_rot, vd, n_vocab_meta = 0;
    meta_u("attention.head_count_kv", &n_kv);
    meta_u("attention.key_length", &head_dim);
    if (head_dim == 0 || n_kv == 0 || n_head % n_kv)
        return gfail(err, errn, "invalid GQA configuration: %llu/%llu with head_dim=%llu", (unsigned long long)n_head,
                     (unsigned long long)n_kv, (unsigned long long)head_dim);
    if (meta_u("attention.value_length", &vd) && vd != head_dim)
        return gfail(err, errn, "value head dimension %llu differs from key dimension %llu", (unsigned long long)vd,
                     (unsigned long long)head_dim);
    n_rot = head_dim;
    meta_u("rope.dimension_count", &n_rot);
    float theta = 10000.0f, eps = 1e-5f;
    meta_f("rope.freq_base", &theta);
    meta_f("attention.layer_norm_rms_epsilon", &eps);
    meta_u("vocab_size", &n_vocab_meta);
    if (n_rot == 0 || n_rot > head_dim || n_rot % 2 || !std::isfinite(theta) || theta <= 0.0f ||
        !std::isfinite(eps) || eps <= 0.0f)
        return gfail(err, errn, "invalid RoPE / RMSNorm configuration");
    if (n_layer > max_layers || !layers)
        return gfail(err, errn, "model has %llu layers, room for %u", (unsigned long long)n_layer, max_layers);
    if (n_layer > 0xFFFFFFFFull || n_embd > 0xFFFFFFFFull || n_ff > 0xFFFFFFFFull || n_head > 0xFFFFFFFFull ||
        head_dim > 0xFFFFFFFFull)
        return gfail(err, errn, "model dimensions overflow 32 bits");
    // the tokenizer's vocabulary and end-of-generation ids
    const Kv *toks = find_kv(g, "tokenizer.ggml.tokens");
    if (!toks || toks->type != KV_ARR || toks->etype != KV_STR) return gfail(err, errn, "metadata tokenizer.ggml.tokens is not a string array");
    const uint64_t vocab = toks->count;
    std::vector<uint32_t> ids;
    uint64_t e;
    if (kv_u64(find_kv(g, "tokenizer.ggml.eos_token_id"), &e)) ids.push_back((uint32_t)e);
    const Kv *tt = find_kv(g, "tokenizer.ggml.token_type");
    const bool have_types = tt && tt->type == KV_ARR && tt->etype == KV_I32 && tt->count >= vocab;
    {
        Reader r{g->bytes, g->len};
        r.o = toks->off;
        for (uint64_t i = 0; i < vocab; i++) {
            size_t so, sl;
            if (!r.str(so, sl)) return gfail(err, errn, "%s", r.err.c_str());
            int32_t ty = 1;
            if (have_types) memcpy(&ty, g->bytes + tt->off + 4 * i, 4);
            if (ty != 2 && ty != 3 && ty != 4) continue;
            const std::string s(reinterpret_cast<const char *>(g->bytes + so), sl);
            if (s == "<|im_end|>" || s == "<|eot|>" || s == "<|endoftext|>") ids.push_back((uint32_t)i);
        }
    }
    std::sort(ids.begin(), ids.end());
    ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
    if (ids.size() > max_eos || (!ids.empty() && !eos))
        return gfail(err, errn, "%zu end-of-generation ids, room for %u", ids.size(), max_eos);
    for (size_t i = 0; i < ids.size(); i++) eos[i] = ids[i];
    // tensors (Model::load's find, model.rs:494-523)
    std::string ferr;
    auto find = [&](const std::string &name, pi_tensor_desc *d) -> bool {
        const int64_t idx = pi_gguf_find_tensor(g, name.c_str());
        if (idx < 0) { ferr = "missing tensor " + name; return false; }
        const TensorInfo &t = g->tensors[(size_t)idx];
        uint64_t be, bb;
        if (!type_block(t.type, &be, &bb)) { ferr = "tensor " + name + ": unsupported type " + std::to_string(t.type); return false; }
        if (t.n_dims == 0 || t.n_dims > 2 || t.ne[0] == 0 || (t.n_dims == 2 && t.ne[1] == 0)) {
            ferr = "tensor " + name + ": expected one or two nonzero dimensions";
            return false;
        }
        const void *data;
        size_t nb;
        char e2[256];
        if (pi_gguf_tensor_data(g, (size_t)idx, &data, &nb, e2, sizeof e2)) {
            ferr = std::string("tensor ") + name + ": out of range (" + e2 + ")";
            return false;
        }
        d->type = t.type;
        d->ne0 = t.ne[0];
        d->ne1 = t.n_dims == 2 ? t.ne[1] : 1;
        d->data = data;
        return true;
    };
    if (!find("token_embd.weight", &m->token_embd)) return gfail(err, errn, "%s", ferr.c_str());
    if (pi_gguf_find_tensor(g, "output.weight") >= 0) {
        if (!find("output.weight", &m->output)) return gfail(err, errn, "%s", ferr.c_str());
    } else {
        m->output = m->token_embd;   // tied embeddings (model.rs:526-530)
    }
    if (!find("output_norm.weight", &m->output_norm)) return gfail(err, errn, "%s", ferr.c_str());
    for (uint64_t l = 0; l < n_layer; l++) {
        const std::string b = "blk." + std::to_string(l) + ".";
        pi_layer_desc &L = layers[l];
        if (!find(b + "attn_q.weight", &L.attn_q) || !find(b + "attn_k.weight", &L.attn_k) ||
            !find(b + "attn_v.weight", &L.attn_v) || !find(b + "attn_output.weight", &L.attn_o) ||
            !find(b + "attn_norm.weight", &L.attn_norm) || !find(b + "ffn_gate.weight", &L.ffn_gate) ||
            !find(b + "ffn_up.weight", &L.ffn_up) || !find(b + "ffn_down.weight", &L.ffn_down) ||
            !find(b + "ffn_norm.weight", &L.ffn_norm))
            return gfail(err, errn, "%s", ferr.c_str());
    }
    // Model::finish (model.rs:571-601)
    if (vocab == 0 || m->token_embd.ne0 != n_embd || m->token_embd.ne1 != vocab || (n_vocab_meta && n_vocab_meta != vocab))
        return gfail(err, errn, "embedding / metadata / tokenizer vocab dimensions disagree");
    auto shape = [&](const pi_tensor_desc &t, uint64_t cols, uint64_t rows) { return t.ne0 == cols && t.ne1 == rows; };
    if (!shape(m->output, n_embd, vocab) || !shape(m->output_norm, n_embd, 1))
        return gfail(err, errn, "output tensor shape mismatch");
    const uint64_t qdim = n_head * head_dim, kdim = n_kv * head_dim;
    for (uint64_t l = 0; l < n_layer; l++) {
        const pi_layer_desc &L = layers[l];
        if (!shape(L.attn_norm, n_embd, 1) || !shape(L.ffn_norm, n_embd, 1) || !shape(L.attn_q, n_embd, qdim) ||
            !shape(L.attn_k, n_embd, kdim) || !shape(L.attn_v, n_embd, kdim) || !shape(L.attn_o, qdim, n_embd) ||
            !shape(L.ffn_gate, n_embd, n_ff) || !shape(L.ffn_up, n_embd, n_ff) || !shape(L.ffn_down, n_ff, n_embd))
            return gfail(err, errn, "layer %llu tensor shape mismatch", (unsigned long long)l);
    }
    m->n_layer = (uint32_t)n_layer;
    m->n_embd = (uint32_t)n_embd;
    m->n_ff = (uint32_t)n_ff;
    m->n_head = (uint32_t)n_head;
    m->n_head_kv = (uint32_t)n_kv;
    m->head_dim = (uint32_t)head_dim;
    m->n_rot = (uint32_t)n_rot;
    m->n_vocab = (uint32_t)vocab;
    m->rope_theta = theta;
    m->rms_eps = eps;
    m->eos_ids = eos;
    m->n_eos = (uint32_t)ids.size();
    m->layers = layers;
    return PI_OK;
}

}  // extern "C"
