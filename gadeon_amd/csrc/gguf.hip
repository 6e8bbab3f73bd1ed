// GGUF v3 reader (host only): map the file, parse the header, the key/value
// metadata and the tensor directory, and hand out each tensor's dims, ggml
// type and bytes inside the mapping.  Same layout and rules as the
// reference's GGUF.swift (LLM/src/Shared/GGUF.swift:45-117): little-endian,
// u64 counts, strings as (u64 length, bytes), tensor data from the first
// multiple of general.alignment (default 32) after the directory, each
// tensor at that start plus its offset.  Every read is bounds-checked against
// the file size, so a truncated or corrupt file is an error, never an
// out-of-range read.
#include "gd_internal.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

struct GgufValue {
    int kind = 0;   // 0 int, 1 float, 2 string, 3 int array, 4 float array, 5 string array, 6 bool
    int64_t i = 0;
    double f = 0;
    std::string s;
    std::vector<int64_t> ia;
    std::vector<double> fa;
    std::vector<std::string> sa;
};

struct GgufTensor {
    int ndim = 0;
    int64_t dims[4] = {1, 1, 1, 1};
    int type = 0;
    const uint8_t *data = nullptr;
    size_t bytes = 0;
};

struct gd_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    size_t size = 0;
    int version = 0;
    std::map<std::string, GgufValue> meta;
    std::map<std::string, GgufTensor> tensors;
};

namespace {

// Bytes of n elements of ggml type t, for the types GGUFType lists
// (GGUF.swift:7-14, rowByteCount :107-117): elements per block and bytes per
// block of each ggml format.  0 for a type outside that list or an element
// count that is not whole blocks; the reader rejects the tensor then.
size_t type_bytes(int t, int64_t n) {
    int64_t per = 0, bytes = 0;
    switch (t) {
    case 0: per = 1; bytes = 4; break;              // f32
    case 1: case 30: per = 1; bytes = 2; break;     // f16, bf16
    case 2: per = 32; bytes = 18; break;            // q4_0
    case 3: per = 32; bytes = 20; break;            // q4_1
    case 6: per = 32; bytes = 22; break;            // q5_0
    case 7: per = 32; bytes = 24; break;            // q5_1
    case 8: per = 32; bytes = 34; break;            // q8_0
    case 9: per = 32; bytes = 36; break;            // q8_1
    case 10: per = 256; bytes = 84; break;          // q2_K
    case 11: per = 256; bytes = 110; break;         // q3_K
    case 12: per = 256; bytes = 144; break;         // q4_K
    case 13: per = 256; bytes = 176; break;         // q5_K
    case 14: per = 256; bytes = 210; break;         // q6_K
    case 15: per = 256; bytes = 292; break;         // q8_K
    case 41: per = 128; bytes = 18; break;          // q1_0
    case 42: per = 128; bytes = 34; break;          // q2_0
    default: return 0;
    }
    return n % per ? 0 : (size_t)(n / per * bytes);
}

struct Cursor {
    const uint8_t *base;
    size_t size, pos = 0;
    bool bad = false;
    const uint8_t *take(size_t n) {
        if (bad || n > size - pos) { bad = true; return nullptr; }
        const uint8_t *p = base + pos;
        pos += n;
        return p;
    }
    template <typename T> T get() {
        T v{};
        if (const uint8_t *p = take(sizeof(T))) memcpy(&v, p, sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (bad || n > size - pos) { bad = true; return {}; }
        const uint8_t *p = take((size_t)n);
        return p ? std::string((const char *)p, (size_t)n) : std::string();
    }
    // One scalar of GGUF value type t into v; false for an unknown type.
    bool scalar(uint32_t t, GgufValue &v) {
        switch (t) {
        case 0: v.kind = 0; v.i = get<uint8_t>(); return true;
        case 1: v.kind = 0; v.i = get<int8_t>(); return true;
        case 2: v.kind = 0; v.i = get<uint16_t>(); return true;
        case 3: v.kind = 0; v.i = get<int16_t>(); return true;
        case 4: v.kind = 0; v.i = get<uint32_t>(); return true;
        case 5: v.kind = 0; v.i = get<int32_t>(); return true;
        case 6: v.kind = 1; v.f = get<float>(); return true;
        case 7: v.kind = 6; v.i = get<uint8_t>() != 0; return true;
        case 8: v.kind = 2; v.s = str(); return true;
        case 10: v.kind = 0; v.i = (int64_t)get<uint64_t>(); return true;
        case 11: v.kind = 0; v.i = get<int64_t>(); return true;
        case 12: v.kind = 1; v.f = get<double>(); return true;
        default: return false;
        }
    }
};

int fail(const char *fmt, const char *a, long long b = 0) {
    return gd_fail(nullptr, GD_EINVAL, fmt, a, b);
}

}  // namespace

extern "C" void gd_gguf_close(gd_gguf *g) {
    if (!g) return;
    if (g->map) munmap(const_cast<uint8_t *>(g->map), g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

extern "C" int gd_gguf_open(const char *path, gd_gguf **out) {
    if (!path || !out) return gd_fail(nullptr, GD_EINVAL, "gd_gguf_open: null argument");
    *out = nullptr;
    gd_gguf *g = new gd_gguf();
    g->fd = open(path, O_RDONLY);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || st.st_size <= 0) {
        gd_gguf_close(g);
        return fail("gd_gguf_open: cannot open %s", path);
    }
    g->size = (size_t)st.st_size;
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        gd_gguf_close(g);
        return fail("gd_gguf_open: cannot map %s", path);
    }
    g->map = (const uint8_t *)m;
    Cursor c{g->map, g->size};
    if (c.get<uint32_t>() != 0x46554747u) {                      // "GGUF"
        gd_gguf_close(g);
        return fail("gd_gguf_open: %s is not a GGUF file (bad magic)", path);
    }
    g->version = (int)c.get<uint32_t>();
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    // Counts far beyond what the file could hold are corruption.
    // Version 1 stored 32-bit counts; 2 and 3 share this layout.
    if (c.bad || g->version < 2 || n_tensors > g->size / 24 || n_kv > g->size / 12) {
        gd_gguf_close(g);
        return fail("gd_gguf_open: %s: bad header (version %lld or counts)", path,
                    (long long)g->version);
    }
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < n_kv && !c.bad; i++) {
        std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        GgufValue v;
        if (t == 9) {                                            // array
            const uint32_t et = c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            // Each element takes at least its scalar's bytes (a string its
            // length): a count the rest of the file cannot hold is corruption,
            // caught before any element is stored.
            const uint64_t least = et <= 1 || et == 7 ? 1 : et <= 3 ? 2 : et <= 6 ? 4 : 8;
            if (c.bad || n > (g->size - c.pos) / least) { c.bad = true; break; }
            // Bool elements read as 0/1 integers (GGUF.swift:263-275).
            v.kind = et == 8 ? 5 : (et == 6 || et == 12) ? 4 : 3;
            for (uint64_t k = 0; k < n && !c.bad; k++) {
                GgufValue e;
                if (!c.scalar(et, e)) { c.bad = true; break; }
                if (v.kind == 5) v.sa.push_back(e.s);
                else if (v.kind == 4) v.fa.push_back(e.f);
                else v.ia.push_back(e.i);
            }
        } else if (!c.scalar(t, v)) {
            gd_gguf_close(g);
            return fail("gd_gguf_open: metadata key %s has unknown type %lld", key.c_str(), t);
        }
        if (key == "general.alignment" && v.kind == 0 && v.i > 0) alignment = (uint64_t)v.i;
        g->meta[key] = std::move(v);
    }
    struct Raw { std::string name; GgufTensor t; uint64_t off; };
    std::vector<Raw> raws;
    for (uint64_t i = 0; i < n_tensors && !c.bad; i++) {
        Raw r;
        r.name = c.str();
        r.t.ndim = (int)c.get<uint32_t>();
        if (r.t.ndim < 1 || r.t.ndim > 4) { c.bad = true; break; }
        for (int d = 0; d < r.t.ndim; d++) r.t.dims[d] = (int64_t)c.get<uint64_t>();
        r.t.type = (int)c.get<uint32_t>();
        r.off = c.get<uint64_t>();
        raws.push_back(std::move(r));
    }
    if (c.bad) {
        gd_gguf_close(g);
        return fail("gd_gguf_open: %s is truncated or corrupt", path);
    }
    const uint64_t start = (c.pos + alignment - 1) / alignment * alignment;
    for (Raw &r : raws) {
        int64_t n = 1;
        for (int d = 0; d < r.t.ndim; d++) {
            if (r.t.dims[d] <= 0 || n > (int64_t)(g->size * 8) / r.t.dims[d]) { n = -1; break; }
            n *= r.t.dims[d];
        }
        r.t.bytes = n > 0 ? type_bytes(r.t.type, n) : 0;
        if (r.t.bytes == 0) {
            gd_gguf_close(g);
            return fail("gd_gguf_open: tensor %s has an unsupported type or shape (type %lld)",
                        r.name.c_str(), r.t.type);
        }
        if (r.off > g->size || start > g->size - r.off || r.t.bytes > g->size - start - r.off) {
            gd_gguf_close(g);
            return fail("gd_gguf_open: tensor %s lies past the end of the file", r.name.c_str());
        }
        r.t.data = g->map + start + r.off;
        g->tensors[r.name] = r.t;
    }
    *out = g;
    return GD_OK;
}

extern "C" int gd_gguf_info(const gd_gguf *g, int64_t *n_tensors, int64_t *n_kv, int *version) {
    if (!g) return GD_EINVAL;
    if (n_tensors) *n_tensors = (int64_t)g->tensors.size();
    if (n_kv) *n_kv = (int64_t)g->meta.size();
    if (version) *version = g->version;
    return GD_OK;
}

extern "C" int gd_gguf_tensor(const gd_gguf *g, const char *name, int *ndim, int64_t dims[4],
                              int *type, const void **data, size_t *bytes) {
    if (!g || !name) return GD_EINVAL;
    auto it = g->tensors.find(name);
    if (it == g->tensors.end()) return fail("gd_gguf_tensor: no tensor %s", name);
    const GgufTensor &t = it->second;
    if (ndim) *ndim = t.ndim;
    if (dims) for (int d = 0; d < 4; d++) dims[d] = t.dims[d];
    if (type) *type = t.type;
    if (data) *data = t.data;
    if (bytes) *bytes = t.bytes;
    return GD_OK;
}

extern "C" int gd_gguf_get_int(const gd_gguf *g, const char *key, int64_t *v) {
    if (!g || !key || !v) return GD_EINVAL;
    auto it = g->meta.find(key);
    if (it == g->meta.end() || it->second.kind != 0)
        return fail("gd_gguf_get_int: no integer key %s", key);
    *v = it->second.i;
    return GD_OK;
}

extern "C" int gd_gguf_get_float(const gd_gguf *g, const char *key, double *v) {
    if (!g || !key || !v) return GD_EINVAL;
    auto it = g->meta.find(key);
    if (it == g->meta.end() || (it->second.kind != 0 && it->second.kind != 1))
        return fail("gd_gguf_get_float: no numeric key %s", key);
    *v = it->second.kind == 1 ? it->second.f : (double)it->second.i;
    return GD_OK;
}

extern "C" int gd_gguf_get_bool(const gd_gguf *g, const char *key, int *v) {
    if (!g || !key || !v) return GD_EINVAL;
    auto it = g->meta.find(key);
    if (it == g->meta.end() || (it->second.kind != 6 && it->second.kind != 0))
        return fail("gd_gguf_get_bool: no bool or integer key %s", key);
    *v = it->second.i != 0;
    return GD_OK;
}

extern "C" int gd_gguf_get_string(const gd_gguf *g, const char *key, const char **v) {
    if (!g || !key || !v) return GD_EINVAL;
    auto it = g->meta.find(key);
    if (it == g->meta.end() || it->second.kind != 2)
        return fail("gd_gguf_get_string: no string key %s", key);
    *v = it->second.s.c_str();
    return GD_OK;
}

extern "C" int gd_gguf_get_ints(const gd_gguf *g, const char *key, const int64_t **v,
                                int64_t *n) {
    if (!g || !key || !v || !n) return GD_EINVAL;
    auto it = g->meta.find(key);
    if (it == g->meta.end() || it->second.kind != 3)
        return fail("gd_gguf_get_ints: no integer array key %s", key);
    *v = it->second.ia.data();
    *n = (int64_t)it->second.ia.size();
    return GD_OK;
}

// Geometry of a qwen35 hybrid from its metadata, with the keys and defaults
// of BonsaiConfig.init (Model.swift:39-69): <arch>.embedding_length,
// feed_forward_length, block_count, attention.head_count(_kv),
// attention.key_length, rope.dimension_count (default: key_length),
// rope.freq_base, attention.layer_norm_rms_epsilon,
// qwen35.full_attention_interval (default 4), ssm.state_size,
// ssm.group_count, ssm.time_step_rank, ssm.inner_size, ssm.conv_kernel; the
// vocabulary is token_embd.weight's second dimension.
// rope.dimension_sections is not read: a text-only sequence gives every
// section the same position, so the sectioned rotation equals the plain one.
extern "C" int gd_gguf_stack_config(const gd_gguf *g, gd_stack_config *cfg) {
    if (!g || !cfg) return gd_fail(nullptr, GD_EINVAL, "gd_gguf_stack_config: null argument");
    std::string arch = "qwen35";
    auto a = g->meta.find("general.architecture");
    if (a != g->meta.end() && a->second.kind == 2) arch = a->second.s;
    if (arch != "qwen35" && arch != "qwen3")
        return fail("gd_gguf_stack_config: architecture '%s' is neither the qwen35 GDN hybrid "
                    "nor the dense qwen3", arch.c_str());
    const bool dense = arch == "qwen3";
    auto get = [&](const char *key, bool required, double dflt, double *v) -> bool {
        auto it = g->meta.find(arch + "." + key);
        if (it == g->meta.end() || (it->second.kind != 0 && it->second.kind != 1)) {
            if (required) {
                fail("gd_gguf_stack_config: missing numeric key %s", (arch + "." + key).c_str());
                return false;
            }
            *v = dflt;
            return true;
        }
        *v = it->second.kind == 1 ? it->second.f : (double)it->second.i;
        return true;
    };
    double e, ff, nl, nh, nkv, hd, rot, base, eps;
    // The dense lineage has every layer attention and no ssm geometry
    // (Model.swift:55-59); the hybrid reads it.
    double ai = 1, ds = 0, nk = 0, nv = 0, inner = 0, dc = 0;
    if (!get("embedding_length", true, 0, &e) || !get("feed_forward_length", true, 0, &ff) ||
        !get("block_count", true, 0, &nl) || !get("attention.head_count", true, 0, &nh) ||
        !get("attention.head_count_kv", true, 0, &nkv) ||
        !get("attention.key_length", true, 0, &hd) ||
        !get("rope.dimension_count", false, hd, &rot) || !get("rope.freq_base", true, 0, &base) ||
        !get("attention.layer_norm_rms_epsilon", true, 0, &eps))
        return GD_EINVAL;
    if (!dense &&
        (!get("full_attention_interval", false, 4, &ai) || !get("ssm.state_size", true, 0, &ds) ||
         !get("ssm.group_count", true, 0, &nk) || !get("ssm.time_step_rank", true, 0, &nv) ||
         !get("ssm.inner_size", true, 0, &inner) || !get("ssm.conv_kernel", true, 0, &dc)))
        return GD_EINVAL;
    const double ints[] = {e, ff, nl, nh, nkv, hd, rot, ai, ds, nk, nv, inner, dc};
    for (int i = 0; i < (int)(sizeof ints / sizeof ints[0]); i++) {
        const double v = ints[i];
        const bool ssm = i >= 8;   // zero on the dense lineage
        if (!(v >= (dense && ssm ? 0 : 1) && v < (double)(1 << 30)) || v != (double)(int64_t)v)
            return fail("gd_gguf_stack_config: a geometry key holds %s, not a positive integer",
                        std::to_string(v).c_str());
    }
    auto t = g->tensors.find("token_embd.weight");
    if (t == g->tensors.end() || t->second.ndim != 2)
        return fail("gd_gguf_stack_config: no 2-D tensor token_embd.weight", "");
    if (inner != ds * nv)
        return fail("gd_gguf_stack_config: ssm.inner_size %s does not equal state_size x "
                    "time_step_rank (%lld)", std::to_string((long long)inner).c_str(),
                    (long long)(ds * nv));
    if (t->second.dims[0] != (int64_t)e)
        return fail("gd_gguf_stack_config: token_embd.weight width %s is not embedding_length",
                    std::to_string((long long)t->second.dims[0]).c_str());
    gd_stack_config c{};
    c.n_layer = (int)nl;
    c.n_embd = (int)e;
    c.n_ff = (int)ff;
    c.n_head = (int)nh;
    c.n_head_kv = (int)nkv;
    c.head_dim = (int)hd;
    c.n_rot = (int)rot;
    c.rope_base = (float)base;
    c.eps = (float)eps;
    c.n_vocab = (int)t->second.dims[1];
    c.attn_interval = (int)ai;
    c.d_state = (int)ds;
    c.n_k_head = (int)nk;
    c.n_v_head = (int)nv;
    c.d_conv = (int)dc;
    c.dense = dense ? 1 : 0;
    *cfg = c;
    return GD_OK;
}

extern "C" int gd_gguf_get_floats(const gd_gguf *g, const char *key, const double **v,
                                  int64_t *n) {
    if (!g || !key || !v || !n) return GD_EINVAL;
    auto it = g->meta.find(key);
    if (it == g->meta.end() || it->second.kind != 4)
        return fail("gd_gguf_get_floats: no float array key %s", key);
    *v = it->second.fa.data();
    *n = (int64_t)it->second.fa.size();
    return GD_OK;
}
