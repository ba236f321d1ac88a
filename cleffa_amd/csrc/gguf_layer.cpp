// Weight binding for the projections either side of the attention path: a read-only GGUF v3
// view over an mmap'd file (the container format tools/convert.py writes, read by clef_gguf.c in
// the reference), the attention geometry of a clef model (clef.c:27-59) and the per-layer
// attention tensors (clef.c:180-256 bind_weights), copied to device buffers the caller owns.
//
// The file is untrusted input: every read is checked against the mapping, every count against
// what the file can hold, and every tensor's type and shape against what its consumer expects,
// before any size derived from it is used.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "clef_hip_attn.h"

namespace {

bool fail(char *err, size_t errlen, const char *fmt, ...) {
    if (err && errlen) {
        int n = snprintf(err, errlen, "hip: ");
        if (n < 0) n = 0;
        if ((size_t)n < errlen) {
            va_list ap;
            va_start(ap, fmt);
            vsnprintf(err + n, errlen - (size_t)n, fmt, ap);
            va_end(ap);
        }
    }
    return false;
}

// GGUF value types and the tensor element types the path takes.
enum : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

uint64_t scalar_bytes(uint32_t t) {
    switch (t) {
        case kU8: case kI8: case kBool: return 1;
        case kU16: case kI16: return 2;
        case kU32: case kI32: case kF32: return 4;
        case kU64: case kI64: case kF64: return 8;
        default: return 0;
    }
}

struct Reader {
    const uint8_t *base;
    uint64_t size, pos;
    bool ok;
    bool take(uint64_t n) {   // n more bytes exist at pos
        if (!ok || n > size || pos > size - n) ok = false;
        return ok;
    }
    uint32_t u32() {
        uint32_t v = 0;
        if (take(4)) { memcpy(&v, base + pos, 4); pos += 4; }
        return v;
    }
    uint64_t u64() {
        uint64_t v = 0;
        if (take(8)) { memcpy(&v, base + pos, 8); pos += 8; }
        return v;
    }
    // a string: its length, then its bytes; returns the byte offset of the bytes
    uint64_t str(uint64_t *len) {
        *len = u64();
        const uint64_t at = pos;
        if (take(*len)) pos += *len;
        else *len = 0;
        return at;
    }
    // steps over one value of type t (arrays nest at most two levels)
    void skip(uint32_t t, int depth) {
        if (depth > 2) { ok = false; return; }
        if (t == kString) { uint64_t n; str(&n); return; }
        if (t == kArray) {
            const uint32_t et = u32();
            const uint64_t n = u64();
            const uint64_t es = scalar_bytes(et);
            if (es) {
                if (n > size / es) { ok = false; return; }
                if (take(n * es)) pos += n * es;
                return;
            }
            for (uint64_t i = 0; i < n && ok; i++) skip(et, depth + 1);
            return;
        }
        const uint64_t s = scalar_bytes(t);
        if (!s) { ok = false; return; }
        if (take(s)) pos += s;
    }
};

struct Kv {
    uint64_t key, key_len;   // offset and length of the key bytes
    uint32_t type;
    uint64_t value;          // offset of the value
};

}  // namespace

struct clef_hip_gguf {
    int fd = -1;
    const uint8_t *base = nullptr;
    uint64_t size = 0, data_offset = 0;
    std::vector<Kv> kv;
    std::vector<clef_hip_gguf_tensor_info> tensors;
    std::vector<std::string> names;

    ~clef_hip_gguf() {
        if (base) munmap((void *)base, (size_t)size);
        if (fd >= 0) close(fd);
    }
    bool key_is(const Kv &k, const char *z) const {
        const size_t n = strlen(z);
        return k.key_len == n && !memcmp(base + k.key, z, n);
    }
    const Kv *find_kv(const char *key) const {
        for (const Kv &k : kv) if (key_is(k, key)) return &k;
        return nullptr;
    }
    int find_tensor(const char *name) const {
        for (size_t i = 0; i < names.size(); i++) if (names[i] == name) return (int)i;
        return -1;
    }
    bool get_u32(const char *key, uint32_t *out) const {
        const Kv *k = find_kv(key);
        if (!k || k->type != kU32) return false;
        Reader r{base, size, k->value, true};
        *out = r.u32();
        return r.ok;
    }
    bool get_f32(const char *key, float *out) const {
        const Kv *k = find_kv(key);
        if (!k || k->type != kF32) return false;
        Reader r{base, size, k->value, true};
        const uint32_t bits = r.u32();
        memcpy(out, &bits, 4);
        return r.ok;
    }
};

extern "C" {

bool clef_hip_gguf_open(const char *path, clef_hip_gguf **out, char *err, size_t errlen) {
    if (!path || !out) return fail(err, errlen, "gguf: null argument");
    *out = nullptr;
    clef_hip_gguf *g = new clef_hip_gguf();
    auto bad = [&](const char *msg) { delete g; return fail(err, errlen, "gguf: %s", msg); };
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) { delete g; return fail(err, errlen, "gguf: cannot open %s", path); }
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size < 24) return bad("file too small");
    g->size = (uint64_t)st.st_size;
    void *m = mmap(nullptr, (size_t)g->size, PROT_READ, MAP_SHARED, g->fd, 0);
    if (m == MAP_FAILED) return bad("mmap failed");
    g->base = (const uint8_t *)m;

    Reader r{g->base, g->size, 0, true};
    if (r.u32() != 0x46554747u) return bad("bad magic");   // "GGUF"
    if (r.u32() != 3) return bad("unsupported version (3 only)");
    const uint64_t n_tensors = r.u64(), n_kv = r.u64();
    // a record is at least 8 bytes on disk: counts the file cannot hold are refused before use
    if (!r.ok || n_kv > g->size / 8 || n_tensors > g->size / 8) return bad("bad header counts");
    uint32_t alignment = 32;
    g->kv.reserve((size_t)n_kv);
    for (uint64_t i = 0; i < n_kv && r.ok; i++) {
        Kv k;
        k.key = r.str(&k.key_len);
        k.type = r.u32();
        k.value = r.pos;
        if (r.ok && k.type == kU32 && g->key_is(k, "general.alignment")) {
            Reader a = r;
            alignment = a.u32();
        }
        r.skip(k.type, 0);
        g->kv.push_back(k);
    }
    if (!r.ok) return bad("truncated metadata");
    if (alignment == 0 || (alignment & (alignment - 1))) return bad("bad alignment");
    g->tensors.reserve((size_t)n_tensors);
    g->names.reserve((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors && r.ok; i++) {
        clef_hip_gguf_tensor_info t;
        memset(&t, 0, sizeof(t));
        uint64_t nlen;
        const uint64_t at = r.str(&nlen);
        t.n_dims = r.u32();
        if (!r.ok || t.n_dims == 0 || t.n_dims > 4) { r.ok = false; break; }
        uint64_t nelem = 1;
        for (int d = 0; d < 4; d++) t.ne[d] = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            t.ne[d] = r.u64();
            if (t.ne[d] == 0 || nelem > UINT64_MAX / t.ne[d]) { r.ok = false; break; }
            nelem *= t.ne[d];
        }
        t.type = r.u32();
        t.offset = r.u64();
        uint64_t es = 0;
        if (t.type == CLEF_HIP_GGML_F32) es = 4;
        else if (t.type == CLEF_HIP_GGML_F16 || t.type == CLEF_HIP_GGML_BF16) es = 2;
        if (!r.ok || !es || nelem > UINT64_MAX / es) { r.ok = false; break; }
        t.nbytes = nelem * es;
        g->tensors.push_back(t);
        g->names.emplace_back((const char *)g->base + at, (size_t)nlen);
    }
    if (!r.ok) return bad("bad tensor table");
    g->data_offset = (r.pos + alignment - 1) & ~(uint64_t)(alignment - 1);
    for (auto &t : g->tensors) {
        if (t.offset > g->size || g->data_offset > g->size - t.offset ||
            t.nbytes > g->size - g->data_offset - t.offset)
            return bad("tensor data out of bounds");
        t.offset += g->data_offset;
        t.data = g->base + t.offset;
    }
    *out = g;
    return true;
}

void clef_hip_gguf_close(clef_hip_gguf *g) { delete g; }

int clef_hip_gguf_tensor_count(const clef_hip_gguf *g) { return g ? (int)g->tensors.size() : 0; }

bool clef_hip_gguf_tensor_at(const clef_hip_gguf *g, int i, clef_hip_gguf_tensor_info *info, char *name, size_t name_len) {
    if (!g || i < 0 || (size_t)i >= g->tensors.size() || !info) return false;
    *info = g->tensors[(size_t)i];
    if (name && name_len) snprintf(name, name_len, "%s", g->names[(size_t)i].c_str());
    return true;
}

bool clef_hip_gguf_find_tensor(const clef_hip_gguf *g, const char *name, clef_hip_gguf_tensor_info *info) {
    if (!g || !name || !info) return false;
    const int i = g->find_tensor(name);
    if (i < 0) return false;
    *info = g->tensors[(size_t)i];
    return true;
}

bool clef_hip_gguf_get_u32(const clef_hip_gguf *g, const char *key, uint32_t *out) {
    return g && key && out && g->get_u32(key, out);
}

bool clef_hip_gguf_get_f32(const clef_hip_gguf *g, const char *key, float *out) {
    return g && key && out && g->get_f32(key, out);
}

bool clef_hip_gguf_attn_config(const clef_hip_gguf *g, clef_hip_attn_config *c, char *err, size_t errlen) {
    if (!g || !c) return fail(err, errlen, "gguf: null argument");
    memset(c, 0, sizeof(*c));
    const Kv *arch = g->find_kv("general.architecture");
    if (!arch || arch->type != kString) return fail(err, errlen, "gguf: not a clef GGUF (no general.architecture)");
    {
        Reader r{g->base, g->size, arch->value, true};
        uint64_t n;
        const uint64_t at = r.str(&n);
        if (!r.ok || n != 4 || memcmp(g->base + at, "clef", 4)) return fail(err, errlen, "gguf: not a clef GGUF");
    }
    struct { const char *key; int *dst; } u[] = {
        {"clef.block_count", &c->n_layer}, {"clef.embedding_length", &c->H},
        {"clef.attention.head_count", &c->nh}, {"clef.attention.head_count_kv", &c->nkv},
        {"clef.attention.key_length", &c->hd}, {"clef.rope.dimension_count", &c->n_rot},
    };
    for (auto &e : u) {
        uint32_t v;
        if (!g->get_u32(e.key, &v) || v == 0 || v > (1u << 24)) return fail(err, errlen, "gguf: missing or invalid %s", e.key);
        *e.dst = (int)v;
    }
    if (!g->get_f32("clef.attention.layer_norm_rms_epsilon", &c->eps) || !g->get_f32("clef.rope.freq_base", &c->rope_theta))
        return fail(err, errlen, "gguf: missing rms eps / rope base");
    if (c->n_layer > CLEF_HIP_MAX_LAYERS) return fail(err, errlen, "gguf: %d layers, at most %d", c->n_layer, CLEF_HIP_MAX_LAYERS);
    const Kv *lt = g->find_kv("clef.layer_types");
    if (!lt || lt->type != kArray) return fail(err, errlen, "gguf: bad layer_types");
    Reader r{g->base, g->size, lt->value, true};
    const uint32_t et = r.u32();
    const uint64_t n = r.u64();
    if (!r.ok || (et != kI32 && et != kU32) || n != (uint64_t)c->n_layer) return fail(err, errlen, "gguf: bad layer_types");
    for (int i = 0; i < c->n_layer; i++) {
        const int32_t v = (int32_t)r.u32();
        if (!r.ok || (v != 0 && v != 1)) return fail(err, errlen, "gguf: layer %d has unknown type %d", i, v);
        c->layer_full[i] = v;
    }
    if (c->nh % c->nkv) return fail(err, errlen, "gguf: head_count %d is not a multiple of head_count_kv %d", c->nh, c->nkv);
    return true;
}

// One tensor with the exact type and shape its consumer expects (clef.c:180-193 bind): rank 1
// when ne1 is 1, else rank 2 with ne[0] the row length.
static bool bind(const clef_hip_gguf *g, const char *name, uint32_t type, uint64_t ne0, uint64_t ne1,
                 const clef_hip_gguf_tensor_info **out, char *err, size_t errlen) {
    const int i = g->find_tensor(name);
    if (i < 0) return fail(err, errlen, "gguf: missing tensor %s", name);
    const clef_hip_gguf_tensor_info &t = g->tensors[(size_t)i];
    const uint32_t rank = ne1 == 1 ? 1 : 2;
    if (t.type != type || t.n_dims != rank || t.ne[0] != ne0 || t.ne[1] != ne1 || t.ne[2] != 1 || t.ne[3] != 1)
        return fail(err, errlen, "gguf: tensor %s has type %u rank %u shape [%llu, %llu], expected type %u [%llu, %llu]",
                    name, t.type, t.n_dims, (unsigned long long)t.ne[0], (unsigned long long)t.ne[1], type,
                    (unsigned long long)ne0, (unsigned long long)ne1);
    *out = &t;
    return true;
}

bool clef_hip_gguf_attn_layer(const clef_hip_gguf *g, const clef_hip_attn_config *c, int layer, uint16_t *w_qkv,
                              uint16_t *w_o, float *q_norm, float *k_norm, void *stream, char *err, size_t errlen) {
    if (!g || !c) return fail(err, errlen, "gguf: null argument");
    if (layer < 0 || layer >= c->n_layer) return fail(err, errlen, "gguf: layer %d out of range (%d layers)", layer, c->n_layer);
    if (!c->layer_full[layer]) return fail(err, errlen, "gguf: layer %d is not a full-attention layer", layer);
    const uint64_t n_attn = 2ull * c->nh * c->hd + 2ull * c->nkv * c->hd;   // [q | gate] per head, K, V
    char name[96];
    const clef_hip_gguf_tensor_info *t[4];
    snprintf(name, sizeof(name), "blk.%d.attn_qkv.weight", layer);
    if (!bind(g, name, CLEF_HIP_GGML_BF16, (uint64_t)c->H, n_attn, &t[0], err, errlen)) return false;
    snprintf(name, sizeof(name), "blk.%d.attn_output.weight", layer);
    if (!bind(g, name, CLEF_HIP_GGML_BF16, (uint64_t)c->nh * c->hd, (uint64_t)c->H, &t[1], err, errlen)) return false;
    snprintf(name, sizeof(name), "blk.%d.attn_q_norm.weight", layer);
    if (!bind(g, name, CLEF_HIP_GGML_F32, (uint64_t)c->hd, 1, &t[2], err, errlen)) return false;
    snprintf(name, sizeof(name), "blk.%d.attn_k_norm.weight", layer);
    if (!bind(g, name, CLEF_HIP_GGML_F32, (uint64_t)c->hd, 1, &t[3], err, errlen)) return false;
    void *dst[4] = {w_qkv, w_o, q_norm, k_norm};
    for (int i = 0; i < 4; i++) {
        if (!dst[i]) continue;   // NULL: that tensor is not wanted
        hipError_t e = hipMemcpyAsync(dst[i], t[i]->data, (size_t)t[i]->nbytes, hipMemcpyHostToDevice, (hipStream_t)stream);
        if (e != hipSuccess) return fail(err, errlen, "gguf: copy of layer %d tensor %d failed: %s", layer, i, hipGetErrorString(e));
    }
    return true;
}

bool clef_hip_gguf_vis_layer(const clef_hip_gguf *g, int layer, int heads, uint16_t *w_qkv, float *b_qkv,
                             uint16_t *w_o, float *b_o, void *stream, char *err, size_t errlen) {
    if (!g || layer < 0 || heads <= 0) return fail(err, errlen, "gguf: bad vision layer arguments");
    const uint64_t E = 72ull * heads;
    char name[96];
    const clef_hip_gguf_tensor_info *t[4];
    snprintf(name, sizeof(name), "v.blk.%d.attn_qkv.weight", layer);
    if (!bind(g, name, CLEF_HIP_GGML_BF16, E, 3 * E, &t[0], err, errlen)) return false;
    snprintf(name, sizeof(name), "v.blk.%d.attn_qkv.bias", layer);
    if (!bind(g, name, CLEF_HIP_GGML_F32, 3 * E, 1, &t[1], err, errlen)) return false;
    snprintf(name, sizeof(name), "v.blk.%d.attn_out.weight", layer);
    if (!bind(g, name, CLEF_HIP_GGML_BF16, E, E, &t[2], err, errlen)) return false;
    snprintf(name, sizeof(name), "v.blk.%d.attn_out.bias", layer);
    if (!bind(g, name, CLEF_HIP_GGML_F32, E, 1, &t[3], err, errlen)) return false;
    void *dst[4] = {w_qkv, b_qkv, w_o, b_o};
    for (int i = 0; i < 4; i++) {
        if (!dst[i]) continue;
        hipError_t e = hipMemcpyAsync(dst[i], t[i]->data, (size_t)t[i]->nbytes, hipMemcpyHostToDevice, (hipStream_t)stream);
        if (e != hipSuccess) return fail(err, errlen, "gguf: copy of vision layer %d tensor %d failed: %s", layer, i, hipGetErrorString(e));
    }
    return true;
}

}  // extern "C"
