// Weight binding for the projections either side of the attention path: the attention geometry
// of a clef model (clef.c:27-59 load_config) and one layer's attention tensors (clef.c:180-256
// bind_weights), read from a GGUF v3 file (the container tools/convert.py writes) and copied to
// device buffers the caller owns.
//
// The file is mapped read-only and indexed once by clef_gguf_view::index_gguf (gguf_view.h),
// which checks every read against the mapping; every tensor's type and shape is then checked
// against what its consumer expects before any size derived from it is used.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <memory>
#include <string>
#include <vector>

#include "clef_hip_attn.h"
#include "gguf_view.h"

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

// A file mapping that unmaps itself.
struct Mapping {
    const uint8_t *bytes = nullptr;
    uint64_t size = 0;
    Mapping() = default;
    Mapping(const Mapping &) = delete;
    Mapping &operator=(const Mapping &) = delete;
    ~Mapping() {
        if (bytes) munmap((void *)bytes, (size_t)size);
    }
};

}  // namespace

struct clef_hip_gguf {
    Mapping map;
    clef_gguf_view::Index index;
    std::vector<clef_hip_gguf_tensor_info> infos;   // the ABI view of index.tensors
};

extern "C" {

bool clef_hip_gguf_open(const char *path, clef_hip_gguf **out, char *err, size_t errlen) {
    using namespace clef_gguf_view;
    if (!path || !out) return fail(err, errlen, "gguf: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(err, errlen, "gguf: cannot open %s", path);
    struct stat st;
    const bool sized = fstat(fd, &st) == 0;
    std::unique_ptr<clef_hip_gguf> g(new clef_hip_gguf());
    if (sized && st.st_size > 0) {
        void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_SHARED, fd, 0);
        if (m != MAP_FAILED) {
            g->map.bytes = (const uint8_t *)m;
            g->map.size = (uint64_t)st.st_size;
        }
    }
    close(fd);   // the mapping stays valid without the descriptor
    if (!sized) return fail(err, errlen, "gguf: cannot stat %s", path);
    if (st.st_size > 0 && !g->map.bytes) return fail(err, errlen, "gguf: cannot map %s", path);
    uint64_t where = 0;
    const Fault f = index_gguf(g->map.bytes, g->map.size, &g->index, &where);
    if (f == Fault::kMetadata || f == Fault::kTensorTable || f == Fault::kTensorData)
        return fail(err, errlen, "gguf: %s (entry %llu) in %s", fault_text(f), (unsigned long long)where, path);
    if (f != Fault::kNone) return fail(err, errlen, "gguf: %s: %s", fault_text(f), path);
    g->infos.resize(g->index.tensors.size());
    for (size_t i = 0; i < g->infos.size(); i++) {
        const TensorEntry &t = g->index.tensors[i];
        clef_hip_gguf_tensor_info &info = g->infos[i];
        memset(&info, 0, sizeof(info));
        info.n_dims = t.rank;
        info.type = t.ggml_type;
        for (int d = 0; d < 4; d++) info.ne[d] = t.extent[d];
        info.offset = t.file_offset;
        info.nbytes = t.bytes;
        info.data = g->map.bytes + t.file_offset;
    }
    *out = g.release();
    return true;
}

void clef_hip_gguf_close(clef_hip_gguf *g) { delete g; }

int clef_hip_gguf_tensor_count(const clef_hip_gguf *g) { return g ? (int)g->infos.size() : 0; }

bool clef_hip_gguf_tensor_at(const clef_hip_gguf *g, int i, clef_hip_gguf_tensor_info *info, char *name, size_t name_len) {
    if (!g || i < 0 || (size_t)i >= g->infos.size() || !info) return false;
    *info = g->infos[(size_t)i];
    if (name && name_len) snprintf(name, name_len, "%s", g->index.tensors[(size_t)i].name.c_str());
    return true;
}

bool clef_hip_gguf_find_tensor(const clef_hip_gguf *g, const char *name, clef_hip_gguf_tensor_info *info) {
    if (!g || !name || !info) return false;
    const int i = g->index.tensor_index(name);
    if (i < 0) return false;
    *info = g->infos[(size_t)i];
    return true;
}

bool clef_hip_gguf_get_u32(const clef_hip_gguf *g, const char *key, uint32_t *out) {
    return g && key && out && g->index.scalar(key, clef_gguf_view::kU32, out);
}

bool clef_hip_gguf_get_f32(const clef_hip_gguf *g, const char *key, float *out) {
    return g && key && out && g->index.scalar(key, clef_gguf_view::kF32, out);
}

bool clef_hip_gguf_attn_config(const clef_hip_gguf *g, clef_hip_attn_config *c, char *err, size_t errlen) {
    using namespace clef_gguf_view;
    if (!g || !c) return fail(err, errlen, "gguf: null argument");
    memset(c, 0, sizeof(*c));
    const MetaEntry *arch = g->index.lookup("general.architecture");
    if (!arch || arch->type != kString) return fail(err, errlen, "gguf: not a clef GGUF (no general.architecture)");
    {
        Cursor v(arch->value, arch->end);
        std::string_view name;
        if (!v.read_string(&name) || name != "clef") return fail(err, errlen, "gguf: not a clef GGUF (architecture is not clef)");
    }
    struct { const char *key; int *dst; } geometry[] = {
        {"clef.block_count", &c->n_layer}, {"clef.embedding_length", &c->H},
        {"clef.attention.head_count", &c->nh}, {"clef.attention.head_count_kv", &c->nkv},
        {"clef.attention.key_length", &c->hd}, {"clef.rope.dimension_count", &c->n_rot},
    };
    for (auto &e : geometry) {
        uint32_t v;
        if (!g->index.scalar(e.key, kU32, &v) || v == 0 || v > (1u << 24)) return fail(err, errlen, "gguf: missing or invalid %s", e.key);
        *e.dst = (int)v;
    }
    if (!g->index.scalar("clef.attention.layer_norm_rms_epsilon", kF32, &c->eps) ||
        !g->index.scalar("clef.rope.freq_base", kF32, &c->rope_theta))
        return fail(err, errlen, "gguf: missing rms eps / rope base");
    if (c->n_layer > CLEF_HIP_MAX_LAYERS) return fail(err, errlen, "gguf: %d layers, at most %d", c->n_layer, CLEF_HIP_MAX_LAYERS);
    const MetaEntry *lt = g->index.lookup("clef.layer_types");
    if (!lt || lt->type != kArray) return fail(err, errlen, "gguf: bad layer_types");
    Cursor v(lt->value, lt->end);
    uint32_t elem = 0;
    uint64_t count = 0;
    if (!v.read(&elem) || !v.read(&count) || (elem != kI32 && elem != kU32) || count != (uint64_t)c->n_layer)
        return fail(err, errlen, "gguf: bad layer_types");
    for (int i = 0; i < c->n_layer; i++) {
        int32_t t = -1;
        if (!v.read(&t) || (t != 0 && t != 1)) return fail(err, errlen, "gguf: layer %d has unknown type %d", i, t);
        c->layer_full[i] = t;
    }
    if (c->nh % c->nkv) return fail(err, errlen, "gguf: head_count %d is not a multiple of head_count_kv %d", c->nh, c->nkv);
    return true;
}

// One tensor with the exact type and shape its consumer expects (clef.c:180-193 bind): rank 1
// when ne1 is 1, else rank 2 with ne[0] the row length.
static bool bind(const clef_hip_gguf *g, const char *name, uint32_t type, uint64_t ne0, uint64_t ne1,
                 const clef_hip_gguf_tensor_info **out, char *err, size_t errlen) {
    const int i = g->index.tensor_index(name);
    if (i < 0) return fail(err, errlen, "gguf: missing tensor %s", name);
    const clef_hip_gguf_tensor_info &t = g->infos[(size_t)i];
    const uint32_t rank = ne1 == 1 ? 1 : 2;
    if (t.type != type || t.n_dims != rank || t.ne[0] != ne0 || t.ne[1] != ne1 || t.ne[2] != 1 || t.ne[3] != 1)
        return fail(err, errlen, "gguf: tensor %s has type %u rank %u shape [%llu, %llu], expected type %u [%llu, %llu]",
                    name, t.type, t.n_dims, (unsigned long long)t.ne[0], (unsigned long long)t.ne[1], type,
                    (unsigned long long)ne0, (unsigned long long)ne1);
    *out = &t;
    return true;
}

// Copies the four bound tensors into the caller's device buffers (NULL skips one) on `stream`
// and waits for the copies: their source is the file mapping, pageable memory that
// clef_hip_gguf_close unmaps, so no copy may still be reading it when this returns.
static bool upload(void *const dst[4], const clef_hip_gguf_tensor_info *const t[4], void *stream, const char *what,
                   int layer, char *err, size_t errlen) {
    bool any = false;
    for (int i = 0; i < 4; i++) {
        if (!dst[i]) continue;
        hipError_t e = hipMemcpyAsync(dst[i], t[i]->data, (size_t)t[i]->nbytes, hipMemcpyHostToDevice, (hipStream_t)stream);
        if (e != hipSuccess) return fail(err, errlen, "gguf: copy of %s %d tensor %d failed: %s", what, layer, i, hipGetErrorString(e));
        any = true;
    }
    if (any) {
        hipError_t e = hipStreamSynchronize((hipStream_t)stream);
        if (e != hipSuccess) return fail(err, errlen, "gguf: waiting for the %s %d copies failed: %s", what, layer, hipGetErrorString(e));
    }
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
    return upload(dst, t, stream, "layer", layer, err, errlen);
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
    return upload(dst, t, stream, "vision layer", layer, err, errlen);
}

}  // extern "C"
