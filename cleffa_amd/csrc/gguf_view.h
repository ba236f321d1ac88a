// A read-only index over a GGUF v3 file held in memory (host code, no HIP).
//
// The format (GGUF v3, little-endian):
//   header    magic "GGUF" (u32 0x46554747), version u32, tensor count u64, metadata count u64
//   metadata  per entry: key (u64 length + bytes), value type u32, value
//             value = fixed-width scalar | string (u64 length + bytes) |
//                     array (element type u32, count u64, elements)
//   tensors   per entry: name (string), rank u32, extents u64 x rank (fastest first),
//             element type u32, data offset u64 (relative to the data section)
//   data      starts at the end of the tensor table rounded up to the file's alignment
//             (metadata key general.alignment, u32, default 32)
//
// The file is untrusted. The index is built in one pass by `index_gguf`, which consumes the
// bytes through `Cursor`: every read is checked against what is left of the buffer, so no count
// or length from the file is trusted before the bytes it promises exist. Loops over counts stop
// at the first failed read, and every entry consumes at least 13 bytes, so a count larger than
// the file can hold fails as truncation without sizing anything by it.
//
// What is refused, and what is deliberately accepted (the acceptance rules of the reference's
// reader, clef_gguf.c:87-161, which the tests compare this index with):
//   - magic other than "GGUF", version other than 3, anything truncated;
//   - a string or array value nested inside more than two arrays (arrays of fixed-width
//     scalars are measured in one step, so only string / array elements count as nesting);
//     an empty array's element type is never looked at;
//   - a value type outside the 13 GGUF types;
//   - an alignment that is zero or not a power of two;
//   - a tensor of rank 0 or above 4, a zero extent, an element count or byte size that
//     overflows 64 bits, or an element type other than F32 / F16 / BF16;
//   - tensor data that does not lie inside the file. Data offsets are not required to be
//     aligned, and tensors may overlap: the reference accepts both.
// Lookups by key or name take the first entry of that key or name.
#pragma once
#include <stdint.h>
#include <string.h>

#include <string>
#include <string_view>
#include <vector>

namespace clef_gguf_view {

// GGUF metadata value types
enum ValueType : uint32_t {
    kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kString, kArray, kU64, kI64, kF64,
};
// bytes of a fixed-width value type, 0 for string / array / unknown
inline uint64_t fixed_width(uint32_t t) {
    static const uint8_t w[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    return t < 13 ? w[t] : 0;
}
// bytes per element of the tensor types the path takes (ggml type ids), 0 otherwise
inline uint64_t tensor_elem_bytes(uint32_t ggml_type) {
    switch (ggml_type) {
        case 0: return 4;    // F32
        case 1: return 2;    // F16
        case 30: return 2;   // BF16
        default: return 0;
    }
}

// Front-to-back consumer of a byte range. A failed read leaves the cursor where it was and
// returns false; callers stop at the first failure.
class Cursor {
   public:
    Cursor(const uint8_t *begin, const uint8_t *end) : at_(begin), end_(end) {}
    uint64_t remaining() const { return (uint64_t)(end_ - at_); }
    const uint8_t *here() const { return at_; }
    bool skip(uint64_t n) {
        if (n > remaining()) return false;
        at_ += n;
        return true;
    }
    template <typename T>
    bool read(T *v) {
        if (sizeof(T) > remaining()) return false;
        memcpy(v, at_, sizeof(T));
        at_ += sizeof(T);
        return true;
    }
    // a GGUF string: u64 length, then that many bytes
    bool read_string(std::string_view *s) {
        uint64_t n;
        const uint8_t *start = at_;
        if (!read(&n) || n > remaining()) { at_ = start; return false; }
        *s = std::string_view((const char *)at_, (size_t)n);
        at_ += n;
        return true;
    }

   private:
    const uint8_t *at_;
    const uint8_t *end_;
};

constexpr int kMaxArrayNesting = 2;

// Consumes one metadata value of type `type`. Arrays are walked with an explicit stack of
// (element type, elements left) frames rather than by recursion; a string or array value whose
// enclosing arrays number more than kMaxArrayNesting is refused.
inline bool consume_value(Cursor &c, uint32_t type) {
    struct Frame { uint32_t elem; uint64_t left; };
    Frame stack[kMaxArrayNesting + 1];
    int depth = 0;   // frames on the stack = arrays enclosing the value about to be read
    uint32_t t = type;
    for (;;) {
        if (depth > kMaxArrayNesting) return false;
        if (t == kString) {
            std::string_view s;
            if (!c.read_string(&s)) return false;
        } else if (t == kArray) {
            uint32_t elem;
            uint64_t count;
            if (!c.read(&elem) || !c.read(&count)) return false;
            if (const uint64_t w = fixed_width(elem)) {
                uint64_t bytes;
                if (__builtin_mul_overflow(count, w, &bytes) || !c.skip(bytes)) return false;
            } else if (count > 0) {
                stack[depth++] = Frame{elem, count};
            }
        } else {
            const uint64_t w = fixed_width(t);
            if (w == 0 || !c.skip(w)) return false;
        }
        // the next value: an element of the innermost array that has any left
        while (depth > 0 && stack[depth - 1].left == 0) depth--;
        if (depth == 0) return true;
        stack[depth - 1].left--;
        t = stack[depth - 1].elem;
    }
}

struct MetaEntry {
    std::string_view key;
    uint32_t type;
    const uint8_t *value;   // first byte of the value
    const uint8_t *end;     // one past its last byte
};

struct TensorEntry {
    std::string name;
    uint32_t rank;
    uint64_t extent[4];     // unused extents are 1
    uint32_t ggml_type;
    uint64_t rel_offset;    // from the file
    uint64_t file_offset;   // absolute, once the data section is known
    uint64_t bytes;
};

struct Index {
    std::vector<MetaEntry> meta;
    std::vector<TensorEntry> tensors;
    uint64_t data_start = 0;
    uint32_t alignment = 32;

    const MetaEntry *lookup(std::string_view key) const {
        for (const MetaEntry &m : meta)
            if (m.key == key) return &m;
        return nullptr;
    }
    int tensor_index(std::string_view name) const {
        for (size_t i = 0; i < tensors.size(); i++)
            if (tensors[i].name == name) return (int)i;
        return -1;
    }
    // a fixed-width scalar of exactly type `type`
    template <typename T>
    bool scalar(std::string_view key, uint32_t type, T *out) const {
        const MetaEntry *m = lookup(key);
        if (!m || m->type != type || (uint64_t)(m->end - m->value) != sizeof(T)) return false;
        memcpy(out, m->value, sizeof(T));
        return true;
    }
};

enum class Fault { kNone, kTooSmall, kMagic, kVersion, kMetadata, kAlignment, kTensorTable, kTensorData };

inline const char *fault_text(Fault f) {
    switch (f) {
        case Fault::kTooSmall: return "shorter than a GGUF header";
        case Fault::kMagic: return "not a GGUF file (magic)";
        case Fault::kVersion: return "GGUF version is not 3";
        case Fault::kMetadata: return "metadata section is malformed or truncated";
        case Fault::kAlignment: return "general.alignment is not a power of two";
        case Fault::kTensorTable: return "malformed tensor table entry";
        case Fault::kTensorData: return "tensor data lies outside the file";
        default: return "ok";
    }
}

// Builds the index of the `size` bytes at `file`. On a fault, *where is the index of the
// metadata or tensor entry it concerns (or 0).
inline Fault index_gguf(const uint8_t *file, uint64_t size, Index *ix, uint64_t *where) {
    *where = 0;
    if (size < 24) return Fault::kTooSmall;
    Cursor c(file, file + size);
    uint32_t magic = 0, version = 0;
    uint64_t n_tensors = 0, n_meta = 0;
    c.read(&magic);
    c.read(&version);
    c.read(&n_tensors);
    c.read(&n_meta);
    if (magic != 0x46554747u) return Fault::kMagic;
    if (version != 3) return Fault::kVersion;

    // Every metadata entry holds at least 13 bytes and every tensor entry 32: reservations are
    // capped by what the file could hold.
    ix->meta.reserve((size_t)(n_meta < size / 13 ? n_meta : size / 13));
    for (uint64_t i = 0; i < n_meta; i++) {
        MetaEntry m;
        if (!c.read_string(&m.key) || !c.read(&m.type)) { *where = i; return Fault::kMetadata; }
        m.value = c.here();
        if (!consume_value(c, m.type)) { *where = i; return Fault::kMetadata; }
        m.end = c.here();
        ix->meta.push_back(m);
    }
    if (const MetaEntry *a = ix->lookup("general.alignment"); a && a->type == kU32)
        memcpy(&ix->alignment, a->value, 4);
    if (ix->alignment == 0 || (ix->alignment & (ix->alignment - 1)) != 0) return Fault::kAlignment;

    ix->tensors.reserve((size_t)(n_tensors < size / 32 ? n_tensors : size / 32));
    for (uint64_t i = 0; i < n_tensors; i++) {
        *where = i;
        TensorEntry t;
        std::string_view name;
        if (!c.read_string(&name) || !c.read(&t.rank) || t.rank < 1 || t.rank > 4) return Fault::kTensorTable;
        uint64_t elems = 1;
        for (int d = 0; d < 4; d++) t.extent[d] = 1;
        for (uint32_t d = 0; d < t.rank; d++)
            if (!c.read(&t.extent[d]) || t.extent[d] == 0 || __builtin_mul_overflow(elems, t.extent[d], &elems))
                return Fault::kTensorTable;
        if (!c.read(&t.ggml_type) || !c.read(&t.rel_offset)) return Fault::kTensorTable;
        const uint64_t eb = tensor_elem_bytes(t.ggml_type);
        if (eb == 0 || __builtin_mul_overflow(elems, eb, &t.bytes)) return Fault::kTensorTable;
        t.name.assign(name.data(), name.size());
        ix->tensors.push_back(std::move(t));
    }
    *where = 0;

    const uint64_t table_end = (uint64_t)(c.here() - file);
    ix->data_start = (table_end + ix->alignment - 1) & ~(uint64_t)(ix->alignment - 1);
    for (size_t i = 0; i < ix->tensors.size(); i++) {
        TensorEntry &t = ix->tensors[i];
        // exact in 128 bits: data_start <= size, and the other two terms are 64-bit values
        const unsigned __int128 stop = (unsigned __int128)ix->data_start + t.rel_offset + t.bytes;
        if (stop > size) { *where = i; return Fault::kTensorData; }
        t.file_offset = ix->data_start + t.rel_offset;
    }
    return Fault::kNone;
}

}  // namespace clef_gguf_view
