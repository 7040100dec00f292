// GGUF v3 reader behind the C ABI: GGUFReader::open / tensor_by_name /
// read_tensor_data (src/gguf.rs:321-514), the tensor-type table and
// TensorInfo::n_bytes (src/gguf.rs:46-201), the metadata keys the models use
// (populate_metadata, src/gguf.rs:517-637), and the raw device upload of
// Model::upload_tensor_quantized (src/model.rs:174-184).
//
// Host code only.  The file is parsed once at open; tensor bytes are read on
// demand with pread, so one reader can serve many uploads, and a device upload
// streams through a pinned staging buffer without holding the tensor in host memory.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "lg_common.hpp"

namespace {

using namespace lg;

// ---- tensor types: the reference's table (src/gguf.rs:46-141), including its
// entries for formats this library does not compute with.  Ids with no entry
// (31-33, 36-38, > 41) are rejected, as TensorType::from_u32 panics on them.
struct TypeRow {
    uint32_t block_bytes, block_elems;
    bool quantized;
};

bool type_row(uint32_t id, TypeRow &r) {
    switch (id) {
    case 0: r = {4, 1, false}; return true;       // F32
    case 1: r = {2, 1, false}; return true;       // F16
    case 2: case 3: r = {1536, 16, true}; return true;  // Q4_0, Q4_1 (as the reference tabulates them)
    case 4: r = {264, 32, true}; return true;     // Q5_0
    case 5: r = {24, 32, true}; return true;      // Q5_1
    case 6: case 10: r = {16, 256, true}; return true;   // Q2_K (10 decodes as Q2_K)
    case 7: case 11: r = {112, 256, true}; return true;  // Q3_K (11 decodes as Q3_K)
    case 8: r = {34, 32, true}; return true;      // Q8_0
    case 9: r = {35, 32, true}; return true;      // Q8_1
    case 12: r = {144, 256, true}; return true;   // Q4_K
    case 13: r = {162, 256, true}; return true;   // Q5_K
    case 14: r = {210, 256, true}; return true;   // Q6_K
    case 15: r = {144, 256, true}; return true;   // Q8_K
    case 16: case 18: case 21: case 23: r = {16, 256, false}; return true;  // IQ2_XXS, IQ3_XXS, IQ3_S, IQ4_XS
    case 17: case 22: r = {256, 256, false}; return true;                   // IQ2_XS, IQ2_S
    case 19: r = {32, 256, false}; return true;   // IQ1_S
    case 20: r = {16, 256, false}; return true;   // IQ4_NL
    case 24: r = {1, 1, false}; return true;      // I8
    case 25: r = {2, 1, false}; return true;      // I16
    case 26: r = {4, 1, false}; return true;      // I32
    case 27: r = {8, 1, false}; return true;      // I64
    case 28: r = {8, 1, false}; return true;      // F64
    case 29: r = {512, 256, false}; return true;  // IQ1_M
    case 30: r = {2, 1, false}; return true;      // BF16
    case 34: r = {256, 256, false}; return true;  // TQ1_0
    case 35: r = {34, 256, false}; return true;   // TQ2_0
    case 39: case 40: r = {832, 256, false}; return true;  // MXFP4, NVFP4
    case 41: r = {256, 256, false}; return true;  // Q1_0
    default: return false;
    }
}

// TensorInfo::n_bytes (src/gguf.rs:182-201): whole blocks, rounding up.
uint64_t tensor_n_bytes(const TypeRow &r, uint64_t n_elements) {
    const uint64_t blocks = (n_elements + r.block_elems - 1) / r.block_elems;
    return blocks * r.block_bytes;
}

// ---- metadata values (GGUFValue, src/gguf.rs:203-230)
enum : uint32_t {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STR = 8, V_ARR = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12
};

struct Value {
    uint32_t type = 0;
    uint64_t u = 0;  // every integer and bool, as its two's-complement bits
    double f = 0.0;  // F32 / F64
    std::string s;
    std::vector<Value> arr;
};

// GGUFValue::as_u64 (src/gguf.rs:239-247): U32, U64, I32, I64 (negative values wrap).
bool as_u64(const Value &v, uint64_t &out) {
    switch (v.type) {
    case V_U32: case V_U64: case V_I32: case V_I64: out = v.u; return true;
    default: return false;
    }
}

// GGUFValue::as_f32 (src/gguf.rs:249-259).
bool as_f32(const Value &v, float &out) {
    switch (v.type) {
    case V_F32: case V_F64: out = (float)v.f; return true;
    case V_U32: case V_U64: out = (float)v.u; return true;
    case V_I32: case V_I64: out = (float)(int64_t)v.u; return true;
    default: return false;
    }
}

// GGUFValue::as_bool (src/gguf.rs:261-272).
bool as_bool(const Value &v, bool &out) {
    switch (v.type) {
    case V_BOOL: case V_U32: case V_U64: case V_I32: case V_I64: out = v.u != 0; return true;
    case V_F32: case V_F64: out = v.f != 0.0; return true;
    default: return false;
    }
}

// ---- a bounds-checked cursor over the header bytes
struct Cursor {
    int fd;
    uint64_t pos = 0, size = 0;
    std::vector<uint8_t> buf;  // read-ahead window
    uint64_t buf_pos = 0;

    bool fill(uint64_t need) {
        if (pos + need > size) return false;
        if (pos >= buf_pos && pos + need <= buf_pos + buf.size()) return true;
        const uint64_t want = need > (1u << 20) ? need : (1u << 20);
        const uint64_t len = size - pos < want ? size - pos : want;
        buf.resize(len);
        uint64_t got = 0;
        while (got < len) {
            const ssize_t r = pread(fd, buf.data() + got, len - got, (off_t)(pos + got));
            if (r <= 0) return false;
            got += (uint64_t)r;
        }
        buf_pos = pos;
        return true;
    }
    bool bytes(void *dst, uint64_t n) {
        if (n == 0) return true;
        if (!fill(n)) return false;
        std::memcpy(dst, buf.data() + (pos - buf_pos), n);
        pos += n;
        return true;
    }
    template <typename T>
    bool get(T &v) {  // little-endian host (x86-64)
        return bytes(&v, sizeof v);
    }
    bool str(std::string &s) {
        uint64_t len = 0;
        if (!get(len) || len > size - pos) return false;
        s.resize(len);
        return bytes(&s[0], len);
    }
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> shape;
    uint32_t dtype;
    uint64_t data_offset, n_elements, n_bytes;
};

}  // namespace

struct lg_gguf {
    int fd = -1;
    std::string path;
    uint32_t version = 0;
    uint64_t tensor_count = 0, field_count = 0, data_offset = 0, file_size = 0;
    std::vector<std::pair<std::string, Value>> fields;
    std::unordered_map<std::string, size_t> field_index;  // first occurrence
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> tensor_index;  // first occurrence (tensor_by_name)
    lg_gguf_meta meta;
};

namespace {

constexpr int MAX_DEPTH = 4;

bool read_value(Cursor &c, uint32_t type, Value &v, int depth) {
    v.type = type;
    switch (type) {
    case V_U8: case V_I8: case V_BOOL: {
        uint8_t b;
        if (!c.get(b)) return false;
        v.u = type == V_I8 ? (uint64_t)(int64_t)(int8_t)b : b;
        if (type == V_BOOL) v.u = b != 0;
        return true;
    }
    case V_U16: case V_I16: {
        uint16_t h;
        if (!c.get(h)) return false;
        v.u = type == V_I16 ? (uint64_t)(int64_t)(int16_t)h : h;
        return true;
    }
    case V_U32: case V_I32: {
        uint32_t w;
        if (!c.get(w)) return false;
        v.u = type == V_I32 ? (uint64_t)(int64_t)(int32_t)w : w;
        return true;
    }
    case V_F32: {
        float f;
        if (!c.get(f)) return false;
        v.f = f;
        return true;
    }
    case V_U64: case V_I64: return c.get(v.u);
    case V_F64: return c.get(v.f);
    case V_STR: return c.str(v.s);
    case V_ARR: {
        uint32_t et;
        uint64_t n;
        if (depth >= MAX_DEPTH || !c.get(et) || !c.get(n)) return false;
        if (n > c.size - c.pos) return false;  // every element takes at least one byte
        v.arr.resize(n);
        for (uint64_t i = 0; i < n; i++)
            if (!read_value(c, et, v.arr[i], depth + 1)) return false;
        return true;
    }
    default: return false;
    }
}

void copy_str(char *dst, size_t cap, const std::string &s) {
    const size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
    std::memcpy(dst, s.data(), n);
    dst[n] = '\0';
}

bool key_is(const std::string &k, std::initializer_list<const char *> names) {
    for (const char *n : names)
        if (k == n) return true;
    return false;
}

// populate_metadata (src/gguf.rs:517-637) for the fields the models read; later
// occurrences of a key overwrite earlier ones, as there.
void populate(lg_gguf_meta &m, const std::string &k, const Value &v) {
    uint64_t u;
    float f;
    bool b;
    auto set_u = [&](uint64_t &dst, uint32_t bit) {
        if (as_u64(v, u)) dst = u, m.present |= bit;
        else m.present &= ~bit;
    };
    auto set_f = [&](float &dst, uint32_t bit) {
        if (as_f32(v, f)) dst = f, m.present |= bit;
        else m.present &= ~bit;
    };
    auto set_s = [&](char *dst, size_t cap, uint32_t bit) {
        if (v.type == V_STR) copy_str(dst, cap, v.s), m.present |= bit;
        else m.present &= ~bit;
    };
    if (k == "general.architecture") set_s(m.architecture, sizeof m.architecture, LG_GGUF_HAS_ARCHITECTURE);
    else if (k == "general.name") set_s(m.general_name, sizeof m.general_name, LG_GGUF_HAS_GENERAL_NAME);
    else if (k == "general.file_type") set_u(m.file_type, LG_GGUF_HAS_FILE_TYPE);
    else if (k == "general.alignment") set_u(m.alignment, LG_GGUF_HAS_ALIGNMENT);
    else if (key_is(k, {"laguna.block_count", "dflash.block_count", "block_count"}))
        set_u(m.block_count, LG_GGUF_HAS_BLOCK_COUNT);
    else if (key_is(k, {"laguna.context_length", "dflash.context_length", "context_length"}))
        set_u(m.context_length, LG_GGUF_HAS_CONTEXT_LENGTH);
    else if (key_is(k, {"laguna.embedding_length", "dflash.embedding_length", "embedding_length"}))
        set_u(m.embedding_length, LG_GGUF_HAS_EMBEDDING_LENGTH);
    else if (key_is(k, {"laguna.feed_forward_length", "dflash.feed_forward_length", "feed_forward_length"}))
        set_u(m.feed_forward_length, LG_GGUF_HAS_FEED_FORWARD_LENGTH);
    else if (key_is(k, {"laguna.attention.head_count", "dflash.attention.head_count", "attention.head_count"})) {
        // an array gives its first entry (a missing or non-integer entry leaves the field unset)
        const Value *e = v.type == V_ARR ? (v.arr.empty() ? nullptr : &v.arr[0]) : &v;
        if (v.type == V_ARR && !e) return;  // empty array: the reference leaves the field as it was
        if (e && as_u64(*e, u)) m.head_count = u, m.present |= LG_GGUF_HAS_HEAD_COUNT;
        else m.present &= ~LG_GGUF_HAS_HEAD_COUNT;
    } else if (key_is(k, {"laguna.attention.head_count_kv", "dflash.attention.head_count_kv",
                          "attention.head_count_kv"})) {
        // an array gives its SECOND entry (src/gguf.rs:543-550), when it has one
        if (v.type == V_ARR) {
            if (v.arr.size() <= 1) return;
            if (as_u64(v.arr[1], u)) m.head_count_kv = u, m.present |= LG_GGUF_HAS_HEAD_COUNT_KV;
            else m.present &= ~LG_GGUF_HAS_HEAD_COUNT_KV;
        } else {
            set_u(m.head_count_kv, LG_GGUF_HAS_HEAD_COUNT_KV);
        }
    } else if (key_is(k, {"laguna.attention.key_length", "dflash.attention.key_length"}))
        set_u(m.key_length, LG_GGUF_HAS_KEY_LENGTH);
    else if (key_is(k, {"laguna.attention.value_length", "dflash.attention.value_length"}))
        set_u(m.value_length, LG_GGUF_HAS_VALUE_LENGTH);
    else if (key_is(k, {"laguna.attention.layer_norm_rms_epsilon", "dflash.attention.layer_norm_rms_epsilon"}))
        set_f(m.rms_epsilon, LG_GGUF_HAS_RMS_EPSILON);
    else if (key_is(k, {"laguna.rope.freq_base", "dflash.rope.freq_base", "rope.freq_base"}))
        set_f(m.rope_freq_base, LG_GGUF_HAS_ROPE_FREQ_BASE);
    else if (key_is(k, {"laguna.rope.dimension_count", "dflash.rope.dimension_count", "rope.dimension_count"}))
        set_u(m.rope_dimension_count, LG_GGUF_HAS_ROPE_DIMENSION_COUNT);
    else if (key_is(k, {"expert.count", "expert_count"}))
        set_u(m.expert_count, LG_GGUF_HAS_EXPERT_COUNT);
    else if (key_is(k, {"expert.used_count", "expert_used_count"}))
        set_u(m.expert_used_count, LG_GGUF_HAS_EXPERT_USED_COUNT);
    else if (key_is(k, {"vocab_size", "general.vocab_size"}))
        set_u(m.vocab_size, LG_GGUF_HAS_VOCAB_SIZE);
    else if (key_is(k, {"dflash.target_layers", "laguna.target_layers", "target_layers"})) {
        if (v.type != V_ARR) return;
        // non-integer entries are skipped (filter_map, src/gguf.rs:621-624)
        uint32_t n = 0;
        for (const Value &e : v.arr)
            if (as_u64(e, u) && n < LG_GGUF_MAX_TARGET_LAYERS) m.target_layers[n++] = (int64_t)u;
        m.n_target_layers = n;
        m.present |= LG_GGUF_HAS_TARGET_LAYERS;
    } else if (key_is(k, {"dflash.decoder_arch", "decoder_arch"}))
        set_s(m.decoder_arch, sizeof m.decoder_arch, LG_GGUF_HAS_DECODER_ARCH);
    else if (key_is(k, {"laguna.expert_weights_norm", "dflash.expert_weights_norm", "expert_weights_norm"})) {
        if (as_bool(v, b)) m.expert_weights_norm = b, m.present |= LG_GGUF_HAS_EXPERT_WEIGHTS_NORM;
        else m.present &= ~LG_GGUF_HAS_EXPERT_WEIGHTS_NORM;
    }
    // an integer array under general.*.rope_dimension_count sets the rope dimension
    // from its first entry (src/gguf.rs:629-637)
    const size_t suf = sizeof(".rope_dimension_count") - 1;
    if (v.type == V_ARR && !v.arr.empty() && as_u64(v.arr[0], u) && k.size() >= suf &&
        k.compare(k.size() - suf, suf, ".rope_dimension_count") == 0 && k.find("general.") != std::string::npos) {
        m.rope_dimension_count = u;
        m.present |= LG_GGUF_HAS_ROPE_DIMENSION_COUNT;
    }
}

int open_file(const char *path, lg_gguf *g) {
    g->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) return fail(LG_EIO, "gguf: cannot open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(g->fd, &st) != 0) return fail(LG_EIO, "gguf: cannot stat %s: %s", path, strerror(errno));
    g->file_size = (uint64_t)st.st_size;
    Cursor c{g->fd};
    c.size = g->file_size;
    char magic[4];
    if (!c.bytes(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return fail(LG_EIO, "gguf: %s: not a GGUF file", path);
    if (!c.get(g->version)) return fail(LG_EIO, "gguf: %s: truncated header", path);
    if (g->version != 3) return fail(LG_EIO, "gguf: %s: only GGUF v3 is supported (found v%u)", path, g->version);
    if (!c.get(g->tensor_count) || !c.get(g->field_count)) return fail(LG_EIO, "gguf: %s: truncated header", path);
    // each field and tensor entry takes more than 8 bytes: counts beyond the file are corrupt
    if (g->field_count > g->file_size / 8 || g->tensor_count > g->file_size / 8)
        return fail(LG_EIO, "gguf: %s: implausible counts (%llu fields, %llu tensors)", path,
                    (unsigned long long)g->field_count, (unsigned long long)g->tensor_count);
    g->fields.reserve(g->field_count);
    for (uint64_t i = 0; i < g->field_count; i++) {
        std::string key;
        uint32_t type;
        Value v;
        if (!c.str(key) || !c.get(type)) return fail(LG_EIO, "gguf: %s: truncated metadata (field %llu)", path, (unsigned long long)i);
        if (!read_value(c, type, v, 0))
            return fail(LG_EIO, "gguf: %s: bad or truncated value of '%s' (type %u)", path, key.c_str(), type);
        populate(g->meta, key, v);
        g->field_index.emplace(key, g->fields.size());
        g->fields.emplace_back(std::move(key), std::move(v));
    }
    uint64_t align = (g->meta.present & LG_GGUF_HAS_ALIGNMENT) ? g->meta.alignment : 32;
    if (align == 0) align = 1;
    g->tensors.reserve(g->tensor_count);
    for (uint64_t i = 0; i < g->tensor_count; i++) {
        Tensor t;
        uint32_t nd;
        if (!c.str(t.name) || !c.get(nd)) return fail(LG_EIO, "gguf: %s: truncated tensor info %llu", path, (unsigned long long)i);
        if (nd > LG_GGUF_MAX_DIMS) return fail(LG_EIO, "gguf: %s: tensor '%s' has %u dims (at most %d)", path, t.name.c_str(), nd, LG_GGUF_MAX_DIMS);
        t.shape.resize(nd);
        t.n_elements = 1;
        for (uint32_t d = 0; d < nd; d++) {
            if (!c.get(t.shape[d])) return fail(LG_EIO, "gguf: %s: truncated tensor info '%s'", path, t.name.c_str());
            t.n_elements *= t.shape[d];
        }
        if (!c.get(t.dtype) || !c.get(t.data_offset)) return fail(LG_EIO, "gguf: %s: truncated tensor info '%s'", path, t.name.c_str());
        TypeRow r;
        if (!type_row(t.dtype, r)) return fail(LG_EIO, "gguf: %s: tensor '%s' has unknown type %u", path, t.name.c_str(), t.dtype);
        t.n_bytes = tensor_n_bytes(r, t.n_elements);
        g->tensor_index.emplace(t.name, g->tensors.size());
        g->tensors.push_back(std::move(t));
    }
    // the data section starts at the next multiple of the alignment (src/gguf.rs:384-388)
    g->data_offset = (c.pos + align - 1) & ~(align - 1);
    return LG_OK;
}

// Field `field`'s value, or element `elem` of an array value (elem = UINT64_MAX:
// the value itself).
int field_elem(const lg_gguf *g, uint64_t field, uint64_t elem, const Value **out) {
    LG_REQUIRE(g, "gguf: null reader");
    LG_REQUIRE(field < g->fields.size(), "gguf: field %llu of %zu", (unsigned long long)field, g->fields.size());
    const char *key = g->fields[field].first.c_str();
    const Value *v = &g->fields[field].second;
    if (elem != UINT64_MAX) {
        if (v->type != V_ARR) return fail(LG_EINVAL, "gguf: '%s' is not an array", key);
        if (elem >= v->arr.size()) return fail(LG_EINVAL, "gguf: '%s' has %zu elements", key, v->arr.size());
        v = &v->arr[elem];
    }
    *out = v;
    return LG_OK;
}

int check_tensor(const lg_gguf *g, uint64_t index, const char *what) {
    LG_REQUIRE(g, "%s: null reader", what);
    LG_REQUIRE(index < g->tensors.size(), "%s: tensor index %llu of %zu", what, (unsigned long long)index,
               g->tensors.size());
    const Tensor &t = g->tensors[index];
    if (g->data_offset + t.data_offset + t.n_bytes > g->file_size || g->data_offset + t.data_offset < g->data_offset)
        return fail(LG_EIO, "%s: tensor '%s' (%llu bytes at %llu) runs past the end of %s", what, t.name.c_str(),
                    (unsigned long long)t.n_bytes, (unsigned long long)t.data_offset, g->path.c_str());
    return LG_OK;
}

int pread_all(int fd, void *dst, uint64_t n, uint64_t off, const char *path) {
    uint8_t *p = static_cast<uint8_t *>(dst);
    while (n) {
        const size_t chunk = n > (1u << 30) ? (1u << 30) : (size_t)n;
        const ssize_t r = pread(fd, p, chunk, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return fail(LG_EIO, "gguf: read of %s failed at %llu: %s", path, (unsigned long long)off,
                                r == 0 ? "unexpected end of file" : strerror(errno));
        p += r, off += (uint64_t)r, n -= (uint64_t)r;
    }
    return LG_OK;
}

}  // namespace

extern "C" {

int lg_gguf_type_info(int dtype, uint32_t *block_bytes, uint32_t *block_elements, int *supported, int *quantized) {
    clear_error();
    TypeRow r;
    if (dtype < 0 || !type_row((uint32_t)dtype, r)) return fail(LG_EINVAL, "gguf: unknown tensor type %d", dtype);
    if (block_bytes) *block_bytes = r.block_bytes;
    if (block_elements) *block_elements = r.block_elems;
    // TensorType::is_supported (src/gguf.rs:143-152)
    if (supported) *supported = dtype == LG_F32 || dtype == LG_F16 || dtype == LG_BF16 || dtype == LG_Q8_0 || dtype == LG_Q4_K;
    if (quantized) *quantized = r.quantized;
    return LG_OK;
}

int lg_gguf_open(const char *path, lg_gguf **out) {
    clear_error();
    LG_REQUIRE(path && out, "lg_gguf_open: null argument");
    *out = nullptr;
    lg_gguf *g = new (std::nothrow) lg_gguf();
    if (!g) return fail(LG_ENOMEM, "lg_gguf_open: out of host memory");
    std::memset(&g->meta, 0, sizeof g->meta);
    g->path = path;
    int st;
    try {
        st = open_file(path, g);
    } catch (const std::bad_alloc &) {
        st = fail(LG_EIO, "gguf: %s: metadata too large for host memory", path);
    }
    if (st != LG_OK) {
        if (g->fd >= 0) ::close(g->fd);
        delete g;
        return st;
    }
    *out = g;
    return LG_OK;
}

int lg_gguf_close(lg_gguf *g) {
    clear_error();
    if (!g) return LG_OK;
    if (g->fd >= 0) ::close(g->fd);
    delete g;
    return LG_OK;
}

int lg_gguf_header(const lg_gguf *g, uint32_t *version, uint64_t *tensor_count, uint64_t *field_count,
                   uint64_t *tensor_data_offset) {
    clear_error();
    LG_REQUIRE(g, "lg_gguf_header: null reader");
    if (version) *version = g->version;
    if (tensor_count) *tensor_count = g->tensor_count;
    if (field_count) *field_count = g->field_count;
    if (tensor_data_offset) *tensor_data_offset = g->data_offset;
    return LG_OK;
}

int lg_gguf_metadata(const lg_gguf *g, lg_gguf_meta *out) {
    clear_error();
    LG_REQUIRE(g && out, "lg_gguf_metadata: null argument");
    *out = g->meta;
    return LG_OK;
}

int lg_gguf_tensor_info(const lg_gguf *g, uint64_t index, lg_gguf_tensor *out) {
    clear_error();
    LG_REQUIRE(g && out, "lg_gguf_tensor_info: null argument");
    LG_REQUIRE(index < g->tensors.size(), "lg_gguf_tensor_info: index %llu of %zu", (unsigned long long)index,
               g->tensors.size());
    const Tensor &t = g->tensors[index];
    std::memset(out, 0, sizeof *out);
    out->name = t.name.c_str();
    out->n_dims = (uint32_t)t.shape.size();
    for (size_t d = 0; d < t.shape.size(); d++) out->shape[d] = t.shape[d];
    out->dtype = (int)t.dtype;
    out->data_offset = t.data_offset;
    out->n_elements = t.n_elements;
    out->n_bytes = t.n_bytes;
    return LG_OK;
}

int lg_gguf_find_tensor(const lg_gguf *g, const char *name, uint64_t *index) {
    clear_error();
    LG_REQUIRE(g && name && index, "lg_gguf_find_tensor: null argument");
    auto it = g->tensor_index.find(name);
    if (it == g->tensor_index.end()) return fail(LG_ENOTFOUND, "gguf: no tensor '%s'", name);
    *index = it->second;
    return LG_OK;
}

int lg_gguf_read_tensor(const lg_gguf *g, uint64_t index, void *dst, uint64_t dst_bytes) {
    clear_error();
    LG_TRY(check_tensor(g, index, "lg_gguf_read_tensor"));
    const Tensor &t = g->tensors[index];
    LG_REQUIRE(dst || t.n_bytes == 0, "lg_gguf_read_tensor: null destination");
    LG_REQUIRE(dst_bytes >= t.n_bytes, "lg_gguf_read_tensor: '%s' needs %llu bytes, destination has %llu",
               t.name.c_str(), (unsigned long long)t.n_bytes, (unsigned long long)dst_bytes);
    return pread_all(g->fd, dst, t.n_bytes, g->data_offset + t.data_offset, g->path.c_str());
}

int lg_gguf_upload_tensor(const lg_gguf *g, uint64_t index, void *dptr, uint64_t dst_bytes, void *stream) {
    clear_error();
    LG_TRY(check_tensor(g, index, "lg_gguf_upload_tensor"));
    const Tensor &t = g->tensors[index];
    LG_REQUIRE(dptr || t.n_bytes == 0, "lg_gguf_upload_tensor: null destination");
    LG_REQUIRE(dst_bytes >= t.n_bytes, "lg_gguf_upload_tensor: '%s' needs %llu bytes, destination has %llu",
               t.name.c_str(), (unsigned long long)t.n_bytes, (unsigned long long)dst_bytes);
    LG_EXTENT(dptr, t.n_bytes, "lg_gguf_upload_tensor");
    if (t.n_bytes == 0) return LG_OK;
    hipStream_t s = (hipStream_t)stream;
    // two pinned halves: the file read of one overlaps the copy of the other
    constexpr uint64_t HALF = 8u << 20;
    void *pin = nullptr;
    LG_HIP_TRY(hipHostMalloc(&pin, 2 * HALF, hipHostMallocDefault));
    hipEvent_t ev[2] = {nullptr, nullptr};
    int st = LG_OK;
    for (int i = 0; i < 2 && st == LG_OK; i++)
        if (hipEventCreateWithFlags(&ev[i], hipEventDisableTiming) != hipSuccess)
            st = fail(LG_EHIP, "lg_gguf_upload_tensor: event creation failed");
    uint64_t done = 0;
    for (int h = 0; st == LG_OK && done < t.n_bytes; h ^= 1) {
        const uint64_t n = t.n_bytes - done < HALF ? t.n_bytes - done : HALF;
        uint8_t *buf = static_cast<uint8_t *>(pin) + h * HALF;
        if (hipEventSynchronize(ev[h]) != hipSuccess) {  // the copy that last used this half has finished
            st = fail(LG_EHIP, "lg_gguf_upload_tensor: wait failed");
            break;
        }
        st = pread_all(g->fd, buf, n, g->data_offset + t.data_offset + done, g->path.c_str());
        if (st != LG_OK) break;
        hipError_t e = hipMemcpyAsync(static_cast<uint8_t *>(dptr) + done, buf, n, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipEventRecord(ev[h], s);
        if (e != hipSuccess) st = fail(LG_EHIP, "lg_gguf_upload_tensor: copy failed: %s", hipGetErrorString(e));
        done += n;
    }
    // the staging memory is released only after every copy from it has finished
    const hipError_t e = hipStreamSynchronize(s);
    if (st == LG_OK && e != hipSuccess) st = fail(LG_EHIP, "lg_gguf_upload_tensor: %s", hipGetErrorString(e));
    for (hipEvent_t x : ev)
        if (x) (void)hipEventDestroy(x);
    (void)hipHostFree(pin);
    return st;
}

// ---- raw metadata fields (GGUFReader::metadata.raw_fields, src/gguf.rs:341-355)

int lg_gguf_field_count(const lg_gguf *g, uint64_t *count) {
    clear_error();
    LG_REQUIRE(g && count, "lg_gguf_field_count: null argument");
    *count = g->fields.size();
    return LG_OK;
}

int lg_gguf_find_field(const lg_gguf *g, const char *key, uint64_t *index) {
    clear_error();
    LG_REQUIRE(g && key && index, "lg_gguf_find_field: null argument");
    auto it = g->field_index.find(key);
    if (it == g->field_index.end()) return fail(LG_ENOTFOUND, "gguf: no metadata key '%s'", key);
    *index = it->second;
    return LG_OK;
}

int lg_gguf_field(const lg_gguf *g, uint64_t index, const char **key, int *type, uint64_t *n_elements,
                  int *element_type) {
    clear_error();
    LG_REQUIRE(g, "lg_gguf_field: null reader");
    LG_REQUIRE(index < g->fields.size(), "lg_gguf_field: index %llu of %zu", (unsigned long long)index,
               g->fields.size());
    const Value &v = g->fields[index].second;
    if (key) *key = g->fields[index].first.c_str();
    if (type) *type = (int)v.type;
    if (n_elements) *n_elements = v.type == V_ARR ? v.arr.size() : 1;
    if (element_type) *element_type = v.type == V_ARR && !v.arr.empty() ? (int)v.arr[0].type : -1;
    return LG_OK;
}

int lg_gguf_get_u64(const lg_gguf *g, uint64_t field, uint64_t elem, uint64_t *out) {
    clear_error();
    LG_REQUIRE(g && out, "lg_gguf_get_u64: null argument");
    const Value *v;
    LG_TRY(field_elem(g, field, elem, &v));
    const char *key = g->fields[field].first.c_str();
    if (!as_u64(*v, *out)) return fail(LG_EINVAL, "gguf: '%s' (type %u) has no integer value", key, v->type);
    return LG_OK;
}

int lg_gguf_get_i64(const lg_gguf *g, uint64_t field, uint64_t elem, int64_t *out) {
    clear_error();
    LG_REQUIRE(g && out, "lg_gguf_get_i64: null argument");
    const Value *v;
    LG_TRY(field_elem(g, field, elem, &v));
    const char *key = g->fields[field].first.c_str();
    if (v->type == V_BOOL || v->type == V_STR || v->type == V_ARR || v->type == V_F32 || v->type == V_F64)
        return fail(LG_EINVAL, "gguf: '%s' (type %u) is not an integer", key, v->type);
    *out = (int64_t)v->u;  // signed types were sign-extended when read
    return LG_OK;
}

int lg_gguf_get_f32(const lg_gguf *g, uint64_t field, uint64_t elem, float *out) {
    clear_error();
    LG_REQUIRE(g && out, "lg_gguf_get_f32: null argument");
    const Value *v;
    LG_TRY(field_elem(g, field, elem, &v));
    const char *key = g->fields[field].first.c_str();
    if (!as_f32(*v, *out)) return fail(LG_EINVAL, "gguf: '%s' (type %u) has no float value", key, v->type);
    return LG_OK;
}

int lg_gguf_get_f64(const lg_gguf *g, uint64_t field, uint64_t elem, double *out) {
    clear_error();
    LG_REQUIRE(g && out, "lg_gguf_get_f64: null argument");
    const Value *v;
    LG_TRY(field_elem(g, field, elem, &v));
    const char *key = g->fields[field].first.c_str();
    if (v->type != V_F32 && v->type != V_F64) return fail(LG_EINVAL, "gguf: '%s' (type %u) is not a float", key, v->type);
    *out = v->f;
    return LG_OK;
}

int lg_gguf_get_bool(const lg_gguf *g, uint64_t field, uint64_t elem, int *out) {
    clear_error();
    LG_REQUIRE(g && out, "lg_gguf_get_bool: null argument");
    const Value *v;
    LG_TRY(field_elem(g, field, elem, &v));
    const char *key = g->fields[field].first.c_str();
    bool b;
    if (!as_bool(*v, b)) return fail(LG_EINVAL, "gguf: '%s' (type %u) has no boolean value", key, v->type);
    *out = b;
    return LG_OK;
}

int lg_gguf_get_str(const lg_gguf *g, uint64_t field, uint64_t elem, const char **out, uint64_t *len) {
    clear_error();
    LG_REQUIRE(g && out, "lg_gguf_get_str: null argument");
    const Value *v;
    LG_TRY(field_elem(g, field, elem, &v));
    const char *key = g->fields[field].first.c_str();
    if (v->type != V_STR) return fail(LG_EINVAL, "gguf: '%s' (type %u) is not a string", key, v->type);
    *out = v->s.c_str();
    if (len) *len = v->s.size();
    return LG_OK;
}

}  // extern "C"
