// cvattn_gguf.cpp -- GGUF v3 reader/writer, the attention geometry of a CosyVoice3 model file and
// the prompt-speech asset (see cvattn_gguf.h).  Host code only.
#include "cvattn_gguf.h"

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <new>

namespace cvattn {

// ---- ggml type table --------------------------------------------------------------------------
// Block bytes and block elements of every ggml_type code (ggml.h / ggml-common.h); codes ggml has
// retired (4, 5, 31-33, 36-38) have none.  A GGUF naming any other code is refused, as the
// reference refuses codes its ggml does not know.
namespace {
struct type_traits {
    uint16_t size;
    uint16_t blck;
};
constexpr type_traits kTypes[] = {
    {4, 1},     // 0  F32
    {2, 1},     // 1  F16
    {18, 32},   // 2  Q4_0
    {20, 32},   // 3  Q4_1
    {0, 0},     // 4  (retired)
    {0, 0},     // 5  (retired)
    {22, 32},   // 6  Q5_0
    {24, 32},   // 7  Q5_1
    {34, 32},   // 8  Q8_0
    {36, 32},   // 9  Q8_1
    {84, 256},  // 10 Q2_K
    {110, 256}, // 11 Q3_K
    {144, 256}, // 12 Q4_K
    {176, 256}, // 13 Q5_K
    {210, 256}, // 14 Q6_K
    {292, 256}, // 15 Q8_K
    {66, 256},  // 16 IQ2_XXS
    {74, 256},  // 17 IQ2_XS
    {98, 256},  // 18 IQ3_XXS
    {50, 256},  // 19 IQ1_S
    {18, 32},   // 20 IQ4_NL
    {110, 256}, // 21 IQ3_S
    {82, 256},  // 22 IQ2_S
    {136, 256}, // 23 IQ4_XS
    {1, 1},     // 24 I8
    {2, 1},     // 25 I16
    {4, 1},     // 26 I32
    {8, 1},     // 27 I64
    {8, 1},     // 28 F64
    {56, 256},  // 29 IQ1_M
    {2, 1},     // 30 BF16
    {0, 0},     // 31 (retired)
    {0, 0},     // 32 (retired)
    {0, 0},     // 33 (retired)
    {54, 256},  // 34 TQ1_0
    {66, 256},  // 35 TQ2_0
    {0, 0},     // 36 (retired)
    {0, 0},     // 37 (retired)
    {0, 0},     // 38 (retired)
    {17, 32},   // 39 MXFP4
};
constexpr int kNumTypes = (int)(sizeof(kTypes) / sizeof(kTypes[0]));
constexpr int kTypeI8 = 24, kTypeI32 = 26;

size_t gguf_value_size(int32_t t) {
    switch (t) {
    case CVATTN_GGUF_TYPE_UINT8:
    case CVATTN_GGUF_TYPE_INT8:
    case CVATTN_GGUF_TYPE_BOOL: return 1;
    case CVATTN_GGUF_TYPE_UINT16:
    case CVATTN_GGUF_TYPE_INT16: return 2;
    case CVATTN_GGUF_TYPE_UINT32:
    case CVATTN_GGUF_TYPE_INT32:
    case CVATTN_GGUF_TYPE_FLOAT32: return 4;
    case CVATTN_GGUF_TYPE_UINT64:
    case CVATTN_GGUF_TYPE_INT64:
    case CVATTN_GGUF_TYPE_FLOAT64: return 8;
    default: return 0; // strings, arrays, unknown codes
    }
}

size_t pad_to(size_t n, size_t a) { return (n + a - 1) & ~(a - 1); }

// Bounds-checked little-endian reads over [p, end).
struct reader {
    const uint8_t *p, *end;
    size_t left() const { return (size_t)(end - p); }
    template <typename T>
    bool get(T &out) {
        if (left() < sizeof(T)) return false;
        std::memcpy(&out, p, sizeof(T));
        p += sizeof(T);
        return true;
    }
    // a GGUF string: u64 length, then the bytes (strings longer than 1 GiB are refused)
    bool str(std::string_view &out) {
        uint64_t n;
        if (!get(n) || n > (1ull << 30) || n > left()) return false;
        out = std::string_view(reinterpret_cast<const char *>(p), (size_t)n);
        p += n;
        return true;
    }
};

std::string join_key(const char *prefix, const char *name) {
    if (!prefix || !*prefix) return name;
    return std::string(prefix) + "." + name;
}
} // namespace

size_t ggml_type_size(int t) { return t >= 0 && t < kNumTypes ? kTypes[t].size : 0; }
int64_t ggml_blck_size(int t) { return t >= 0 && t < kNumTypes ? kTypes[t].blck : 0; }

// ---- parser -----------------------------------------------------------------------------------

bool gguf_parser::fail(std::string msg) {
    err_ = std::move(msg);
    return false;
}

bool gguf_parser::parse(const uint8_t *buffer, size_t size) {
    kv.clear();
    info.clear();
    alignment = CVATTN_GGUF_DEFAULT_ALIGNMENT;
    err_.clear();
    if (!buffer || size < 24) return fail("buffer too small");
    reader r{buffer, buffer + size};
    if (std::memcmp(r.p, "GGUF", 4) != 0) return fail("bad magic (expected GGUF)");
    r.p += 4;
    uint32_t version = 0;
    if (!r.get(version) || version != 3) return fail("unsupported GGUF version " + std::to_string(version));
    int64_t n_tensors = 0, n_kv = 0;
    if (!r.get(n_tensors) || !r.get(n_kv) || n_tensors < 0 || n_kv < 0) return fail("bad header counts");
    // every key/value takes at least 12 bytes and every tensor info at least 24: counts the
    // image cannot hold are refused before anything is reserved
    if ((uint64_t)n_kv > r.left() / 12 || (uint64_t)n_tensors > r.left() / 24) return fail("counts exceed the image");
    kv.reserve((size_t)n_kv);
    info.reserve((size_t)n_tensors);

    for (int64_t i = 0; i < n_kv; i++) {
        gguf_kv_entry e;
        std::string_view key;
        if (!r.str(key)) return fail("truncated key " + std::to_string(i));
        e.key.assign(key);
        int32_t type;
        if (!r.get(type)) return fail("truncated value type of '" + e.key + "'");
        if (type == CVATTN_GGUF_TYPE_ARRAY) {
            e.is_array = true;
            uint64_t n;
            if (!r.get(e.type) || !r.get(n)) return fail("truncated array header of '" + e.key + "'");
            e.arr_len = (size_t)n;
            if (e.type == CVATTN_GGUF_TYPE_STRING) {
                if (n > r.left() / 8) return fail("array '" + e.key + "' exceeds the image");
                e.arr_strings.resize((size_t)n);
                for (uint64_t j = 0; j < n; j++)
                    if (!r.str(e.arr_strings[(size_t)j])) return fail("truncated string array '" + e.key + "'");
            } else {
                const size_t es = gguf_value_size(e.type);
                if (es == 0) return fail("array '" + e.key + "' has element type " + std::to_string(e.type));
                if (n > r.left() / es) return fail("array '" + e.key + "' exceeds the image");
                e.arr_data.assign(r.p, r.p + (size_t)n * es);
                r.p += (size_t)n * es;
            }
        } else {
            e.type = type;
            const size_t es = gguf_value_size(type);
            if (es > 0) {
                if (r.left() < es) return fail("truncated value of '" + e.key + "'");
                e.data.assign(r.p, r.p + es);
                r.p += es;
            } else if (type == CVATTN_GGUF_TYPE_STRING) {
                std::string_view v;
                if (!r.str(v)) return fail("truncated string '" + e.key + "'");
                e.str_value.assign(v);
            } else {
                return fail("key '" + e.key + "' has value type " + std::to_string(type));
            }
        }
        kv.push_back(std::move(e));
    }

    for (int64_t i = 0; i < n_tensors; i++) {
        gguf_tensor_info ti;
        std::memset(&ti.t, 0, sizeof(ti.t));
        ti.t.ne[0] = ti.t.ne[1] = ti.t.ne[2] = ti.t.ne[3] = 1;
        std::string_view name;
        if (!r.str(name)) return fail("truncated tensor name " + std::to_string(i));
        if (name.size() >= CVATTN_GGUF_MAX_NAME) return fail("tensor name " + std::to_string(i) + " too long");
        ti.name.assign(name);
        uint32_t n_dims;
        if (!r.get(n_dims)) return fail("truncated tensor '" + ti.name + "'");
        if (n_dims > 4) return fail("tensor '" + ti.name + "' has " + std::to_string(n_dims) + " dimensions");
        int64_t elems = 1;
        for (uint32_t j = 0; j < n_dims; j++) {
            if (!r.get(ti.t.ne[j])) return fail("truncated tensor '" + ti.name + "'");
            if (ti.t.ne[j] < 0) return fail("tensor '" + ti.name + "' has a negative dimension");
        }
        for (int j = 0; j < 4; j++)
            if (__builtin_mul_overflow(elems, ti.t.ne[j], &elems)) return fail("tensor '" + ti.name + "' overflows");
        int32_t type;
        if (!r.get(type)) return fail("truncated tensor '" + ti.name + "'");
        const size_t ts = ggml_type_size(type);
        const int64_t bs = ggml_blck_size(type);
        if (ts == 0 || bs == 0) return fail("tensor '" + ti.name + "' has type " + std::to_string(type));
        if (ti.t.ne[0] % bs != 0) return fail("tensor '" + ti.name + "' row is not a whole number of blocks");
        ti.t.type = type;
        ti.t.nb[0] = ts;
        ti.t.nb[1] = (size_t)(ti.t.ne[0] / bs) * ts;
        for (int j = 2; j < 4; j++) ti.t.nb[j] = ti.t.nb[j - 1] * (size_t)ti.t.ne[j - 1];
        if (!r.get(ti.offset)) return fail("truncated tensor '" + ti.name + "'");
        info.push_back(std::move(ti));
    }

    // general.alignment: the first key of that name, read as the reference reads it (its first
    // four value bytes), and a power of two
    for (const auto &e : kv)
        if (e.key == "general.alignment") {
            if (e.data.size() >= 4) {
                uint32_t a;
                std::memcpy(&a, e.data.data(), 4);
                alignment = a;
            }
            break;
        }
    if (alignment == 0 || (alignment & (alignment - 1)) != 0)
        return fail("alignment " + std::to_string(alignment) + " is not a power of 2");

    const size_t data_start = pad_to((size_t)(r.p - buffer), alignment);
    if (data_start > size) return fail("data section beyond the image");
    // tensors lie end to end, each padded to the alignment
    uint64_t expected = 0;
    for (auto &ti : info) {
        if (ti.offset != expected)
            return fail("tensor '" + ti.name + "' at offset " + std::to_string(ti.offset) + ", expected " +
                        std::to_string(expected));
        size_t bytes = 0;
        if (ti.t.ne[0] > 0 && ti.t.ne[1] > 0 && ti.t.ne[2] > 0 && ti.t.ne[3] > 0) bytes = ti.t.nb[3] * (size_t)ti.t.ne[3];
        expected += pad_to(bytes, alignment);
        if (expected > size - data_start) return fail("tensor '" + ti.name + "' data beyond the image");
        ti.t.data = const_cast<uint8_t *>(buffer + data_start + ti.offset);
    }
    return true;
}

int64_t gguf_parser::find_key(const char *key_name) const {
    if (!key_name) return -1;
    for (size_t i = 0; i < kv.size(); i++)
        if (kv[i].key == key_name) return (int64_t)i;
    return -1;
}

int32_t gguf_parser::arr_type(int64_t id) const {
    if (id < 0 || id >= n_kv()) return CVATTN_GGUF_TYPE_COUNT;
    return kv[(size_t)id].is_array ? kv[(size_t)id].type : CVATTN_GGUF_TYPE_COUNT;
}

uint32_t gguf_parser::val_u32(int64_t id) const {
    if (id < 0 || id >= n_kv() || kv[(size_t)id].data.size() < 4) return 0;
    uint32_t v;
    std::memcpy(&v, kv[(size_t)id].data.data(), 4);
    return v;
}

int32_t gguf_parser::val_i32(int64_t id) const { return (int32_t)val_u32(id); }

float gguf_parser::val_f32(int64_t id) const {
    const uint32_t u = val_u32(id);
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

const char *gguf_parser::val_str(int64_t id) const {
    if (id < 0 || id >= n_kv()) return "";
    return kv[(size_t)id].str_value.c_str();
}

size_t gguf_parser::arr_n(int64_t id) const {
    if (id < 0 || id >= n_kv()) return 0;
    const auto &e = kv[(size_t)id];
    if (!e.is_array) return 0;
    return e.type == CVATTN_GGUF_TYPE_STRING ? e.arr_strings.size() : e.arr_len;
}

const void *gguf_parser::arr_data(int64_t id) const {
    if (id < 0 || id >= n_kv()) return nullptr;
    const auto &e = kv[(size_t)id];
    if (!e.is_array || e.type == CVATTN_GGUF_TYPE_STRING) return nullptr;
    return e.arr_data.data();
}

std::string_view gguf_parser::arr_str(int64_t id, size_t i) const {
    if (id < 0 || id >= n_kv()) return {};
    const auto &e = kv[(size_t)id];
    return i < e.arr_strings.size() ? e.arr_strings[i] : std::string_view{};
}

const gguf_tensor_info *gguf_parser::find_tensor(const char *name) const {
    if (!name) return nullptr;
    for (const auto &ti : info)
        if (ti.name == name) return &ti;
    return nullptr;
}

// ---- writer -----------------------------------------------------------------------------------

void gguf_writer::set_val_u32(const char *key, uint32_t v) {
    for (auto &e : kv_)
        if (e.key == key) {
            e.v = v;
            return;
        }
    kv_.push_back({key, v});
}

void gguf_writer::add_tensor(const char *name, int type, int n_dims, const int64_t *ne, const void *data) {
    tensor t;
    t.name = name;
    t.type = type;
    t.n_dims = n_dims;
    for (int j = 0; j < 4; j++) t.ne[j] = j < n_dims ? ne[j] : 1;
    t.data = data;
    const int64_t bs = ggml_blck_size(type);
    t.bytes = bs ? (size_t)(t.ne[0] / bs) * ggml_type_size(type) * (size_t)(t.ne[1] * t.ne[2] * t.ne[3]) : 0;
    tensors_.push_back(t);
}

std::vector<uint8_t> gguf_writer::serialize() const {
    std::vector<uint8_t> out;
    auto put = [&](const void *p, size_t n) {
        const uint8_t *b = static_cast<const uint8_t *>(p);
        out.insert(out.end(), b, b + n);
    };
    auto put_str = [&](const std::string &s) {
        const uint64_t n = s.size();
        put(&n, 8);
        put(s.data(), s.size());
    };
    const size_t align = CVATTN_GGUF_DEFAULT_ALIGNMENT;
    put("GGUF", 4);
    const uint32_t version = 3;
    put(&version, 4);
    const int64_t n_tensors = (int64_t)tensors_.size(), n_kv = (int64_t)kv_.size();
    put(&n_tensors, 8);
    put(&n_kv, 8);
    for (const auto &e : kv_) {
        put_str(e.key);
        const int32_t type = CVATTN_GGUF_TYPE_UINT32;
        put(&type, 4);
        put(&e.v, 4);
    }
    uint64_t offset = 0;
    for (const auto &t : tensors_) {
        put_str(t.name);
        // ggml writes the dimensions up to the last one above 1 (at least one)
        uint32_t n_dims = 1;
        for (int j = 3; j >= 1; j--)
            if (t.ne[j] > 1) {
                n_dims = (uint32_t)j + 1;
                break;
            }
        put(&n_dims, 4);
        for (uint32_t j = 0; j < n_dims; j++) put(&t.ne[j], 8);
        const int32_t type = t.type;
        put(&type, 4);
        put(&offset, 8);
        offset += pad_to(t.bytes, align);
    }
    out.resize(pad_to(out.size(), align), 0);
    for (const auto &t : tensors_) {
        if (t.bytes) put(t.data, t.bytes);
        out.resize(pad_to(out.size(), align), 0);
    }
    return out;
}

bool gguf_writer::write_to_file(const char *filename) const {
    if (!filename) return false;
    const std::vector<uint8_t> bytes = serialize();
    FILE *f = std::fopen(filename, "wb");
    if (!f) return false;
    const bool ok = std::fwrite(bytes.data(), 1, bytes.size(), f) == bytes.size();
    return std::fclose(f) == 0 && ok;
}

// ---- prompt speech ----------------------------------------------------------------------------

namespace {
struct crc_table {
    uint32_t t[256];
    crc_table() {
        for (uint32_t i = 0; i < 256; i++) {
            uint32_t c = i;
            for (int k = 0; k < 8; k++) c = (c & 1) ? (c >> 1) ^ 0xEDB88320u : c >> 1;
            t[i] = c;
        }
    }
};
const crc_table &crc_tab() {
    static const crc_table tab;
    return tab;
}
} // namespace

uint32_t prompt_crc32(const void *data, size_t length, uint32_t value) {
    const uint32_t *t = crc_tab().t;
    const uint8_t *b = static_cast<const uint8_t *>(data);
    for (size_t i = 0; i < length; i++) value = (value >> 8) ^ t[(value ^ b[i]) & 0xFFu];
    return ~value;
}

// The checksum runs over each part's bytes followed by its size field, in the order text, feat,
// embedding, tokens (src/cosyvoice-prompt.cpp:36-51): the text length and token count as u32, the
// matrix shapes as their two u32 (rows, cols).
void prompt_speech::calculate_crc32() {
    const uint32_t text_len = (uint32_t)text.size(), n_tokens = (uint32_t)tokens.size();
    uint32_t c = prompt_crc32(text.data(), text.size());
    c = prompt_crc32(&text_len, 4, c);
    c = prompt_crc32(feat.data(), feat.size() * sizeof(float), c);
    c = prompt_crc32(feat_shape, 8, c);
    c = prompt_crc32(embedding.data(), embedding.size() * sizeof(float), c);
    c = prompt_crc32(embedding_shape, 8, c);
    c = prompt_crc32(tokens.data(), tokens.size() * sizeof(int32_t), c);
    c = prompt_crc32(&n_tokens, 4, c);
    crc32 = c;
}

} // namespace cvattn

// ---- C ABI ------------------------------------------------------------------------------------

using namespace cvattn;

struct cvattn_gguf {
    gguf_parser p;
};
struct cvattn_prompt_speech {
    prompt_speech s;
};

namespace {
bool is_matrix(const cvattn_tensor &t) { return t.ne[2] == 1 && t.ne[3] == 1; }
bool is_vector(const cvattn_tensor &t) { return t.ne[1] == 1 && t.ne[2] == 1 && t.ne[3] == 1; }
int64_t elems(const cvattn_tensor &t) { return t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]; }

cvattn_prompt_speech *eilseq() {
    errno = EILSEQ;
    return nullptr;
}
} // namespace

extern "C" {

CVATTN_API int cvattn_gguf_open(const void *data, size_t size, cvattn_gguf **out, char *err, size_t err_len) {
    if (!out) return CVATTN_ERR_BAD_ARGS;
    *out = nullptr;
    cvattn_gguf *g = new (std::nothrow) cvattn_gguf;
    if (!g) return CVATTN_ERR_BAD_ARGS;
    if (!g->p.parse(static_cast<const uint8_t *>(data), size)) {
        if (err && err_len) {
            std::strncpy(err, g->p.error().c_str(), err_len - 1);
            err[err_len - 1] = 0;
        }
        delete g;
        return CVATTN_ERR_BAD_ARGS;
    }
    *out = g;
    return CVATTN_OK;
}

CVATTN_API void cvattn_gguf_close(cvattn_gguf *g) { delete g; }
CVATTN_API size_t cvattn_gguf_alignment(const cvattn_gguf *g) { return g ? g->p.alignment : 0; }
CVATTN_API int64_t cvattn_gguf_n_kv(const cvattn_gguf *g) { return g ? g->p.n_kv() : 0; }
CVATTN_API int64_t cvattn_gguf_find_key(const cvattn_gguf *g, const char *key) { return g ? g->p.find_key(key) : -1; }

CVATTN_API const char *cvattn_gguf_key(const cvattn_gguf *g, int64_t id) {
    if (!g || id < 0 || id >= g->p.n_kv()) return nullptr;
    return g->p.kv[(size_t)id].key.c_str();
}

CVATTN_API int cvattn_gguf_kv_type(const cvattn_gguf *g, int64_t id) {
    if (!g || id < 0 || id >= g->p.n_kv()) return -1;
    const auto &e = g->p.kv[(size_t)id];
    return e.is_array ? CVATTN_GGUF_TYPE_ARRAY : e.type;
}

CVATTN_API int cvattn_gguf_arr_type(const cvattn_gguf *g, int64_t id) {
    return g ? g->p.arr_type(id) : CVATTN_GGUF_TYPE_COUNT;
}
CVATTN_API uint32_t cvattn_gguf_val_u32(const cvattn_gguf *g, int64_t id) { return g ? g->p.val_u32(id) : 0; }
CVATTN_API int32_t cvattn_gguf_val_i32(const cvattn_gguf *g, int64_t id) { return g ? g->p.val_i32(id) : 0; }
CVATTN_API float cvattn_gguf_val_f32(const cvattn_gguf *g, int64_t id) { return g ? g->p.val_f32(id) : 0.0f; }

CVATTN_API const void *cvattn_gguf_val_data(const cvattn_gguf *g, int64_t id, size_t *bytes) {
    if (bytes) *bytes = 0;
    if (!g || id < 0 || id >= g->p.n_kv()) return nullptr;
    const auto &e = g->p.kv[(size_t)id];
    if (e.is_array || e.data.empty()) return nullptr;
    if (bytes) *bytes = e.data.size();
    return e.data.data();
}

CVATTN_API const char *cvattn_gguf_val_str(const cvattn_gguf *g, int64_t id) { return g ? g->p.val_str(id) : ""; }
CVATTN_API size_t cvattn_gguf_arr_n(const cvattn_gguf *g, int64_t id) { return g ? g->p.arr_n(id) : 0; }
CVATTN_API const void *cvattn_gguf_arr_data(const cvattn_gguf *g, int64_t id) { return g ? g->p.arr_data(id) : nullptr; }

CVATTN_API const char *cvattn_gguf_arr_str(const cvattn_gguf *g, int64_t id, size_t i, size_t *len) {
    if (len) *len = 0;
    if (!g) return nullptr;
    const std::string_view s = g->p.arr_str(id, i);
    if (len) *len = s.size();
    return s.data();
}

CVATTN_API int64_t cvattn_gguf_n_tensors(const cvattn_gguf *g) { return g ? (int64_t)g->p.info.size() : 0; }

CVATTN_API int64_t cvattn_gguf_find_tensor(const cvattn_gguf *g, const char *name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->p.info.size(); i++)
        if (g->p.info[i].name == name) return (int64_t)i;
    return -1;
}

CVATTN_API int cvattn_gguf_tensor(const cvattn_gguf *g, int64_t i, cvattn_tensor *t, const char **name,
                                  uint64_t *offset) {
    if (!g || i < 0 || i >= (int64_t)g->p.info.size()) return CVATTN_ERR_BAD_ARGS;
    const auto &ti = g->p.info[(size_t)i];
    if (t) *t = ti.t;
    if (name) *name = ti.name.c_str();
    if (offset) *offset = ti.offset;
    return CVATTN_OK;
}

CVATTN_API int cvattn_gguf_llm_attn_config(const cvattn_gguf *g, const char *prefix, cvattn_llm_attn_config *out) {
    if (!g || !out) return CVATTN_ERR_BAD_ARGS;
    const gguf_parser &p = g->p;
    const int64_t k_layers = p.find_key(join_key(prefix, "num_hidden_layers").c_str());
    const int64_t k_heads = p.find_key(join_key(prefix, "num_attention_heads").c_str());
    const int64_t k_kv = p.find_key(join_key(prefix, "num_key_value_heads").c_str());
    const int64_t k_theta = p.find_key(join_key(prefix, "rope_theta").c_str());
    if (k_layers < 0 || k_heads < 0 || k_kv < 0 || k_theta < 0) return CVATTN_ERR_BAD_ARGS;
    const std::string layer0 = join_key(prefix, "layers") + ".0.self_attn.";
    const gguf_tensor_info *kp = p.find_tensor((layer0 + "k_proj.weight").c_str());
    const gguf_tensor_info *vp = p.find_tensor((layer0 + "v_proj.weight").c_str());
    const int32_t n_kv = p.val_i32(k_kv);
    if (!kp || !vp || n_kv <= 0) return CVATTN_ERR_BAD_ARGS;
    out->n_layers = p.val_i32(k_layers);
    out->n_heads = p.val_i32(k_heads);
    out->n_kv_heads = n_kv;
    out->k_head_dim = (int32_t)(kp->t.ne[1] / n_kv);
    out->v_head_dim = (int32_t)(vp->t.ne[1] / n_kv);
    out->rope_theta = p.val_f32(k_theta);
    return CVATTN_OK;
}

CVATTN_API int cvattn_gguf_dit_attn_config(const cvattn_gguf *g, const char *prefix, cvattn_dit_attn_config *out) {
    if (!g || !out) return CVATTN_ERR_BAD_ARGS;
    const gguf_parser &p = g->p;
    const int64_t k_heads = p.find_key(join_key(prefix, "heads").c_str());
    const int64_t k_depth = p.find_key(join_key(prefix, "depth").c_str());
    if (k_heads < 0 || k_depth < 0) return CVATTN_ERR_BAD_ARGS;
    // the reference names the blocks "<prefix>.transformer_blocks.<i>" (src/cosyvoice-loader.cpp:256)
    const std::string block0 = std::string(prefix ? prefix : "") + ".transformer_blocks.0.attn.";
    const gguf_tensor_info *kp = p.find_tensor((block0 + "to_k.weight").c_str());
    const gguf_tensor_info *vp = p.find_tensor((block0 + "to_v.weight").c_str());
    const int32_t heads = p.val_i32(k_heads);
    if (!kp || !vp || heads <= 0) return CVATTN_ERR_BAD_ARGS;
    out->depth = p.val_i32(k_depth);
    out->heads = heads;
    out->k_head_dim = (int32_t)(kp->t.ne[1] / heads);
    out->v_head_dim = (int32_t)(vp->t.ne[1] / heads);
    return CVATTN_OK;
}

CVATTN_API cvattn_prompt_speech *cvattn_prompt_speech_load(const void *data, size_t size) {
    gguf_parser p;
    if (!p.parse(static_cast<const uint8_t *>(data), size)) return eilseq();
    const gguf_tensor_info *feat = p.find_tensor("feat"), *emb = p.find_tensor("embedding");
    const gguf_tensor_info *tok = p.find_tensor("tokens"), *text = p.find_tensor("text");
    if (!feat || !emb || !tok || !text || !is_matrix(feat->t) || !is_matrix(emb->t) || !is_vector(tok->t) ||
        !is_vector(text->t) || feat->t.type != CVATTN_TYPE_F32 || emb->t.type != CVATTN_TYPE_F32 ||
        tok->t.type != kTypeI32 || text->t.type != kTypeI8)
        return eilseq();
    if (feat->t.ne[0] > UINT32_MAX || feat->t.ne[1] > UINT32_MAX || emb->t.ne[0] > UINT32_MAX ||
        emb->t.ne[1] > UINT32_MAX || tok->t.ne[0] > UINT32_MAX || text->t.ne[0] > UINT32_MAX)
        return eilseq();
    cvattn_prompt_speech *ps = new (std::nothrow) cvattn_prompt_speech;
    if (!ps) return nullptr;
    prompt_speech &s = ps->s;
    // a matrix is [cols, rows] in ggml order: shape = (ne[1], ne[0])
    s.feat_shape[0] = (uint32_t)feat->t.ne[1];
    s.feat_shape[1] = (uint32_t)feat->t.ne[0];
    s.embedding_shape[0] = (uint32_t)emb->t.ne[1];
    s.embedding_shape[1] = (uint32_t)emb->t.ne[0];
    const float *fd = static_cast<const float *>(feat->t.data);
    const float *ed = static_cast<const float *>(emb->t.data);
    s.feat.assign(fd, fd + elems(feat->t));
    s.embedding.assign(ed, ed + elems(emb->t));
    const int32_t *td = static_cast<const int32_t *>(tok->t.data);
    s.tokens.assign(td, td + tok->t.ne[0]);
    const char *xd = static_cast<const char *>(text->t.data);
    s.text.assign(xd, xd + text->t.ne[0]);
    s.calculate_crc32();
    const int64_t id = p.find_key("crc32");
    if (id >= 0 && p.val_u32(id) != s.crc32) {
        delete ps;
        return eilseq();
    }
    return ps;
}

CVATTN_API cvattn_prompt_speech *cvattn_prompt_speech_load_from_file(const char *filename) {
    if (!filename) return nullptr;
    FILE *f = std::fopen(filename, "rb");
    if (!f) return nullptr;
    std::vector<uint8_t> bytes;
    uint8_t buf[1 << 16];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) bytes.insert(bytes.end(), buf, buf + n);
    const bool err = std::ferror(f) != 0;
    std::fclose(f);
    if (err) return nullptr;
    return cvattn_prompt_speech_load(bytes.data(), bytes.size());
}

CVATTN_API int cvattn_prompt_speech_save_to_file(const cvattn_prompt_speech *ps, const char *filename) {
    if (!ps || !filename) return 0;
    const prompt_speech &s = ps->s;
    gguf_writer w;
    const int64_t fne[2] = {s.feat_shape[1], s.feat_shape[0]};
    const int64_t ene[2] = {s.embedding_shape[1], s.embedding_shape[0]};
    const int64_t tne[1] = {(int64_t)s.tokens.size()};
    const int64_t xne[1] = {(int64_t)s.text.size()};
    w.add_tensor("feat", CVATTN_TYPE_F32, 2, fne, s.feat.data());
    w.add_tensor("embedding", CVATTN_TYPE_F32, 2, ene, s.embedding.data());
    w.add_tensor("tokens", kTypeI32, 1, tne, s.tokens.data());
    w.add_tensor("text", kTypeI8, 1, xne, s.text.data());
    w.set_val_u32("crc32", s.crc32);
    return w.write_to_file(filename) ? 1 : 0;
}

CVATTN_API uint32_t cvattn_prompt_speech_get_crc32(const cvattn_prompt_speech *ps) { return ps ? ps->s.crc32 : 0; }
CVATTN_API void cvattn_prompt_speech_free(cvattn_prompt_speech *ps) { delete ps; }

CVATTN_API cvattn_prompt_speech *cvattn_prompt_speech_create(const char *text, uint32_t text_len, const float *feat,
                                                             uint32_t feat_rows, uint32_t feat_cols,
                                                             const float *embedding, uint32_t emb_rows,
                                                             uint32_t emb_cols, const int32_t *tokens,
                                                             uint32_t n_tokens) {
    const uint64_t nf = (uint64_t)feat_rows * feat_cols, ne = (uint64_t)emb_rows * emb_cols;
    if ((text_len && !text) || (nf && !feat) || (ne && !embedding) || (n_tokens && !tokens)) return nullptr;
    cvattn_prompt_speech *ps = new (std::nothrow) cvattn_prompt_speech;
    if (!ps) return nullptr;
    prompt_speech &s = ps->s;
    s.text.assign(text, text + text_len);
    s.feat_shape[0] = feat_rows;
    s.feat_shape[1] = feat_cols;
    s.feat.assign(feat, feat + nf);
    s.embedding_shape[0] = emb_rows;
    s.embedding_shape[1] = emb_cols;
    s.embedding.assign(embedding, embedding + ne);
    s.tokens.assign(tokens, tokens + n_tokens);
    s.calculate_crc32();
    return ps;
}

CVATTN_API int cvattn_prompt_speech_get(const cvattn_prompt_speech *ps, cvattn_prompt_speech_view *out) {
    if (!ps || !out) return CVATTN_ERR_BAD_ARGS;
    const prompt_speech &s = ps->s;
    out->text = s.text.data();
    out->text_len = (uint32_t)s.text.size();
    out->feat = s.feat.data();
    out->feat_rows = s.feat_shape[0];
    out->feat_cols = s.feat_shape[1];
    out->embedding = s.embedding.data();
    out->emb_rows = s.embedding_shape[0];
    out->emb_cols = s.embedding_shape[1];
    out->tokens = s.tokens.data();
    out->n_tokens = (uint32_t)s.tokens.size();
    return CVATTN_OK;
}

} // extern "C"
