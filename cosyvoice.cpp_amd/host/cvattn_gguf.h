// cvattn_gguf.h -- the GGUF v3 container and the prompt-speech asset for C++ hosts.
//
// gguf_parser mirrors the reader cosyvoice.cpp uses for its model and prompt files
// (common/gguf_parser.h: parse + key/array accessors, common/gguf_parser.cpp:142-407).  The
// parse rules are the reference's: version 3 only, at most 4 dimensions, non-negative and
// non-overflowing shapes, a known ggml type whose block divides ne[0], tensors laid end to end in
// the data section at `alignment`-padded offsets, a power-of-two `general.alignment`.  Where the
// reference then builds a ggml context of tensor descriptors, the parser keeps the descriptors
// itself (find_tensor) as cvattn_tensor, the engine's ggml_tensor mirror.  The parser does not
// copy the buffer: string arrays and tensor data point into it, so it must outlive the parser.
//
// gguf_writer produces the files ggml's gguf_write_to_file writes (header, key/values, tensor
// infos, zero padding to the alignment, each tensor's data padded to the alignment).
//
// prompt_speech is cosyvoice_prompt_speech (src/cosyvoice-internal.h:122-131) with its load
// (src/cosyvoice-prompt.cpp:62-108), save (:213-241) and crc32 (:8-51).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

#include "../../include/cvattn.h"
#include "../../include/cvattn_gguf.h"

namespace cvattn {

// Bytes of one ggml block (type_size) and elements per block (blck_size) of ggml type t;
// 0 for codes ggml does not define.
size_t ggml_type_size(int t);
int64_t ggml_blck_size(int t);

struct gguf_kv_entry {
    std::string key;
    bool is_array = false;
    int32_t type = CVATTN_GGUF_TYPE_UINT8;  // value type, or the element type of an array
    std::vector<uint8_t> data;              // scalar value bytes (not for strings)
    std::string str_value;                  // string scalar
    std::vector<uint8_t> arr_data;          // numeric array elements
    size_t arr_len = 0;
    std::vector<std::string_view> arr_strings;  // string array elements (into the buffer)
};

struct gguf_tensor_info {
    std::string name;
    cvattn_tensor t;   // type, ne, nb (contiguous), data = the tensor's bytes in the buffer
    uint64_t offset;   // from the start of the data section
};

class gguf_parser {
public:
    size_t alignment = CVATTN_GGUF_DEFAULT_ALIGNMENT;
    std::vector<gguf_kv_entry> kv;
    std::vector<gguf_tensor_info> info;

    // Parses a whole GGUF image.  On failure returns false and error() says why.
    bool parse(const uint8_t *buffer, size_t size);
    const std::string &error() const { return err_; }

    int64_t find_key(const char *key_name) const;
    int64_t n_kv() const { return static_cast<int64_t>(kv.size()); }
    int32_t arr_type(int64_t id) const;  // CVATTN_GGUF_TYPE_COUNT when not an array
    uint32_t val_u32(int64_t id) const;  // the first 4 value bytes; 0 when there are fewer
    int32_t val_i32(int64_t id) const;
    float val_f32(int64_t id) const;
    const char *val_str(int64_t id) const;
    size_t arr_n(int64_t id) const;
    const void *arr_data(int64_t id) const;
    std::string_view arr_str(int64_t id, size_t i) const;

    // The tensor descriptor named `name`, or nullptr (ggml_get_tensor on the reference's context).
    const gguf_tensor_info *find_tensor(const char *name) const;

private:
    std::string err_;
    bool fail(std::string msg);
};

class gguf_writer {
public:
    void set_val_u32(const char *key, uint32_t v);
    // The tensor's bytes are copied when the file is written; `data` must stay valid until then.
    void add_tensor(const char *name, int type, int n_dims, const int64_t *ne, const void *data);
    std::vector<uint8_t> serialize() const;
    bool write_to_file(const char *filename) const;

private:
    struct kv_u32 {
        std::string key;
        uint32_t v;
    };
    struct tensor {
        std::string name;
        int type;
        int n_dims;
        int64_t ne[4];
        const void *data;
        size_t bytes;
    };
    std::vector<kv_u32> kv_;
    std::vector<tensor> tensors_;
};

// The prompt-speech asset: the prompt's text (bytes), its mel features (rows x cols f32), the
// speaker embedding (rows x cols f32) and the speech tokens (i32).
struct prompt_speech {
    std::vector<char> text;
    uint32_t feat_shape[2] = {0, 0};
    std::vector<float> feat;
    uint32_t embedding_shape[2] = {0, 0};
    std::vector<float> embedding;
    std::vector<int32_t> tokens;
    uint32_t crc32 = 0;

    void calculate_crc32();
};

// The reference's running checksum: crc32_update(v, bytes) = ~crc(v, bytes) with the reflected
// 0xEDB88320 table and no initial inversion, chained by passing the previous result.
uint32_t prompt_crc32(const void *data, size_t length, uint32_t value = 0);

} // namespace cvattn
