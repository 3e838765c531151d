/*
 * cvattn_gguf.h -- C ABI of the model-file side of the attention engine (libcvattn_host.so):
 *   - a GGUF v3 reader: the container cosyvoice.cpp loads its weights and prompt assets from
 *     (common/gguf_parser.h, common/gguf_parser.cpp:142-407), with tensor descriptors handed out
 *     as cvattn_tensor (the engine's ggml_tensor mirror, data pointing into the caller's buffer);
 *   - the attention geometry the loader reads from a CosyVoice3 GGUF to build the LLM and DiT KV
 *     caches (src/cosyvoice-loader.cpp:247-251, 447-454, 996-1025);
 *   - the prompt-speech asset (cosyvoice_prompt_speech_*, include/cosyvoice.h:540-565,
 *     src/cosyvoice-prompt.cpp:8-108,213-241): a GGUF file of tensors feat / embedding / tokens /
 *     text with a crc32 key.
 * Nothing here touches the GPU.  Functions return cvattn_status codes (or NULL / 0 as stated) and
 * never abort.
 */
#ifndef CVATTN_GGUF_H
#define CVATTN_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "cvattn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* gguf_type values */
enum {
    CVATTN_GGUF_TYPE_UINT8 = 0,
    CVATTN_GGUF_TYPE_INT8 = 1,
    CVATTN_GGUF_TYPE_UINT16 = 2,
    CVATTN_GGUF_TYPE_INT16 = 3,
    CVATTN_GGUF_TYPE_UINT32 = 4,
    CVATTN_GGUF_TYPE_INT32 = 5,
    CVATTN_GGUF_TYPE_FLOAT32 = 6,
    CVATTN_GGUF_TYPE_BOOL = 7,
    CVATTN_GGUF_TYPE_STRING = 8,
    CVATTN_GGUF_TYPE_ARRAY = 9,
    CVATTN_GGUF_TYPE_UINT64 = 10,
    CVATTN_GGUF_TYPE_INT64 = 11,
    CVATTN_GGUF_TYPE_FLOAT64 = 12,
    CVATTN_GGUF_TYPE_COUNT = 13,
};
#define CVATTN_GGUF_DEFAULT_ALIGNMENT 32
#define CVATTN_GGUF_MAX_NAME 64 /* tensor names are shorter than this (GGML_MAX_NAME) */

typedef struct cvattn_gguf cvattn_gguf;

/* Parses the GGUF image data[0..size) (gguf_parser::parse).  On success *out is a handle that
 * refers into `data`, which must outlive it.  On a malformed image returns CVATTN_ERR_BAD_ARGS and,
 * when err is non-NULL, writes the reason (truncated to err_len bytes, NUL-terminated). */
CVATTN_API int cvattn_gguf_open(const void *data, size_t size, cvattn_gguf **out, char *err, size_t err_len);
CVATTN_API void cvattn_gguf_close(cvattn_gguf *g);

CVATTN_API size_t cvattn_gguf_alignment(const cvattn_gguf *g);
CVATTN_API int64_t cvattn_gguf_n_kv(const cvattn_gguf *g);
/* index of `key`, or -1 (gguf_parser::find_key) */
CVATTN_API int64_t cvattn_gguf_find_key(const cvattn_gguf *g, const char *key);
CVATTN_API const char *cvattn_gguf_key(const cvattn_gguf *g, int64_t id);
/* the value type (CVATTN_GGUF_TYPE_ARRAY for arrays) and the element type of an array */
CVATTN_API int cvattn_gguf_kv_type(const cvattn_gguf *g, int64_t id);
CVATTN_API int cvattn_gguf_arr_type(const cvattn_gguf *g, int64_t id);
/* scalar values as the reference reads them: the first 4 bytes of the value (0 if fewer) */
CVATTN_API uint32_t cvattn_gguf_val_u32(const cvattn_gguf *g, int64_t id);
CVATTN_API int32_t cvattn_gguf_val_i32(const cvattn_gguf *g, int64_t id);
CVATTN_API float cvattn_gguf_val_f32(const cvattn_gguf *g, int64_t id);
/* raw bytes of a scalar (numeric or bool) value and their count */
CVATTN_API const void *cvattn_gguf_val_data(const cvattn_gguf *g, int64_t id, size_t *bytes);
/* string scalar ("" for other types) */
CVATTN_API const char *cvattn_gguf_val_str(const cvattn_gguf *g, int64_t id);
CVATTN_API size_t cvattn_gguf_arr_n(const cvattn_gguf *g, int64_t id);
CVATTN_API const void *cvattn_gguf_arr_data(const cvattn_gguf *g, int64_t id);
/* element i of a string array: its bytes (not NUL-terminated) and length */
CVATTN_API const char *cvattn_gguf_arr_str(const cvattn_gguf *g, int64_t id, size_t i, size_t *len);

CVATTN_API int64_t cvattn_gguf_n_tensors(const cvattn_gguf *g);
/* index of the tensor named `name`, or -1 */
CVATTN_API int64_t cvattn_gguf_find_tensor(const cvattn_gguf *g, const char *name);
/* descriptor of tensor i: type, ne, contiguous nb and data pointer into the image; its name and
 * its offset in the data section */
CVATTN_API int cvattn_gguf_tensor(const cvattn_gguf *g, int64_t i, cvattn_tensor *t, const char **name,
                                  uint64_t *offset);

/* The attention geometry of a CosyVoice3 model file, as the loader derives it
 * (src/cosyvoice-loader.cpp:447-454 and 996-1008 for the LLM, 247-251 and 1013-1025 for the DiT):
 *   LLM  num_hidden_layers, num_attention_heads, num_key_value_heads, rope_theta under `prefix`;
 *        head sizes = ne[1] of layers.0.self_attn.{k,v}_proj.weight / num_key_value_heads;
 *   DiT  depth, heads under `prefix` (decoder.estimator); head sizes = ne[1] of
 *        transformer_blocks.0.attn.{to_k,to_v}.weight / heads.
 * A missing key or tensor gives CVATTN_ERR_BAD_ARGS. */
typedef struct cvattn_llm_attn_config {
    int32_t n_layers, n_heads, n_kv_heads, k_head_dim, v_head_dim;
    float rope_theta;
} cvattn_llm_attn_config;
typedef struct cvattn_dit_attn_config {
    int32_t depth, heads, k_head_dim, v_head_dim;
} cvattn_dit_attn_config;
CVATTN_API int cvattn_gguf_llm_attn_config(const cvattn_gguf *g, const char *prefix, cvattn_llm_attn_config *out);
CVATTN_API int cvattn_gguf_dit_attn_config(const cvattn_gguf *g, const char *prefix, cvattn_dit_attn_config *out);

/* ---- prompt speech ---- */
typedef struct cvattn_prompt_speech cvattn_prompt_speech;

/* cosyvoice_prompt_speech_load: tensors feat (f32 matrix [cols, rows]), embedding (f32 matrix),
 * tokens (i32 vector), text (i8 vector); the optional u32 key crc32 must match the checksum of the
 * contents.  NULL on a malformed file (errno = EILSEQ, as the reference sets it).  The data buffer
 * can be freed after the call. */
CVATTN_API cvattn_prompt_speech *cvattn_prompt_speech_load(const void *data, size_t size);
CVATTN_API cvattn_prompt_speech *cvattn_prompt_speech_load_from_file(const char *filename);
/* cosyvoice_prompt_speech_save_to_file: 1 on success, 0 on failure */
CVATTN_API int cvattn_prompt_speech_save_to_file(const cvattn_prompt_speech *p, const char *filename);
CVATTN_API uint32_t cvattn_prompt_speech_get_crc32(const cvattn_prompt_speech *p);
CVATTN_API void cvattn_prompt_speech_free(cvattn_prompt_speech *p);

/* Builds a prompt-speech object from its parts (copied), with its crc32 computed; what the
 * reference's frontend produces (cosyvoice_frontend_prompt_speech).  NULL on bad arguments. */
CVATTN_API cvattn_prompt_speech *cvattn_prompt_speech_create(const char *text, uint32_t text_len, const float *feat,
                                                             uint32_t feat_rows, uint32_t feat_cols,
                                                             const float *embedding, uint32_t emb_rows,
                                                             uint32_t emb_cols, const int32_t *tokens,
                                                             uint32_t n_tokens);
/* Read-only view of the parts (pointers valid until cvattn_prompt_speech_free). */
typedef struct cvattn_prompt_speech_view {
    const char *text;
    uint32_t text_len;
    const float *feat;
    uint32_t feat_rows, feat_cols;
    const float *embedding;
    uint32_t emb_rows, emb_cols;
    const int32_t *tokens;
    uint32_t n_tokens;
} cvattn_prompt_speech_view;
CVATTN_API int cvattn_prompt_speech_get(const cvattn_prompt_speech *p, cvattn_prompt_speech_view *out);

#ifdef __cplusplus
}
#endif
#endif
