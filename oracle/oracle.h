/*
 * oracle.h -- CPU restatement of the arithmetic behind cosyvoice.cpp's attention
 * operator boundary.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library, and only as the checker or as the timed CPU
 * baseline.  The product library (libcvattn.so) never links or calls it.
 *
 * What it restates:
 *   - the ggml block formats the KV cache uses (src/cosyvoice-kv-cache.cpp:113-114 picks
 *     k_type/v_type; src/cosyvoice-loader.cpp:468-510 lists f32/f16/q8_0/q5_1/q5_0/q4_1/q4_0)
 *     together with ggml's reference quantizers/dequantizers (ggml-quants.c, not vendored:
 *     the reference clones ggml at configure time, cmake/Dependencies.cmake:98-106);
 *   - the ggml_flash_attn_ext op contract used at src/cosyvoice-kv-cache.cpp:383-384 and
 *     src/cosyvoice-graph.cpp:375-376, as an fp64 textbook softmax(QK^T*scale+mask)V;
 *   - ggml's CPU flash-attention loop (ggml-cpu/ops.cpp), as the reported CPU baseline;
 *   - the caller-built masks (src/cosyvoice-llm.cpp:20-29, src/cosyvoice-token2wav.cpp:285-298);
 *   - the KV write ggml_set_rows (src/cosyvoice-kv-cache.cpp:316,322);
 *   - the rotary embedding the callers apply to Q and K before it, ggml_rope_ext
 *     (src/cosyvoice-llm.cpp:56-57, src/cosyvoice-graph.cpp:351-352).
 *
 * Pinning (how each function is checked beyond retyping it; see tests/test_oracle_*.py):
 *   or_fp32_to_fp16 / or_fp16_to_fp32 : exhaustive vs numpy float16 casts (all 65536 halves,
 *                                       and ties/overflow/subnormal sweeps).
 *   or_quantize_row / or_dequantize_row: closed forms + invariants (amax -> +-127, the max-|x|
 *                                       element -> code 0 for q4_0, |x - deq| <= d/2, code
 *                                       ranges), exhaustive dequant over every fp16 scale, and
 *                                       committed golden blocks.
 *   or_flash_attn_ext_f64             : torch scaled_dot_product_attention (fp64, CPU) on the
 *                                       same dequantized tensors, plus invariants (n_kv=1,
 *                                       identical keys, key permutation, all-masked row -> 0).
 *   or_flash_attn_ext_ggml_cpu        : within tolerance of or_flash_attn_ext_f64.  Its exact
 *                                       bits (q8_0 rounding of Q, fp16 V accumulation, expf)
 *                                       follow ggml's published CPU loop and are parity
 *                                       unpinned: ggml is not available to compare against.
 *   or_causal_mask / or_chunk_mask    : brute-force predicate checks.
 *   or_set_rows                       : equals or_quantize_row per row (by construction) and
 *                                       is checked for untouched rows / index semantics.
 *   or_rope_f32                       : position 0 is the identity; a hand-computed known answer
 *                                       (x = (1, 0) at p = 1 gives (cos 1, sin 1)); float64
 *                                       rotation by the same float32 angles; angles against the
 *                                       closed form p * base^(-2k/n); pair norms preserved;
 *                                       scores depend only on the position difference; NEOX is
 *                                       NORMAL under the pairing permutation (bit-exact); dims
 *                                       from n_dims on copied bit-exactly.
 */
#ifndef CVATTN_ORACLE_H
#define CVATTN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_type numbering (ggml.h): the KV cache types used by cosyvoice.cpp. */
enum {
    OR_TYPE_F32 = 0,
    OR_TYPE_F16 = 1,
    OR_TYPE_Q4_0 = 2,
    OR_TYPE_Q4_1 = 3,
    OR_TYPE_Q5_0 = 6,
    OR_TYPE_Q5_1 = 7,
    OR_TYPE_Q8_0 = 8,
    OR_TYPE_Q8_1 = 9, /* only as ggml's vec_dot type for q4_1/q5_1 keys */
};

/* Mirrors the ggml_tensor fields the op reads: data, type, ne[4], nb[4] (bytes). */
typedef struct or_tensor {
    void *data;
    int32_t type;
    int64_t ne[4];
    size_t nb[4];
} or_tensor;

uint16_t or_fp32_to_fp16(float f);
float or_fp16_to_fp32(uint16_t h);
void or_fp32_to_fp16_row(const float *x, uint16_t *y, int64_t n);
void or_fp16_to_fp32_row(const uint16_t *x, float *y, int64_t n);

int64_t or_block_size(int type);  /* elements per block (1 for f32/f16) */
int64_t or_type_size(int type);   /* bytes per block */
int64_t or_row_size(int type, int64_t n);

/* ggml reference quantizers (quantize_row_*_ref) and dequantizers; k % block == 0. */
int or_quantize_row(int type, const float *x, void *y, int64_t k);
int or_dequantize_row(int type, const void *x, float *y, int64_t k);

/* ggml's x86 CPU row quantizer for q8_0 (used to convert Q to the vec-dot type on CPU). */
void or_quantize_row_q8_0_cpu(const float *x, void *y, int64_t k);
void or_quantize_row_q8_1_cpu(const float *x, void *y, int64_t k);

/* fp64 textbook attention with ggml_flash_attn_ext semantics; dst f32 [Dv, H, n_q, B]. */
int or_flash_attn_ext_f64(const or_tensor *q, const or_tensor *k, const or_tensor *v,
                          const or_tensor *mask, float *dst, float scale);

/* ggml CPU flash-attention loop restated (one online-softmax pass per row); rows are
 * split over n_threads POSIX threads like ggml's CPU backend splits them. */
int or_flash_attn_ext_ggml_cpu(const or_tensor *q, const or_tensor *k, const or_tensor *v,
                               const or_tensor *mask, float *dst, float scale, int n_threads);

/* Non-flash path (src/cosyvoice-kv-cache.cpp:387-395): V stored transposed. */
int or_attn_nonfa_f64(const or_tensor *q, const or_tensor *k, const or_tensor *vt,
                      const or_tensor *mask, float *dst, float scale);

/* Masks as the callers fill them (0 or -inf as fp16 0xFC00). */
void or_causal_mask(uint16_t *mask, uint32_t n_batch, uint32_t seq_len);
void or_chunk_mask(uint16_t *mask, int64_t n, const uint32_t *bounds, int64_t n_bounds);

/* ggml_set_rows: dst rows idx[i] <- quantize(src row i).  dst is [ne0, rows, ...]
 * with row stride dst_nb1; src f32 rows of ne0 with stride src_nb1. */
int or_set_rows(void *dst, int dst_type, size_t dst_nb1, int64_t dst_rows, const float *src,
                size_t src_nb1, int64_t ne0, const int32_t *idx, int64_t n_rows);

/* ggml_rope_ext with freq_factors NULL, ext_factor 0 and attn_factor 1 (the forms cosyvoice.cpp
 * calls: src/cosyvoice-llm.cpp:56-57 NEOX with theta from the GGUF; src/cosyvoice-graph.cpp:351-352
 * ggml_rope NORMAL, base 10000, 64 rotated dims of a 1024-wide row).  n_rows contiguous f32 rows
 * of ne0 elements; row r is at position pos[r].  Pair k (k < n_dims/2) is (2k, 2k+1) for NORMAL
 * and (k, k + n_dims/2) for NEOX, rotated by theta_k = p * s^k with s = powf(freq_base,
 * -2/n_dims) applied by repeated float multiplication, then times freq_scale; elements from
 * n_dims on are copied. */
enum { OR_ROPE_NORMAL = 0, OR_ROPE_NEOX = 2 };
int or_rope_f32(const float *src, float *dst, int64_t ne0, int64_t n_rows, const int32_t *pos, int n_dims,
                int mode, float freq_base, float freq_scale);

#ifdef __cplusplus
}
#endif
#endif
