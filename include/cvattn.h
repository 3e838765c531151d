/*
 * cvattn.h -- C ABI of the MI355X (gfx950) attention engine for cosyvoice.cpp.
 *
 * The engine replaces the GGML_OP_FLASH_ATTN_EXT nodes that cosyvoice.cpp builds at
 *   src/cosyvoice-kv-cache.cpp:383-384   (LLM decode/prefill over the KV cache, and the DiT
 *                                         streaming-cache path)
 *   src/cosyvoice-graph.cpp:375-376      (DiT attention without a cache)
 * and the GGML_OP_SET_ROWS KV write at src/cosyvoice-kv-cache.cpp:316,322, plus the backend
 * capability probes at src/cosyvoice-loader.cpp:555-566.
 *
 * Tensors are described exactly as ggml describes them (data, type, ne[4], nb[4] in bytes), so
 * a ggml backend can forward a node's src[] tensors field by field.  Type codes are ggml_type
 * values.  All entry points are reentrant, keep no state between calls, never allocate device
 * memory and never abort: failures come back as cvattn_status codes.  Only the set-up call
 * cvattn_fa_batch_prepare waits for the device.  Pointers in descriptors are device pointers.
 */
#ifndef CVATTN_H
#define CVATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(_WIN32)
#define CVATTN_API __declspec(dllexport)
#else
#define CVATTN_API __attribute__((visibility("default")))
#endif

/* hipStream_t is `struct ihipStream_t *`; declared here so callers need no HIP headers. */
struct ihipStream_t;
typedef struct ihipStream_t *cvattn_stream_t;

/* ggml_type values of the KV cache formats (include/cosyvoice.h:32-42 lists the same set). */
typedef enum cvattn_type {
    CVATTN_TYPE_F32 = 0,
    CVATTN_TYPE_F16 = 1,
    CVATTN_TYPE_Q4_0 = 2,
    CVATTN_TYPE_Q4_1 = 3,
    CVATTN_TYPE_Q5_0 = 6,
    CVATTN_TYPE_Q5_1 = 7,
    CVATTN_TYPE_Q8_0 = 8,
    CVATTN_TYPE_I32 = 26,
} cvattn_type;

/* ggml_prec values accepted by cvattn_flash_attn_ext (all math is fp32-accumulated). */
#define CVATTN_PREC_DEFAULT 0
#define CVATTN_PREC_F32 10

typedef enum cvattn_status {
    CVATTN_OK = 0,
    CVATTN_ERR_UNSUPPORTED = 1,
    CVATTN_ERR_BAD_ARGS = 2,
    CVATTN_ERR_WORKSPACE_TOO_SMALL = 3,
    CVATTN_ERR_HIP = 4,
} cvattn_status;

/* Mirrors ggml_tensor's data/type/ne/nb. */
typedef struct cvattn_tensor {
    void *data;
    int32_t type;
    int64_t ne[4];
    size_t nb[4];
} cvattn_tensor;

/* --------------------------------------------------------------------------------------------
 * Flash attention: dst = softmax(scale * Q K^T + mask) V, the ggml_flash_attn_ext contract.
 *   q    f32|f16 [D, n_q, H, B]            (any strides)
 *   k    f32|f16|q8_0|q4_0|q4_1|q5_0|q5_1 [D, n_kv, H_kv, B_k]   (nb0 = element or block size;
 *        a head row of a block type is D/32 consecutive blocks)
 *   v    same type set, [Dv, n_kv, H_kv, B_v]
 *   mask NULL or f16 [>= n_kv, >= n_q, 1|H, 1|B]; row index = local query index; -inf drops a key
 *   dst  f32 contiguous [Dv, H, n_q, B]
 * H % H_kv == 0 and the kv head of q head h is h / (H / H_kv); B % B_k == 0.
 * A query row whose keys are all masked yields 0.  D = Dv = 64 (the head size of every attention
 * site in cosyvoice.cpp); other sizes are reported unsupported.  max_bias and logit_softcap must
 * be 0 (cosyvoice.cpp always passes 0, src/cosyvoice-kv-cache.cpp:383, src/cosyvoice-graph.cpp:375).
 * n_kv is read from k->ne[1] at call time (the reference grows it in place between decode steps,
 * src/cosyvoice-kv-cache.cpp:398-408).
 * -------------------------------------------------------------------------------------------- */

/* Replaces ggml_backend_supports_op(backend, ggml_flash_attn_ext(...)) as used by
 * cosyvoice_check_kv_cache_types, src/cosyvoice-loader.cpp:543-567. */
CVATTN_API int cvattn_supports_flash_attn_ext(const cvattn_tensor *q, const cvattn_tensor *k,
                                              const cvattn_tensor *v, const cvattn_tensor *mask);

/* Bytes of device workspace cvattn_flash_attn_ext needs for these shapes: the partial results
 * of a KV sequence split over several workgroups, and fp16 copies of fp32 K/V that many query
 * row groups read (the DiT call without cache).  0 is a valid answer. */
CVATTN_API size_t cvattn_flash_attn_ext_workspace(const cvattn_tensor *q, const cvattn_tensor *k,
                                                  const cvattn_tensor *v, const cvattn_tensor *mask);

/* Replaces the GGML_OP_FLASH_ATTN_EXT node built by ggml_flash_attn_ext(ctx, q, k, v, mask,
 * scale, max_bias, logit_softcap) + ggml_flash_attn_ext_set_prec(node, prec) at
 * src/cosyvoice-kv-cache.cpp:383-384 and src/cosyvoice-graph.cpp:375-376.  Asynchronous on
 * `stream`; `ws` must hold cvattn_flash_attn_ext_workspace() bytes (may be NULL when that is 0)
 * and be 256-byte aligned (hipMalloc and torch allocations are); else CVATTN_ERR_BAD_ARGS. */
CVATTN_API int cvattn_flash_attn_ext(const cvattn_tensor *q, const cvattn_tensor *k,
                                     const cvattn_tensor *v, const cvattn_tensor *mask,
                                     const cvattn_tensor *dst, float scale, float max_bias,
                                     float logit_softcap, int prec, void *ws, size_t ws_bytes,
                                     cvattn_stream_t stream);

/* cvattn_flash_attn_ext without a caller workspace and without any allocation.  No counterpart
 * in the reference: it is for callers that cannot allocate or pass scratch memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Its workspace is a
 * fixed array of CVATTN_NOALLOC_SCRATCH_BYTES in the library's device memory, one per GPU, held
 * until the process ends; a call whose shapes need more (cvattn_flash_attn_ext_workspace) returns
 * CVATTN_ERR_WORKSPACE_TOO_SMALL.  All calls on one GPU share that array: calls that overlap on
 * one GPU (two streams, or two threads) race and must be serialised by the caller.  Otherwise it
 * behaves exactly as cvattn_flash_attn_ext (same kernels, same results). */
#define CVATTN_NOALLOC_SCRATCH_BYTES (32u << 20)
CVATTN_API int cvattn_flash_attn_ext_noalloc(const cvattn_tensor *q, const cvattn_tensor *k,
                                             const cvattn_tensor *v, const cvattn_tensor *mask,
                                             const cvattn_tensor *dst, float scale, float max_bias,
                                             float logit_softcap, int prec, cvattn_stream_t stream);

/* --------------------------------------------------------------------------------------------
 * Batched flash attention: many independent ggml_flash_attn_ext problems in one launch.
 * cosyvoice.cpp runs one FA node per layer per worker (src/cosyvoice-llm.cpp:247-255,
 * src/cosyvoice-model.cpp:102-107); serving several workers or sequences at once
 * (tools/server/cosyvoice-server.cpp:318-323) gives many such nodes per step.  All problems must
 * share q/k/v/mask presence and types, D/Dv, H, H_kv, n_q and B; n_kv, pointers and strides may
 * differ per problem (ragged KV lengths).
 *   cvattn_fa_batch_workspace   bytes needed for n problems (includes the device problem table);
 *                               the workspace must be 256-byte aligned (else CVATTN_ERR_BAD_ARGS)
 *   cvattn_fa_batch_prepare     validates the problems, uploads the problem table and zeroed
 *                               split counters into ws (one host->device copy on `stream`, then
 *                               waits for it: a set-up call) and fills a host-side plan
 *   cvattn_fa_batch_launch      runs a prepared plan: one kernel launch, split partials merged by
 *                               the last workgroup of each split group (no host->device traffic;
 *                               may be called repeatedly, or captured in a HIP graph, while ws and
 *                               the tensors stay valid; launches sharing one ws must not overlap)
 * -------------------------------------------------------------------------------------------- */
typedef struct cvattn_fa_problem {
    cvattn_tensor q, k, v, mask, dst; /* mask.data == NULL: no mask */
} cvattn_fa_problem;

/* Opaque launch plan filled by cvattn_fa_batch_prepare (caller-owned host memory). */
typedef struct cvattn_fa_plan {
    uint64_t opaque[64];
} cvattn_fa_plan;

CVATTN_API size_t cvattn_fa_batch_workspace(const cvattn_fa_problem *problems, int n);
CVATTN_API int cvattn_fa_batch_prepare(const cvattn_fa_problem *problems, int n, float scale,
                                       void *ws, size_t ws_bytes, cvattn_stream_t stream,
                                       cvattn_fa_plan *plan);
CVATTN_API int cvattn_fa_batch_launch(const cvattn_fa_plan *plan, cvattn_stream_t stream);

/* A prepared batch whose KV lengths live in device memory and are read at every launch: the
 * decode loop of src/cosyvoice-llm.cpp:216-222 reuses one graph and grows n_kv in place with
 * shift_kv_node_pos (src/cosyvoice-kv-cache.cpp:398-408); here one captured HIP graph
 * (cvattn_shift_n_kv + cvattn_fa_batch_launch) serves every token with no re-prepare and no
 * host synchronisation.
 *   n_kv_dev     device int32; problem i reads n_kv_dev[i * n_kv_stride] (stride 0: one length
 *                shared by every problem, e.g. the 24 layers of one sequence; stride 1: one per
 *                problem, e.g. serving sequences).  Values are clamped to [0, capacity].
 *   problems     as for cvattn_fa_batch_prepare, with k/v ne[1] = the capacity (e.g. max_seq):
 *                the token splits are planned for it and each launch spreads the current length
 *                over them; a mask must cover the capacity.
 * The workspace size is cvattn_fa_batch_workspace(problems, n). */
CVATTN_API int cvattn_fa_batch_prepare_dynamic(const cvattn_fa_problem *problems, int n, float scale,
                                               const int32_t *n_kv_dev, int n_kv_stride, void *ws,
                                               size_t ws_bytes, cvattn_stream_t stream, cvattn_fa_plan *plan);
/* n_kv_dev[i] += delta for i < n, as a kernel on `stream` (capturable): the in-graph length
 * update of a dynamic plan. */
CVATTN_API int cvattn_shift_n_kv(int32_t *n_kv_dev, int n, int32_t delta, cvattn_stream_t stream);

/* --------------------------------------------------------------------------------------------
 * The non-flash-attention path (--llm-flash-attn 0 / --flow-flash-attn 0): the node sequence
 *   scores = mul_mat(K, Q) (prec F32) -> soft_max_ext(scores, mask, scale, 0)
 *   -> mul_mat(V^T, weights) -> permute(0, 2, 1, 3) -> cont
 * of src/cosyvoice-kv-cache.cpp:387-395 and src/cosyvoice-graph.cpp:378-388, in one call that
 * never materialises the scores.  V is the transposed cache view that path keeps:
 *   vt   f32/f16 [n_kv, Dv, H_kv, B_v], tokens contiguous (nb0 = element size), nb1 = the dim
 *        stride (src/cosyvoice-kv-cache.cpp:345: view_4d(v, cur_len + n, Dv, heads, batch))
 * q, k, mask, dst, scale and the workspace are as for cvattn_flash_attn_ext (K may be any KV
 * type; the loader keeps V unquantized in this mode, src/cosyvoice-loader.cpp:639-641).  A row
 * whose keys are all masked yields NaN, as ggml's soft_max does.
 * -------------------------------------------------------------------------------------------- */
CVATTN_API int cvattn_supports_attn_nonfa(const cvattn_tensor *q, const cvattn_tensor *k,
                                          const cvattn_tensor *vt, const cvattn_tensor *mask);
CVATTN_API size_t cvattn_attn_nonfa_workspace(const cvattn_tensor *q, const cvattn_tensor *k,
                                              const cvattn_tensor *vt, const cvattn_tensor *mask);
CVATTN_API int cvattn_attn_nonfa(const cvattn_tensor *q, const cvattn_tensor *k, const cvattn_tensor *vt,
                                 const cvattn_tensor *mask, const cvattn_tensor *dst, float scale, void *ws,
                                 size_t ws_bytes, cvattn_stream_t stream);

/* --------------------------------------------------------------------------------------------
 * Block formats.
 * -------------------------------------------------------------------------------------------- */

/* Elements per block (32 for q*, 1 for f16/f32) and bytes per block; 0 for unknown types. */
CVATTN_API int64_t cvattn_block_size(int type);
CVATTN_API int64_t cvattn_type_size(int type);

/* dst[0..n) = dequantized src (ggml's dequantize_row_* for `type`); n % block size == 0.
 * Test entry for the in-register dequantizers the attention kernels use. */
CVATTN_API int cvattn_dequantize(int type, const void *src, float *dst, int64_t n,
                                 cvattn_stream_t stream);

/* --------------------------------------------------------------------------------------------
 * KV write: the GGML_OP_SET_ROWS node of cosyvoice_kv_cache::update_cache
 * (src/cosyvoice-kv-cache.cpp:316,322): dst[:, idx[i], i2, i3] = quantize_ref(src[:, i, i2, i3]).
 *   dst  cache tensor of a KV type, [ne0, rows, ne2, ne3]
 *   src  f32 [ne0, n, ne2, ne3]
 *   idx  i32 [n] (positions; ggml broadcasts a 1-D index over ne2/ne3)
 * Quantization follows ggml's quantize_row_*_ref bit for bit.  With ne0 = 1 it is the element
 * scatter of the transposed V cache: dst/src flattened to [1, N] and idx the v_idxs the host
 * fills (src/cosyvoice-kv-cache.cpp:338-343,357-377).
 * -------------------------------------------------------------------------------------------- */
CVATTN_API int cvattn_supports_set_rows(const cvattn_tensor *dst, const cvattn_tensor *src,
                                        const cvattn_tensor *idx);
CVATTN_API int cvattn_set_rows(const cvattn_tensor *dst, const cvattn_tensor *src,
                               const cvattn_tensor *idx, cvattn_stream_t stream);

/* --------------------------------------------------------------------------------------------
 * Rotary position embedding, ggml_rope_ext with freq_factors NULL, ext_factor 0 and
 * attn_factor 1 -- the forms cosyvoice.cpp builds:
 *   src/cosyvoice-llm.cpp:56-57     Q and K of each Qwen2 layer: NEOX, n_dims = head dim (64),
 *                                   freq_base = rope_theta from the GGUF;
 *   src/cosyvoice-graph.cpp:351-352 DiT query/key rows [1024, 1, T*B]: ggml_rope NORMAL,
 *                                   n_dims = 64 (only the first 64 of 1024 dims), base 10000.
 * Pair k < n_dims/2 is (2k, 2k+1) for NORMAL and (k, k + n_dims/2) for NEOX; its angle is
 * p * s^k * freq_scale with s = powf(freq_base, -2/n_dims) (taken on the host, then applied by
 * repeated float multiplication, as ggml's CPU backend does); dims from n_dims on are copied.
 * -------------------------------------------------------------------------------------------- */
#define CVATTN_ROPE_NORMAL 0
#define CVATTN_ROPE_NEOX 2

/* dst = rope(src): src/dst f32 [ne0, ne1, ne2, ne3] (any strides, nb0 = 4), pos i32 [ne2]
 * (the position of each i2, as ggml_rope_ext takes it).  dst may alias src exactly. */
CVATTN_API int cvattn_rope(const cvattn_tensor *dst, const cvattn_tensor *src, const cvattn_tensor *pos,
                           int n_dims, int mode, float freq_base, float freq_scale, cvattn_stream_t stream);

/* The KV write with RoPE fused in front: cvattn_set_rows(dst, rope(src), idx) without the
 * intermediate tensor.  This is cosyvoice_kv_cache::update_cache (src/cosyvoice-kv-cache.cpp:
 * 316,322) fed by the K rope of the same layer (src/cosyvoice-llm.cpp:57,
 * src/cosyvoice-graph.cpp:352).  src is in the set_rows layout, f32 [ne0, n, ne2, ne3]; each row
 * is ne0/head rope inputs of `head` elements (head 64 for the LLM's H_kv heads, 1024 for the DiT
 * row that ggml_rope sees as one head).  pos is i32, contiguous, one position per source row:
 * row (i1, i2, i3) takes pos[i1 + n*(i2 + ne2*i3)] -- the flattened position_ids the callers pass
 * to both ops.  dst and idx follow cvattn_set_rows. */
CVATTN_API int cvattn_rope_set_rows(const cvattn_tensor *dst, const cvattn_tensor *src, const cvattn_tensor *idx,
                                    const cvattn_tensor *pos, int64_t head, int n_dims, int mode, float freq_base,
                                    float freq_scale, cvattn_stream_t stream);

/* --------------------------------------------------------------------------------------------
 * DiT streaming KV cache (cosyvoice_kv_cache as the flow decoder uses it,
 * src/cosyvoice-kv-cache.cpp:45-146,148-290,398-467, built at src/cosyvoice-loader.cpp:1011-1029;
 * driven by the slot schedule of src/cosyvoice-token2wav.cpp:101-167,265-420).
 *
 * Slots: each cached ODE step keeps its own K/V (the DiT input differs per step).  n_slots
 * device slots hold layers x {K, V} of [H*D, max_seq, batch] (V transposed to
 * [max_seq, H*D, batch] when flash_attn is 0), slot-major, each tensor 256-byte aligned; slot 0
 * is the staging slot of the offloadable steps, whose K/V rows move to pinned host slots between
 * uses.  The caller allocates both buffers (sizes from the *_bytes calls) and keeps them for the
 * cache's lifetime; the cache object itself only records layout and state.
 * -------------------------------------------------------------------------------------------- */
typedef struct cvattn_dit_cache cvattn_dit_cache;

typedef struct cvattn_dit_cache_params {
    int32_t layers;          /* DiT transformer blocks (22) */
    int32_t heads;           /* attention heads = kv heads (16) */
    int32_t head_dim;        /* 64 */
    int32_t max_seq;         /* dit_kv_cache_length */
    int32_t batch;           /* 2: the CFG pair */
    int32_t k_type, v_type;  /* ggml type codes of the cache */
    int32_t n_slots;         /* device slots: fixed slots + (offloadable slots ? 1 : 0) */
    int32_t n_host_slots;    /* offloadable slots (host copies) */
    int32_t flash_attn;      /* 1: V rows like K; 0: V transposed (non-flash-attention path) */
} cvattn_dit_cache_params;

CVATTN_API size_t cvattn_dit_cache_device_bytes(const cvattn_dit_cache_params *p);
CVATTN_API size_t cvattn_dit_cache_host_bytes(const cvattn_dit_cache_params *p);
/* Creates the cache over device_buf (device memory) and host_buf (pinned host memory, may be
 * NULL when n_host_slots is 0).  Slot 0 is bound and the cached length is 0. */
CVATTN_API int cvattn_dit_cache_create(const cvattn_dit_cache_params *p, void *device_buf, size_t device_bytes,
                                       void *host_buf, size_t host_bytes, cvattn_dit_cache **out);
CVATTN_API void cvattn_dit_cache_destroy(cvattn_dit_cache *c);

/* bind_slot (kv-cache.cpp:415-420), slide_kv_slot (:422-465: the next slot takes over the
 * views; flash attention only), and the cached length cur_len. */
CVATTN_API int cvattn_dit_cache_bind_slot(cvattn_dit_cache *c, int slot);
CVATTN_API int cvattn_dit_cache_slide(cvattn_dit_cache *c);
CVATTN_API int cvattn_dit_cache_slot(const cvattn_dit_cache *c);
CVATTN_API int cvattn_dit_cache_set_len(cvattn_dit_cache *c, uint32_t cur_len);
CVATTN_API uint32_t cvattn_dit_cache_len(const cvattn_dit_cache *c);

/* The bound slot's tensors of one layer, as update_cache uses them (kv-cache.cpp:309-355):
 *   k_cache, v_cache  the whole cache tensors (set_rows targets; with flash_attn 0, v_cache is
 *                     the transposed tensor [max_seq, H*D, batch] -- flatten it to [1, N] for
 *                     the v_idxs scatter);
 *   k_view, v_view    the attention views over n_kv = cur_len + n_new tokens: [D, n_kv, H, B]
 *                     for K (and V with flash attention), [n_kv, D, H, B] for the transposed V.
 * Any output pointer may be NULL. */
CVATTN_API int cvattn_dit_cache_layer(const cvattn_dit_cache *c, int layer, int64_t n_kv, cvattn_tensor *k_cache,
                                      cvattn_tensor *v_cache, cvattn_tensor *k_view, cvattn_tensor *v_view);

/* offload_slot / load_slot (kv-cache.cpp:148-246,276-290): asynchronous copies of the first
 * n_tokens rows of every layer's K and V of the bound slot to host slot `host_slot`, and back
 * (load sets cur_len to the stored length).  The host layout per slot is layer-major,
 * {K of batch 0..B-1, V of batch 0..B-1} of n_tokens rows each (the transposed V as its
 * [n_tokens, H*D] block per batch).  Ordered on `stream`; the host data is complete after it. */
CVATTN_API int cvattn_dit_cache_offload(cvattn_dit_cache *c, int host_slot, uint32_t n_tokens,
                                        cvattn_stream_t stream);
CVATTN_API int cvattn_dit_cache_load(cvattn_dit_cache *c, int host_slot, cvattn_stream_t stream);

/* The DiT step inputs the host fills before each graph compute (token2wav.cpp:273-302), built
 * on the device:
 *   cvattn_fill_positions  pos i32 [n, B] contiguous: pos[b][j] = j + base (base = cur_len for
 *                          cached steps, 0 otherwise);
 *   cvattn_chunk_mask      f16 mask [n_cols, n_rows]: row i sees keys j < the first chunk
 *                          boundary greater than i (n_cols if none), -inf beyond; bounds sorted
 *                          ascending, at most CVATTN_MAX_CHUNK_BOUNDS of them;
 *   cvattn_v_idxs          the element-scatter index of the transposed V write, as
 *                          set_input_v_idxs builds it (kv-cache.cpp:357-377), from the device
 *                          positions pos[0..n_per_batch): idx i32 [n_embd * n_tokens]. */
#define CVATTN_MAX_CHUNK_BOUNDS 256
CVATTN_API int cvattn_fill_positions(const cvattn_tensor *pos, int32_t base, cvattn_stream_t stream);
CVATTN_API int cvattn_chunk_mask(const cvattn_tensor *mask, const uint32_t *bounds, int n_bounds,
                                 cvattn_stream_t stream);
CVATTN_API int cvattn_v_idxs(int32_t *idx, const int32_t *pos, uint32_t n_tokens, uint32_t n_per_batch,
                             uint32_t n_embd, uint32_t max_seq, cvattn_stream_t stream);

/* The per-ODE-step plan of a streaming (or one-shot) token2wav call, dit_sched_config
 * (token2wav.cpp:101-167), with the device slot each step computes on and the host slot it loads
 * or offloads (the bind/slide and offload counters of token2wav.cpp:352-412 replayed):
 *   slot       device slot bound while the step runs (-1: no cache)
 *   host_slot  host slot loaded before / offloaded after the step (-1: none) */
typedef struct cvattn_dit_step {
    int32_t rebuild, cache_kv, load, offload, slide, slice, mask;
    int32_t slot, host_slot;
    int64_t cut_len;
} cvattn_dit_step;
CVATTN_API int cvattn_dit_schedule(int n_steps, int n_fixed_slots, int n_offloadable_slots, int64_t cut_len,
                                   uint32_t offset, int streaming, int kv_slidable, cvattn_dit_step *out);

/* Human-readable name of a status code. */
CVATTN_API const char *cvattn_status_string(int status);

#ifdef __cplusplus
}
#endif
#endif
