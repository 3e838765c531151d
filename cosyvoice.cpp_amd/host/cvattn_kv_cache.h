// cvattn_kv_cache.h -- the KV cache class of cosyvoice.cpp (cosyvoice_kv_cache,
// src/cosyvoice-kv-cache.h:9-69) on the engine's C ABI, for C++ hosts.
//
// The methods keep the reference's names, argument order and meaning.  Where the reference
// builds ggml graph nodes, the methods here run the work on `stream` at once.  The engine's
// cvattn_tensor stands in for ggml_tensor: it has the same data/type/ne/nb fields.
//
// Two things differ from the reference.
//   - Errors.  The reference aborts on a failed GGML_ASSERT.  Here every method returns an
//     engine status code (CVATTN_OK, or a cvattn_status_string() code).
//   - State.  The reference re-points graph views between calls (shift_kv_node_pos,
//     slide_kv_slot).  Here the views are rebuilt from cur_len and the bound slot at every
//     update_cache, so those two methods only change that state.
//
// LLM prefill/decode step (src/cosyvoice-llm.cpp:31-76,95-299), one call pair per layer:
//     cache.update_cache(k, v, position_ids, layer, stream);  // k, v now hold the cache views
//     cache.attention_forward(q, k, v, mask, out, stream);
// After the last layer, advance cur_len.  There are two ways, as in the reference:
//     cache.cur_len += n;                // after building a graph (llm.cpp:197,299)
//     cache.shift_kv_node_pos(n);        // flash attention, reusing a graph (llm.cpp:124,221)
// In the non-flash mode, call set_input_v_idxs(positions, n, n) before the layers.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "../../include/cvattn.h"

namespace cvattn {

class kv_cache {
public:
    kv_cache() = default;
    ~kv_cache();
    kv_cache(const kv_cache &) = delete;
    kv_cache &operator=(const kv_cache &) = delete;

    // build_kv_cache (src/cosyvoice-kv-cache.cpp:45-117).  Each layer of each of the n_slots
    // device slots holds K [k_head_dim*H_kv, max_seq, batch].  V has the same shape, transposed
    // to [max_seq, v_head_dim*H_kv, batch] when fattn is false.  There are also
    // n_offloaded_kv_slots pinned host slots.  Allocates the device memory with hipMalloc and the
    // host slots with hipHostMalloc, as the reference allocates its backend buffer.  The caches
    // of cosyvoice.cpp have k_head_dim == v_head_dim == 64 (src/cosyvoice-loader.cpp:995-1028).
    int build_kv_cache(int layers, int k_head_dim, int v_head_dim, int num_key_value_heads, uint32_t max_seq,
                       int k_type, int v_type, int batch_size, int n_kv_slots, int n_offloaded_kv_slots, bool fattn);

    // update_cache (src/cosyvoice-kv-cache.cpp:309-355).
    //   k, v          in: the new rows, f32 [head_dim, H_kv, n, batch] (nb0 = 4, heads adjacent:
    //                 nb1 = 4 * head_dim).
    //                 out: the attention views of the layer over cur_len + n tokens,
    //                 [head_dim, n_kv, H_kv, batch].  In the non-flash mode, v is the transposed
    //                 view [n_kv, head_dim, H_kv, batch].
    //   position_ids  i32 [n], or [n, batch] (one row per batch), on the device.
    // The rows go into layer layer_idx of the bound slot.  In the flash mode they are written
    // with set_rows.  In the non-flash mode, K is written with set_rows and V with the element
    // scatter through the index that set_input_v_idxs built.
    int update_cache(cvattn_tensor &k, cvattn_tensor &v, const cvattn_tensor &position_ids, int layer_idx,
                     cvattn_stream_t stream);

    // update_cache with the layer's K rope fused in front.  k holds the rows before the rope.
    // The rope positions are position_ids, which must be contiguous: each row (i, b) of k rotates
    // at position_ids[i + n*b].  Each row of k is ne0*H_kv/rope_head rope inputs of rope_head
    // elements.  The two call sites of the reference:
    //   - LLM (src/cosyvoice-llm.cpp:57): NEOX, rope_head = n_dims = head_dim.
    //   - DiT (src/cosyvoice-graph.cpp:352): NORMAL, rope_head = 1024, n_dims = 64.
    int update_cache_rope(cvattn_tensor &k, cvattn_tensor &v, const cvattn_tensor &position_ids, int layer_idx,
                          int64_t rope_head, int n_dims, int mode, float freq_base, float freq_scale,
                          cvattn_stream_t stream);

    // set_input_v_idxs (src/cosyvoice-kv-cache.cpp:357-377).  Builds the element-scatter index of
    // the transposed V write on the device.  positions[0 .. n_tokens_per_batch) are the
    // positions on the device (the reference takes host positions and uploads the whole index).
    // Does nothing in the flash mode.
    int set_input_v_idxs(const int32_t *positions, uint32_t n_tokens, uint32_t n_tokens_per_batch,
                         cvattn_stream_t stream);

    // attention_forward (src/cosyvoice-kv-cache.cpp:379-396).  Attention of query_states
    // [head_dim, n_q, H, batch] (any strides) over the views that update_cache returned, with
    // scale 1/sqrt(head_dim).  The flash mode uses cvattn_flash_attn_ext.  The non-flash mode
    // uses cvattn_attn_nonfa (the mul_mat -> soft_max -> mul_mat sequence).
    //   attention_mask  f16 [>= n_kv, >= n_q, ...], or nullptr.
    //   dst             f32 contiguous [head_dim, H, n_q, batch]: the layout of both of the
    //                   reference's outputs.
    // The split workspace grows on demand and is kept for later calls.
    int attention_forward(const cvattn_tensor &query_states, const cvattn_tensor &key_states,
                          const cvattn_tensor &value_states, const cvattn_tensor *attention_mask,
                          const cvattn_tensor &dst, cvattn_stream_t stream);

    // shift_kv_node_pos (:398-408): cur_len += shift_pos.  Flash attention only.
    int shift_kv_node_pos(uint32_t shift_pos);
    bool can_reuse() const { return fattn_; }
    // bind_slot (:415-420): false for a slot past the last.
    bool bind_slot(int slot_idx);
    // slide_kv_slot (:422-465): binds the next slot.  Flash attention only.
    int slide_kv_slot();

    // offload_slot / load_slot (:276-290), and offload_cache / load_cache (:148-246) on host
    // slot 0, as the LLM uses them (src/cosyvoice-model.cpp:586-601).  Asynchronous copies on
    // `stream` of the first n_tokens rows of every layer of the bound slot, to a host slot and
    // back.  load_slot sets cur_len to the stored length.  The host data is complete once the
    // stream reaches the copy.  The reference offloads slot 0 whatever slot is bound; its
    // callers bind slot 0 first (src/cosyvoice-token2wav.cpp:389).
    int offload_slot(int offloaded_slot_idx, uint32_t n_tokens, cvattn_stream_t stream);
    int load_slot(int offloaded_slot_idx, cvattn_stream_t stream);
    int offload_cache(uint32_t n_tokens, cvattn_stream_t stream) { return offload_slot(0, n_tokens, stream); }
    int load_cache(cvattn_stream_t stream) { return load_slot(0, stream); }
    // Bytes of the stored rows in the host slots.  The host slots themselves stay allocated until
    // destruction (pinned memory).
    size_t get_offloaded_cache_size() const;
    // Forgets the stored rows: a later load_slot sets cur_len to 0 and copies nothing.
    void clear_offloaded_cache();

    // The bound slot's cache tensors and its views over n_kv tokens for one layer.  For hosts that
    // drive the engine directly, and for tests.
    int layer_tensors(int layer_idx, int64_t n_kv, cvattn_tensor *k_cache, cvattn_tensor *v_cache,
                      cvattn_tensor *k_view, cvattn_tensor *v_view) const;
    int slot() const { return cache_ ? cvattn_dit_cache_slot(cache_) : -1; }
    bool fattn() const { return fattn_; }

    uint32_t cur_len = 0;

private:
    struct rope_spec {
        int64_t head;
        int n_dims, mode;
        float freq_base, freq_scale;
    };
    int update(cvattn_tensor &k, cvattn_tensor &v, const cvattn_tensor &position_ids, int layer_idx,
               const rope_spec *rope, cvattn_stream_t stream);
    void release();
    int rows_src(const cvattn_tensor &x, cvattn_tensor *src) const;
    int write_v(const cvattn_tensor &v, const cvattn_tensor &position_ids, int layer_idx, cvattn_stream_t stream);
    int views(cvattn_tensor &k, cvattn_tensor &v, int64_t n, int layer_idx) const;

    cvattn_dit_cache *cache_ = nullptr;
    cvattn_dit_cache_params p_{};
    void *dev_ = nullptr;    // slots (hipMalloc)
    void *host_ = nullptr;   // host slots (hipHostMalloc)
    void *ws_ = nullptr;     // split partials of attention_forward
    size_t ws_bytes_ = 0;
    int32_t *vidx_ = nullptr; // v_idxs: max_seq * batch * n_embd entries (non-flash mode)
    uint32_t vidx_count_ = 0; // entries the last set_input_v_idxs built
    std::vector<uint32_t> host_len_;
    size_t host_row_bytes_ = 0; // host bytes per stored token (all layers, K and V, all batches)
    bool fattn_ = true;
};

} // namespace cvattn
