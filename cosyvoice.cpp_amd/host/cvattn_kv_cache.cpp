// cvattn_kv_cache.cpp -- cvattn::kv_cache, the cosyvoice_kv_cache mirror
// (src/cosyvoice-kv-cache.cpp).  Host code over the engine's C ABI.  The slot layout, views and
// offload copies are the engine's cvattn_dit_cache.  The device work is cvattn_set_rows /
// cvattn_rope_set_rows / cvattn_v_idxs / cvattn_flash_attn_ext / cvattn_attn_nonfa.
#include "cvattn_kv_cache.h"

#include <hip/hip_runtime_api.h>

#include <cmath>

namespace cvattn {

namespace {

constexpr size_t kWorkspaceQuantum = size_t(1) << 20;

bool is_f32_rows(const cvattn_tensor &x) {
    return x.type == CVATTN_TYPE_F32 && x.nb[0] == 4 && x.nb[1] == 4 * (size_t)x.ne[0];
}

} // namespace

kv_cache::~kv_cache() { release(); }

void kv_cache::release() {
    if (cache_) cvattn_dit_cache_destroy(cache_);
    cache_ = nullptr;
    // device buffers may still be read by queued work on any stream
    if (dev_ || ws_ || vidx_ || host_) (void)hipDeviceSynchronize();
    if (dev_) (void)hipFree(dev_);
    if (ws_) (void)hipFree(ws_);
    if (vidx_) (void)hipFree(vidx_);
    if (host_) (void)hipHostFree(host_);
    dev_ = host_ = ws_ = nullptr;
    vidx_ = nullptr;
    ws_bytes_ = 0;
    vidx_count_ = 0;
    host_len_.clear();
    cur_len = 0;
}

int kv_cache::build_kv_cache(int layers, int k_head_dim, int v_head_dim, int num_key_value_heads, uint32_t max_seq,
                             int k_type, int v_type, int batch_size, int n_kv_slots, int n_offloaded_kv_slots,
                             bool fattn) {
    release();
    // the engine's attention takes equal K and V head sizes (64 at every site of cosyvoice.cpp)
    if (k_head_dim != v_head_dim) return CVATTN_ERR_UNSUPPORTED;
    if (max_seq == 0 || max_seq > (uint32_t)INT32_MAX) return CVATTN_ERR_BAD_ARGS;
    cvattn_dit_cache_params p{};
    p.layers = layers;
    p.heads = num_key_value_heads;
    p.head_dim = k_head_dim;
    p.max_seq = (int32_t)max_seq;
    p.batch = batch_size;
    p.k_type = k_type;
    p.v_type = v_type;
    p.n_slots = n_kv_slots;
    p.n_host_slots = n_offloaded_kv_slots;
    p.flash_attn = fattn ? 1 : 0;
    const size_t dev_bytes = cvattn_dit_cache_device_bytes(&p);
    if (!dev_bytes) {
        // the same checks give the reason
        cvattn_dit_cache *probe = nullptr;
        int rc = cvattn_dit_cache_create(&p, nullptr, 0, nullptr, 0, &probe);
        return rc ? rc : CVATTN_ERR_BAD_ARGS;
    }
    const size_t host_bytes = cvattn_dit_cache_host_bytes(&p);
    if (hipMalloc(&dev_, dev_bytes) != hipSuccess) {
        dev_ = nullptr;
        return CVATTN_ERR_HIP;
    }
    if (host_bytes && hipHostMalloc(&host_, host_bytes, hipHostMallocDefault) != hipSuccess) {
        host_ = nullptr;
        release();
        return CVATTN_ERR_HIP;
    }
    int rc = cvattn_dit_cache_create(&p, dev_, dev_bytes, host_, host_bytes, &cache_);
    if (rc) {
        release();
        return rc;
    }
    if (!fattn) {
        // the largest index set_input_v_idxs builds: every position of every batch entry
        const size_t n = (size_t)max_seq * (size_t)batch_size * (size_t)num_key_value_heads * (size_t)v_head_dim;
        if (n > (size_t)UINT32_MAX || hipMalloc((void **)&vidx_, n * sizeof(int32_t)) != hipSuccess) {
            vidx_ = nullptr;
            release();
            return CVATTN_ERR_HIP;
        }
    }
    p_ = p;
    fattn_ = fattn;
    host_len_.assign((size_t)n_offloaded_kv_slots, 0u);
    host_row_bytes_ = max_seq ? host_bytes / (n_offloaded_kv_slots ? (size_t)n_offloaded_kv_slots : 1) / max_seq : 0;
    cur_len = 0;
    return CVATTN_OK;
}

// x f32 [head_dim, H_kv, n, batch] with the heads of a token adjacent, as the set_rows source
// [head_dim*H_kv, n, batch] (the reshape of src/cosyvoice-kv-cache.cpp:315).
int kv_cache::rows_src(const cvattn_tensor &x, cvattn_tensor *src) const {
    if (!is_f32_rows(x)) return CVATTN_ERR_UNSUPPORTED;
    if (x.ne[0] != p_.head_dim || x.ne[1] != p_.heads || x.ne[3] != p_.batch || x.ne[2] < 0)
        return CVATTN_ERR_BAD_ARGS;
    src->data = x.data;
    src->type = CVATTN_TYPE_F32;
    src->ne[0] = x.ne[0] * x.ne[1];
    src->ne[1] = x.ne[2];
    src->ne[2] = x.ne[3];
    src->ne[3] = 1;
    src->nb[0] = 4;
    src->nb[1] = x.nb[2];
    src->nb[2] = x.nb[3];
    src->nb[3] = x.nb[3] * (size_t)x.ne[3];
    return CVATTN_OK;
}

int kv_cache::views(cvattn_tensor &k, cvattn_tensor &v, int64_t n, int layer_idx) const {
    return cvattn_dit_cache_layer(cache_, layer_idx, (int64_t)cur_len + n, nullptr, nullptr, &k, &v);
}

int kv_cache::write_v(const cvattn_tensor &v, const cvattn_tensor &position_ids, int layer_idx,
                      cvattn_stream_t stream) {
    cvattn_tensor v_cache;
    int rc = cvattn_dit_cache_layer(cache_, layer_idx, 0, nullptr, &v_cache, nullptr, nullptr);
    if (rc) return rc;
    cvattn_tensor src;
    rc = rows_src(v, &src);
    if (rc) return rc;
    if (fattn_) return cvattn_set_rows(&v_cache, &src, &position_ids, stream);
    // transposed V: both sides flattened to [1, N], each element scattered to its own index
    // (src/cosyvoice-kv-cache.cpp:326-343)
    const int64_t n_src = src.ne[0] * src.ne[1] * src.ne[2];
    if (src.nb[2] != src.nb[1] * (size_t)src.ne[1]) return CVATTN_ERR_UNSUPPORTED; // ggml_reshape needs contiguity
    if ((uint64_t)n_src != vidx_count_) return CVATTN_ERR_BAD_ARGS; // set_input_v_idxs built another size
    const int64_t n_dst = v_cache.ne[0] * v_cache.ne[1] * v_cache.ne[2];
    const size_t es = v_cache.nb[0];
    const cvattn_tensor dst = {v_cache.data, v_cache.type, {1, n_dst, 1, 1}, {es, es, es * n_dst, es * n_dst}};
    const cvattn_tensor flat = {src.data, CVATTN_TYPE_F32, {1, n_src, 1, 1}, {4, 4, 4 * (size_t)n_src, 4 * (size_t)n_src}};
    const cvattn_tensor idx = {vidx_, CVATTN_TYPE_I32, {n_src, 1, 1, 1},
                               {4, 4 * (size_t)n_src, 4 * (size_t)n_src, 4 * (size_t)n_src}};
    return cvattn_set_rows(&dst, &flat, &idx, stream);
}

// update_cache and update_cache_rope: K (rotated on the way when rope is set), then V, then the
// views over cur_len + n tokens.
int kv_cache::update(cvattn_tensor &k, cvattn_tensor &v, const cvattn_tensor &position_ids, int layer_idx,
                     const rope_spec *rope, cvattn_stream_t stream) {
    if (!cache_) return CVATTN_ERR_BAD_ARGS;
    for (int i = 0; i < 4; i++) // ggml_are_same_shape(k, v)
        if (k.ne[i] != v.ne[i]) return CVATTN_ERR_BAD_ARGS;
    const int64_t n = position_ids.ne[0];
    if (n != k.ne[2] || (int64_t)cur_len + n > p_.max_seq) return CVATTN_ERR_BAD_ARGS;
    cvattn_tensor k_cache, src;
    int rc = cvattn_dit_cache_layer(cache_, layer_idx, 0, &k_cache, nullptr, nullptr, nullptr);
    if (rc) return rc;
    rc = rows_src(k, &src);
    if (rc) return rc;
    rc = rope ? cvattn_rope_set_rows(&k_cache, &src, &position_ids, &position_ids, rope->head, rope->n_dims, rope->mode,
                                     rope->freq_base, rope->freq_scale, stream)
              : cvattn_set_rows(&k_cache, &src, &position_ids, stream);
    if (rc) return rc;
    rc = write_v(v, position_ids, layer_idx, stream);
    if (rc) return rc;
    return views(k, v, n, layer_idx);
}

int kv_cache::update_cache(cvattn_tensor &k, cvattn_tensor &v, const cvattn_tensor &position_ids, int layer_idx,
                           cvattn_stream_t stream) {
    return update(k, v, position_ids, layer_idx, nullptr, stream);
}

int kv_cache::update_cache_rope(cvattn_tensor &k, cvattn_tensor &v, const cvattn_tensor &position_ids, int layer_idx,
                                int64_t rope_head, int n_dims, int mode, float freq_base, float freq_scale,
                                cvattn_stream_t stream) {
    const rope_spec r = {rope_head, n_dims, mode, freq_base, freq_scale};
    return update(k, v, position_ids, layer_idx, &r, stream);
}

int kv_cache::set_input_v_idxs(const int32_t *positions, uint32_t n_tokens, uint32_t n_tokens_per_batch,
                               cvattn_stream_t stream) {
    if (!cache_) return CVATTN_ERR_BAD_ARGS;
    if (fattn_) return CVATTN_OK; // the reference builds no index in this mode
    const uint64_t n_embd = (uint64_t)p_.heads * (uint64_t)p_.head_dim;
    if ((uint64_t)n_tokens * n_embd > (uint64_t)p_.max_seq * (uint64_t)p_.batch * n_embd) return CVATTN_ERR_BAD_ARGS;
    int rc = cvattn_v_idxs(vidx_, positions, n_tokens, n_tokens_per_batch, (uint32_t)n_embd, (uint32_t)p_.max_seq,
                           stream);
    if (rc) return rc;
    vidx_count_ = (uint32_t)((uint64_t)n_tokens * n_embd);
    return CVATTN_OK;
}

int kv_cache::attention_forward(const cvattn_tensor &query_states, const cvattn_tensor &key_states,
                                const cvattn_tensor &value_states, const cvattn_tensor *attention_mask,
                                const cvattn_tensor &dst, cvattn_stream_t stream) {
    if (!cache_) return CVATTN_ERR_BAD_ARGS;
    const float scale = 1.0f / std::sqrt((float)key_states.ne[0]);
    const size_t need = fattn_ ? cvattn_flash_attn_ext_workspace(&query_states, &key_states, &value_states, attention_mask)
                               : cvattn_attn_nonfa_workspace(&query_states, &key_states, &value_states, attention_mask);
    if (need > ws_bytes_) {
        // the old workspace may still be read by queued work
        if (ws_) {
            (void)hipDeviceSynchronize();
            (void)hipFree(ws_);
            ws_ = nullptr;
            ws_bytes_ = 0;
        }
        const size_t bytes = (need + kWorkspaceQuantum - 1) / kWorkspaceQuantum * kWorkspaceQuantum;
        if (hipMalloc(&ws_, bytes) != hipSuccess) {
            ws_ = nullptr;
            return CVATTN_ERR_HIP;
        }
        ws_bytes_ = bytes;
    }
    if (fattn_)
        return cvattn_flash_attn_ext(&query_states, &key_states, &value_states, attention_mask, &dst, scale, 0.0f, 0.0f,
                                     CVATTN_PREC_F32, ws_, ws_bytes_, stream);
    return cvattn_attn_nonfa(&query_states, &key_states, &value_states, attention_mask, &dst, scale, ws_, ws_bytes_,
                             stream);
}

int kv_cache::shift_kv_node_pos(uint32_t shift_pos) {
    if (!fattn_) return CVATTN_ERR_UNSUPPORTED; // GGML_ASSERT(fattn)
    if ((uint64_t)cur_len + shift_pos > (uint64_t)p_.max_seq) return CVATTN_ERR_BAD_ARGS;
    cur_len += shift_pos;
    return CVATTN_OK;
}

bool kv_cache::bind_slot(int slot_idx) { return cache_ && cvattn_dit_cache_bind_slot(cache_, slot_idx) == CVATTN_OK; }

int kv_cache::slide_kv_slot() { return cache_ ? cvattn_dit_cache_slide(cache_) : CVATTN_ERR_BAD_ARGS; }

int kv_cache::offload_slot(int offloaded_slot_idx, uint32_t n_tokens, cvattn_stream_t stream) {
    if (!cache_) return CVATTN_ERR_BAD_ARGS;
    int rc = cvattn_dit_cache_offload(cache_, offloaded_slot_idx, n_tokens, stream);
    if (rc) return rc;
    host_len_[(size_t)offloaded_slot_idx] = n_tokens;
    return CVATTN_OK;
}

int kv_cache::load_slot(int offloaded_slot_idx, cvattn_stream_t stream) {
    if (!cache_ || offloaded_slot_idx < 0 || (size_t)offloaded_slot_idx >= host_len_.size()) return CVATTN_ERR_BAD_ARGS;
    if (host_len_[(size_t)offloaded_slot_idx] == 0) { // nothing stored (load_cache returns early on 0)
        cur_len = 0;
        return CVATTN_OK;
    }
    int rc = cvattn_dit_cache_load(cache_, offloaded_slot_idx, stream);
    if (rc) return rc;
    cur_len = cvattn_dit_cache_len(cache_);
    return CVATTN_OK;
}

size_t kv_cache::get_offloaded_cache_size() const {
    size_t n = 0;
    for (uint32_t len : host_len_) n += (size_t)len * host_row_bytes_;
    return n;
}

void kv_cache::clear_offloaded_cache() {
    for (uint32_t &len : host_len_) len = 0;
}

int kv_cache::layer_tensors(int layer_idx, int64_t n_kv, cvattn_tensor *k_cache, cvattn_tensor *v_cache,
                            cvattn_tensor *k_view, cvattn_tensor *v_view) const {
    if (!cache_) return CVATTN_ERR_BAD_ARGS;
    return cvattn_dit_cache_layer(cache_, layer_idx, n_kv, k_cache, v_cache, k_view, v_view);
}

} // namespace cvattn
