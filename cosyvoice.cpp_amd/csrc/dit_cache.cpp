// dit_cache.cpp -- the DiT streaming KV cache of include/cvattn.h: slot layout over caller-owned
// device / pinned host buffers, slot binding and sliding, asynchronous offload/load of a slot's
// rows, the device-built step inputs (positions, chunk mask, v_idxs) and the per-step plan of a
// token2wav call.  Host code only; the copies are HIP async copies on the caller's stream.
//
// Reference: cosyvoice_kv_cache (src/cosyvoice-kv-cache.cpp:45-146 layout, :148-290 offload and
// load, :398-467 slots) as built for the flow decoder (src/cosyvoice-loader.cpp:1011-1029), and
// the schedule / slot bookkeeping of src/cosyvoice-token2wav.cpp:101-167,265-420.
#include "../../include/cvattn.h"

#include <hip/hip_runtime.h>

#include <cstring>
#include <new>
#include <vector>

#include "cvattn_common.h"
#include "cvattn_launch.h"

using namespace cvattn;

namespace {

constexpr size_t kTensorAlign = 256;

size_t align_to(size_t x, size_t a) { return (x + a - 1) / a * a; }

bool cache_type_ok(int t) {
    return t == T_F32 || t == T_F16 || t == T_Q8_0 || t == T_Q4_0 || t == T_Q4_1 || t == T_Q5_0 || t == T_Q5_1;
}

// bytes of n elements of type t (n a multiple of the block size)
size_t row_size(int t, int64_t n) { return (size_t)(n / type_block(t)) * (size_t)type_bytes(t); }

int check_params(const cvattn_dit_cache_params *p) {
    if (!p) return CVATTN_ERR_BAD_ARGS;
    if (p->layers <= 0 || p->heads <= 0 || p->head_dim <= 0 || p->max_seq <= 0 || p->batch <= 0) return CVATTN_ERR_BAD_ARGS;
    if (p->n_slots <= 0 || p->n_host_slots < 0) return CVATTN_ERR_BAD_ARGS;
    if (p->n_host_slots > 0 && p->n_slots < 1) return CVATTN_ERR_BAD_ARGS;
    if (!cache_type_ok(p->k_type) || !cache_type_ok(p->v_type)) return CVATTN_ERR_UNSUPPORTED;
    const int64_t e = (int64_t)p->heads * p->head_dim;
    if (e % type_block(p->k_type) || e % type_block(p->v_type)) return CVATTN_ERR_BAD_ARGS;
    // the transposed V of the non-flash path is kept unquantized (src/cosyvoice-loader.cpp:639-641)
    if (!p->flash_attn && p->v_type != T_F32 && p->v_type != T_F16) return CVATTN_ERR_UNSUPPORTED;
    return CVATTN_OK;
}

struct Layout {
    size_t k_row;     // bytes of one token row of K (H*D elements)
    size_t v_row;     // bytes of one token row of V (flash attention)
    size_t v_es;      // element bytes of the transposed V
    size_t k_bytes, v_bytes, k_al, v_al;
    size_t host_layer; // host bytes per layer per slot at capacity (max_seq tokens)
};

Layout layout_of(const cvattn_dit_cache_params *p) {
    Layout L;
    const int64_t e = (int64_t)p->heads * p->head_dim;
    L.k_row = row_size(p->k_type, e);
    L.v_row = p->flash_attn ? row_size(p->v_type, e) : 0;
    L.v_es = (size_t)type_bytes(p->v_type);
    L.k_bytes = L.k_row * (size_t)p->max_seq * (size_t)p->batch;
    L.v_bytes = p->flash_attn ? L.v_row * (size_t)p->max_seq * (size_t)p->batch
                              : L.v_es * (size_t)p->max_seq * (size_t)e * (size_t)p->batch;
    L.k_al = align_to(L.k_bytes, kTensorAlign);
    L.v_al = align_to(L.v_bytes, kTensorAlign);
    L.host_layer = L.k_bytes + L.v_bytes;
    return L;
}

int hip_rc(hipError_t e) { return e == hipSuccess ? CVATTN_OK : CVATTN_ERR_HIP; }

} // namespace

struct cvattn_dit_cache {
    cvattn_dit_cache_params p;
    Layout L;
    uint8_t *dev;
    uint8_t *host;
    int slot;
    uint32_t cur_len;
    std::vector<uint32_t> host_len; // tokens stored per host slot

    uint8_t *k_tensor(int s, int layer) const { return dev + ((size_t)s * p.layers + layer) * (L.k_al + L.v_al); }
    uint8_t *v_tensor(int s, int layer) const { return k_tensor(s, layer) + L.k_al; }
    uint8_t *host_layer(int h, int layer) const {
        return host + ((size_t)h * p.layers + layer) * L.host_layer;
    }
};

extern "C" {

CVATTN_API size_t cvattn_dit_cache_device_bytes(const cvattn_dit_cache_params *p) {
    if (check_params(p)) return 0;
    const Layout L = layout_of(p);
    return (size_t)p->n_slots * (size_t)p->layers * (L.k_al + L.v_al);
}

CVATTN_API size_t cvattn_dit_cache_host_bytes(const cvattn_dit_cache_params *p) {
    if (check_params(p)) return 0;
    const Layout L = layout_of(p);
    return (size_t)p->n_host_slots * (size_t)p->layers * L.host_layer;
}

CVATTN_API int cvattn_dit_cache_create(const cvattn_dit_cache_params *p, void *device_buf, size_t device_bytes,
                                       void *host_buf, size_t host_bytes, cvattn_dit_cache **out) {
    if (!out) return CVATTN_ERR_BAD_ARGS;
    *out = nullptr;
    int rc = check_params(p);
    if (rc) return rc;
    if (!device_buf || device_bytes < cvattn_dit_cache_device_bytes(p)) return CVATTN_ERR_WORKSPACE_TOO_SMALL;
    if (p->n_host_slots > 0 && (!host_buf || host_bytes < cvattn_dit_cache_host_bytes(p)))
        return CVATTN_ERR_WORKSPACE_TOO_SMALL;
    if ((uintptr_t)device_buf % kTensorAlign) return CVATTN_ERR_BAD_ARGS;
    cvattn_dit_cache *c = new (std::nothrow) cvattn_dit_cache();
    if (!c) return CVATTN_ERR_HIP;
    c->p = *p;
    c->L = layout_of(p);
    c->dev = (uint8_t *)device_buf;
    c->host = (uint8_t *)host_buf;
    c->slot = 0;
    c->cur_len = 0;
    c->host_len.assign((size_t)p->n_host_slots, 0u);
    *out = c;
    return CVATTN_OK;
}

CVATTN_API void cvattn_dit_cache_destroy(cvattn_dit_cache *c) { delete c; }

CVATTN_API int cvattn_dit_cache_bind_slot(cvattn_dit_cache *c, int slot) {
    if (!c || slot < 0 || slot >= c->p.n_slots) return CVATTN_ERR_BAD_ARGS;
    c->slot = slot;
    return CVATTN_OK;
}

CVATTN_API int cvattn_dit_cache_slide(cvattn_dit_cache *c) {
    if (!c) return CVATTN_ERR_BAD_ARGS;
    // the reference re-points graph views to the next slot, which it only does in flash mode
    if (!c->p.flash_attn) return CVATTN_ERR_UNSUPPORTED;
    if (c->slot + 1 >= c->p.n_slots) return CVATTN_ERR_BAD_ARGS;
    c->slot++;
    return CVATTN_OK;
}

CVATTN_API int cvattn_dit_cache_slot(const cvattn_dit_cache *c) { return c ? c->slot : -1; }

CVATTN_API int cvattn_dit_cache_set_len(cvattn_dit_cache *c, uint32_t cur_len) {
    if (!c || cur_len > (uint32_t)c->p.max_seq) return CVATTN_ERR_BAD_ARGS;
    c->cur_len = cur_len;
    return CVATTN_OK;
}

CVATTN_API uint32_t cvattn_dit_cache_len(const cvattn_dit_cache *c) { return c ? c->cur_len : 0u; }

CVATTN_API int cvattn_dit_cache_layer(const cvattn_dit_cache *c, int layer, int64_t n_kv, cvattn_tensor *k_cache,
                                      cvattn_tensor *v_cache, cvattn_tensor *k_view, cvattn_tensor *v_view) {
    if (!c || layer < 0 || layer >= c->p.layers || n_kv < 0 || n_kv > c->p.max_seq) return CVATTN_ERR_BAD_ARGS;
    const cvattn_dit_cache_params &p = c->p;
    const Layout &L = c->L;
    const int64_t e = (int64_t)p.heads * p.head_dim;
    uint8_t *kt = c->k_tensor(c->slot, layer), *vt = c->v_tensor(c->slot, layer);
    auto set = [](cvattn_tensor *t, void *data, int type, const int64_t ne[4], const size_t nb[4]) {
        if (!t) return;
        t->data = data;
        t->type = type;
        for (int i = 0; i < 4; i++) {
            t->ne[i] = ne[i];
            t->nb[i] = nb[i];
        }
    };
    const size_t kb0 = (size_t)type_bytes(p.k_type);
    {   // K cache [H*D, max_seq, B] and its view [D, n_kv, H, B] (kv-cache.cpp:316-318)
        const int64_t ne[4] = {e, p.max_seq, p.batch, 1};
        const size_t nb[4] = {kb0, L.k_row, L.k_row * (size_t)p.max_seq, L.k_row * (size_t)p.max_seq * p.batch};
        set(k_cache, kt, p.k_type, ne, nb);
        const int64_t vne[4] = {p.head_dim, n_kv, p.heads, p.batch};
        const size_t vnb[4] = {kb0, L.k_row, L.k_row / (size_t)p.heads, L.k_row * (size_t)p.max_seq};
        set(k_view, kt, p.k_type, vne, vnb);
    }
    const size_t vb0 = (size_t)type_bytes(p.v_type);
    if (p.flash_attn) { // V like K (kv-cache.cpp:322-324)
        const int64_t ne[4] = {e, p.max_seq, p.batch, 1};
        const size_t nb[4] = {vb0, L.v_row, L.v_row * (size_t)p.max_seq, L.v_row * (size_t)p.max_seq * p.batch};
        set(v_cache, vt, p.v_type, ne, nb);
        const int64_t vne[4] = {p.head_dim, n_kv, p.heads, p.batch};
        const size_t vnb[4] = {vb0, L.v_row, L.v_row / (size_t)p.heads, L.v_row * (size_t)p.max_seq};
        set(v_view, vt, p.v_type, vne, vnb);
    } else { // transposed V [max_seq, H*D, B] and its view [n_kv, D, H, B] (kv-cache.cpp:104-108,345)
        const size_t col = L.v_es * (size_t)p.max_seq;
        const int64_t ne[4] = {p.max_seq, e, p.batch, 1};
        const size_t nb[4] = {L.v_es, col, col * (size_t)e, col * (size_t)e * p.batch};
        set(v_cache, vt, p.v_type, ne, nb);
        const int64_t vne[4] = {n_kv, p.head_dim, p.heads, p.batch};
        const size_t vnb[4] = {L.v_es, col, col * (size_t)p.head_dim, col * (size_t)e};
        set(v_view, vt, p.v_type, vne, vnb);
    }
    return CVATTN_OK;
}

// Copies between the bound slot's first n rows and host slot h; to_host picks the direction.
static int slot_copy(cvattn_dit_cache *c, int h, uint32_t n, bool to_host, hipStream_t st) {
    const cvattn_dit_cache_params &p = c->p;
    const Layout &L = c->L;
    const int64_t e = (int64_t)p.heads * p.head_dim;
    if (n == 0) return CVATTN_OK;
    for (int l = 0; l < p.layers; l++) {
        uint8_t *hk = c->host_layer(h, l);
        uint8_t *dk = c->k_tensor(c->slot, l), *dv = c->v_tensor(c->slot, l);
        // K: n rows of each batch entry, batch entries max_seq rows apart on the device
        const size_t kw = L.k_row * n, kp = L.k_row * (size_t)p.max_seq;
        hipError_t err = to_host ? hipMemcpy2DAsync(hk, kw, dk, kp, kw, (size_t)p.batch, hipMemcpyDeviceToHost, st)
                                 : hipMemcpy2DAsync(dk, kp, hk, kw, kw, (size_t)p.batch, hipMemcpyHostToDevice, st);
        if (err != hipSuccess) return CVATTN_ERR_HIP;
        uint8_t *hv = hk + kw * (size_t)p.batch;
        if (p.flash_attn) {
            const size_t vw = L.v_row * n, vp = L.v_row * (size_t)p.max_seq;
            err = to_host ? hipMemcpy2DAsync(hv, vw, dv, vp, vw, (size_t)p.batch, hipMemcpyDeviceToHost, st)
                          : hipMemcpy2DAsync(dv, vp, hv, vw, vw, (size_t)p.batch, hipMemcpyHostToDevice, st);
        } else {
            // the first n tokens of every (feature, batch) column of the transposed cache
            const size_t vw = L.v_es * n, vp = L.v_es * (size_t)p.max_seq, rows = (size_t)e * p.batch;
            err = to_host ? hipMemcpy2DAsync(hv, vw, dv, vp, vw, rows, hipMemcpyDeviceToHost, st)
                          : hipMemcpy2DAsync(dv, vp, hv, vw, vw, rows, hipMemcpyHostToDevice, st);
        }
        if (err != hipSuccess) return CVATTN_ERR_HIP;
    }
    return CVATTN_OK;
}

CVATTN_API int cvattn_dit_cache_offload(cvattn_dit_cache *c, int host_slot, uint32_t n_tokens,
                                        cvattn_stream_t stream) {
    if (!c || host_slot < 0 || host_slot >= c->p.n_host_slots || n_tokens > (uint32_t)c->p.max_seq)
        return CVATTN_ERR_BAD_ARGS;
    int rc = slot_copy(c, host_slot, n_tokens, true, (hipStream_t)stream);
    if (rc) return rc;
    c->host_len[(size_t)host_slot] = n_tokens;
    return CVATTN_OK;
}

CVATTN_API int cvattn_dit_cache_load(cvattn_dit_cache *c, int host_slot, cvattn_stream_t stream) {
    if (!c || host_slot < 0 || host_slot >= c->p.n_host_slots) return CVATTN_ERR_BAD_ARGS;
    const uint32_t n = c->host_len[(size_t)host_slot];
    int rc = slot_copy(c, host_slot, n, false, (hipStream_t)stream);
    if (rc) return rc;
    c->cur_len = n;
    return CVATTN_OK;
}

CVATTN_API int cvattn_fill_positions(const cvattn_tensor *pos, int32_t base, cvattn_stream_t stream) {
    if (!pos || pos->type != T_I32 || pos->nb[0] != 4) return CVATTN_ERR_BAD_ARGS;
    if (pos->ne[2] != 1 || pos->ne[3] != 1 || pos->ne[0] < 0 || pos->ne[1] < 0) return CVATTN_ERR_BAD_ARGS;
    if (pos->ne[0] * pos->ne[1] > 0 && !pos->data) return CVATTN_ERR_BAD_ARGS;
    if (pos->nb[1] < 4 * (size_t)pos->ne[0] || pos->nb[1] % 4) return CVATTN_ERR_BAD_ARGS;
    return hip_rc(fill_positions_launch((int32_t *)pos->data, pos->ne[0], pos->ne[1], (int64_t)pos->nb[1], base,
                                        (hipStream_t)stream));
}

CVATTN_API int cvattn_chunk_mask(const cvattn_tensor *mask, const uint32_t *bounds, int n_bounds,
                                 cvattn_stream_t stream) {
    if (!mask || mask->type != T_F16 || mask->nb[0] != 2) return CVATTN_ERR_BAD_ARGS;
    if (mask->ne[2] != 1 || mask->ne[3] != 1 || mask->ne[0] < 0 || mask->ne[1] < 0) return CVATTN_ERR_BAD_ARGS;
    if (n_bounds < 0 || n_bounds > CVATTN_MAX_CHUNK_BOUNDS || (n_bounds > 0 && !bounds)) return CVATTN_ERR_BAD_ARGS;
    if (mask->ne[0] > 0x7fffffff || mask->ne[1] > 0x7fffffff) return CVATTN_ERR_UNSUPPORTED;
    if (mask->ne[0] * mask->ne[1] > 0 && !mask->data) return CVATTN_ERR_BAD_ARGS;
    for (int i = 1; i < n_bounds; i++)
        if (bounds[i] < bounds[i - 1]) return CVATTN_ERR_BAD_ARGS; // upper_bound needs them sorted
    ChunkMaskArgs a;
    std::memset(&a, 0, sizeof(a));
    a.mask = (uint8_t *)mask->data;
    a.nb1 = (int64_t)mask->nb[1];
    a.n_cols = (int32_t)mask->ne[0];
    a.n_rows = (int32_t)mask->ne[1];
    a.n_bounds = n_bounds;
    for (int i = 0; i < n_bounds; i++) a.bounds[i] = bounds[i];
    return hip_rc(chunk_mask_launch(a, (hipStream_t)stream));
}

CVATTN_API int cvattn_v_idxs(int32_t *idx, const int32_t *pos, uint32_t n_tokens, uint32_t n_per_batch,
                             uint32_t n_embd, uint32_t max_seq, cvattn_stream_t stream) {
    if (n_per_batch == 0 || n_embd == 0 || max_seq == 0) return CVATTN_ERR_BAD_ARGS;
    if ((uint64_t)n_tokens * n_embd > 0 && (!idx || !pos)) return CVATTN_ERR_BAD_ARGS;
    // every index must fit the 32-bit index tensor the scatter reads
    const uint64_t batches = (n_tokens + n_per_batch - 1) / n_per_batch;
    if (batches * (uint64_t)max_seq * n_embd > 0x7fffffffull) return CVATTN_ERR_UNSUPPORTED;
    return hip_rc(v_idxs_launch(idx, pos, n_tokens, n_per_batch, n_embd, max_seq, (hipStream_t)stream));
}

CVATTN_API int cvattn_dit_schedule(int n_steps, int n_fixed_slots, int n_offloadable_slots, int64_t cut_len,
                                   uint32_t offset, int streaming, int kv_slidable, cvattn_dit_step *out) {
    if (!out || n_steps < 2 || n_fixed_slots < 0 || n_offloadable_slots < 0) return CVATTN_ERR_BAD_ARGS;
    if (streaming && n_fixed_slots + n_offloadable_slots > n_steps) return CVATTN_ERR_BAD_ARGS;
    const int n = n_steps;
    for (int i = 0; i < n; i++) std::memset(&out[i], 0, sizeof(out[i]));
    if (!streaming) {
        // one-shot: graphs at steps 0, 1 and the last, which takes the cut
        out[0].rebuild = out[1].rebuild = out[n - 1].rebuild = 1;
        out[n - 1].cut_len = cut_len;
    } else {
        if (offset != 0) cut_len = 0;
        const int n_off = n_offloadable_slots, n_fix = n_fixed_slots;
        const int first_cached = n - n_off - n_fix; // steps before it run without a cache
        for (int i = 0; i < n; i++) {
            cvattn_dit_step &s = out[i];
            const bool cached = i >= first_cached;
            const bool offl = cached && i < first_cached + n_off;
            s.cache_kv = cached;
            s.offload = offl;
            s.load = offl && offset != 0;
            s.mask = !cached && offset != 0;
            s.cut_len = (i == n - 1 && offset == 0) ? cut_len : 0;
            if (offset != 0 && i == first_cached - 1) s.cut_len = offset;
            s.slice = offset != 0 && i == first_cached;
            s.rebuild = i <= 1 || (offset != 0 && i == first_cached - 1) || i == first_cached ||
                        (i == n - 1 && cut_len != 0) || (!kv_slidable && cached);
            s.slide = kv_slidable && cached && (!offl || i == first_cached + n_off - 1) && i != n - 1;
        }
    }
    // replay the slot bookkeeping: bind at step 0, rebind on rebuilds of cached steps (offloadable
    // steps share device slot 0, fixed step i takes slot i + slot_offset), slide after a step;
    // host slots count the offloadable steps
    const int slot_offset = n_fixed_slots - n + (n_offloadable_slots ? 1 : 0);
    int cur = 0, host = 0;
    for (int i = 0; i < n; i++) {
        cvattn_dit_step &s = out[i];
        if (i == 0 && s.cache_kv) cur = 0;
        if (i > 0 && s.rebuild && s.cache_kv) cur = s.offload ? 0 : i + slot_offset;
        s.slot = s.cache_kv ? cur : -1;
        s.host_slot = (s.load || s.offload) ? host : -1;
        if (s.offload) host++;
        if (s.slide) cur++;
    }
    return CVATTN_OK;
}

} // extern "C"
