// kv_cache_test.cpp -- parity test of the C++ host class cvattn::kv_cache.  The class mirrors
// cosyvoice_kv_cache (src/cosyvoice-kv-cache.cpp).  The test drives it the way the reference's
// callers drive cosyvoice_kv_cache, and checks every result against the oracle (liboracle.so).
//
//   llm     Qwen2 layers: 14 query / 2 kv heads, head_dim 64, batch 1 (src/cosyvoice-llm.cpp:
//           31-76,95-299).  A 37-token causal prefill, then decode steps.  K goes through the fused
//           NEOX rope (base 1e6).  The cache is offloaded, clobbered and loaded back
//           (src/cosyvoice-model.cpp:586-601), then decoded again.  Runs in the flash-attention
//           mode (q8_0/q4_0 and f16/f16) and in the non-flash mode (q8_0 K, transposed f16 V,
//           set_input_v_idxs + the element scatter).
//   dit     Flow-DiT streaming slots: 16 heads, batch 2 (the CFG pair), rows of 1024 with NORMAL
//           rope over the first 64 dims (src/cosyvoice-graph.cpp:345-377).  Two chunks over three
//           ODE-step slots.  Slot 0 is the staging slot, offloaded after chunk 1 and loaded back
//           before chunk 2 (src/cosyvoice-token2wav.cpp:311-348,389-393).  Slots are changed with
//           bind_slot and slide_kv_slot.
//
// Checks:
//   - V cache bytes of every written row are bit-exact against the oracle's quantizers.
//   - K rows pass through the rope, which is within 2e-6 of the oracle's rope, not bit-exact
//     (the device takes its own cos/sin).  So each K row is checked against the oracle's
//     quantization of the oracle's rotated row to the same bounds as the rope tests:
//       f16: within one fp16 ulp.  f32: within 2e-6.
//       Block types: block scales equal; every dequantized element within one quantization
//       step (the block scale).
//   - Every attention output is within max-abs 2e-3 / mean-abs 2e-4 of the oracle's fp64
//     attention over the oracle's bytes.
//
// Usage: kv_cache_test [--no-gpu].  --no-gpu runs only the argument checks that need no device.
// Exit status 0 when every check passes.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "../../cosyvoice.cpp_amd/host/cvattn_kv_cache.h"
#include "../../oracle/oracle.h"

namespace {

constexpr double kMaxAbs = 2e-3, kMeanAbs = 2e-4;
int g_fail = 0;

void check(bool ok, const std::string &what) {
    if (!ok) {
        std::printf("FAIL %s\n", what.c_str());
        g_fail++;
    }
}

#define HIP_OK(x)                                                                                        \
    do {                                                                                                 \
        hipError_t e_ = (x);                                                                             \
        if (e_ != hipSuccess) {                                                                          \
            std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__);           \
            std::exit(2);                                                                                \
        }                                                                                                \
    } while (0)

#define RC_OK(x, what)                                                                                   \
    do {                                                                                                 \
        int rc_ = (x);                                                                                   \
        if (rc_ != CVATTN_OK) {                                                                          \
            std::printf("FAIL %s: %s\n", std::string(what).c_str(), cvattn_status_string(rc_));          \
            std::exit(1);                                                                                \
        }                                                                                                \
    } while (0)

struct DevBuf {
    void *p = nullptr;
    size_t n = 0;
    explicit DevBuf(size_t bytes) : n(bytes) { HIP_OK(hipMalloc(&p, bytes ? bytes : 1)); }
    ~DevBuf() { (void)hipFree(p); }
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    template <class T> void put(const std::vector<T> &v) {
        HIP_OK(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
    }
};

std::vector<float> randn(std::mt19937 &g, size_t n) {
    std::normal_distribution<float> d(0.0f, 1.0f);
    std::vector<float> v(n);
    for (float &x : v) x = d(g);
    return v;
}

cvattn_tensor tensor(void *data, int type, std::initializer_list<int64_t> ne, std::initializer_list<size_t> nb) {
    cvattn_tensor t;
    t.data = data;
    t.type = type;
    int i = 0;
    for (int64_t e : ne) t.ne[i++] = e;
    i = 0;
    for (size_t b : nb) t.nb[i++] = b;
    return t;
}

or_tensor otensor(const void *data, int type, const int64_t ne[4], const size_t nb[4]) {
    or_tensor t;
    t.data = (void *)data;
    t.type = type;
    for (int i = 0; i < 4; i++) {
        t.ne[i] = ne[i];
        t.nb[i] = nb[i];
    }
    return t;
}

void compare(const std::vector<float> &got, const std::vector<float> &want, const std::string &what) {
    double mx = 0.0, sum = 0.0;
    bool finite = true;
    for (size_t i = 0; i < got.size(); i++) {
        if (!std::isfinite(got[i])) finite = false;
        const double e = std::fabs((double)got[i] - (double)want[i]);
        mx = e > mx ? e : mx;
        sum += e;
    }
    const double mean = got.empty() ? 0.0 : sum / (double)got.size();
    const bool ok = finite && mx <= kMaxAbs && mean <= kMeanAbs;
    std::printf("%s %s: max-abs %.3g mean-abs %.3g\n", ok ? "ok  " : "FAIL", what.c_str(), mx, mean);
    if (!ok) g_fail++;
}

// The oracle's copy of one layer of one slot: the rotated f32 rows the host wrote, by token.
struct LayerMirror {
    int64_t e = 0, max_seq = 0, batch = 0;
    std::vector<float> k, v; // [batch][max_seq][e]
    void init(int64_t e_, int64_t ms, int64_t b) {
        e = e_;
        max_seq = ms;
        batch = b;
        k.assign((size_t)(b * ms * e), 0.0f);
        v.assign((size_t)(b * ms * e), 0.0f);
    }
    float *krow(int64_t b, int64_t t) { return &k[(size_t)((b * max_seq + t) * e)]; }
    float *vrow(int64_t b, int64_t t) { return &v[(size_t)((b * max_seq + t) * e)]; }
};

// Quantized bytes of rows [0, n) of each batch entry: [batch][n][row bytes].
std::vector<uint8_t> quantize_rows(const std::vector<float> &rows, int type, int64_t e, int64_t max_seq, int64_t batch,
                                   int64_t n) {
    const int64_t rb = or_row_size(type, e);
    std::vector<uint8_t> out((size_t)(batch * n * rb));
    for (int64_t b = 0; b < batch; b++)
        for (int64_t t = 0; t < n; t++)
            or_quantize_row(type, &rows[(size_t)((b * max_seq + t) * e)], &out[(size_t)((b * n + t) * rb)], e);
    return out;
}

// The transposed f16 V of rows [0, n): [batch][e][n].
std::vector<uint16_t> transpose_f16(const std::vector<float> &rows, int64_t e, int64_t max_seq, int64_t batch, int64_t n) {
    std::vector<uint16_t> out((size_t)(batch * e * n));
    for (int64_t b = 0; b < batch; b++)
        for (int64_t t = 0; t < n; t++)
            for (int64_t f = 0; f < e; f++)
                out[(size_t)((b * e + f) * n + t)] = or_fp32_to_fp16(rows[(size_t)((b * max_seq + t) * e + f)]);
    return out;
}

// Device cache bytes of rows [0, n) of each batch entry, laid out like quantize_rows.
std::vector<uint8_t> fetch_rows(const cvattn_tensor &cache, int64_t n) {
    const size_t rb = cache.nb[1];
    std::vector<uint8_t> out((size_t)cache.ne[2] * n * rb);
    for (int64_t b = 0; b < cache.ne[2]; b++)
        HIP_OK(hipMemcpy(&out[(size_t)b * n * rb], (const uint8_t *)cache.data + b * cache.nb[2], n * rb,
                         hipMemcpyDeviceToHost));
    return out;
}

// K rows of the device against the oracle's, to the rope's bound (see the file comment).
bool k_rows_close(int type, const std::vector<uint8_t> &got, const std::vector<uint8_t> &want, int64_t e) {
    if (got.size() != want.size()) return false;
    if (type == OR_TYPE_F16) {
        const uint16_t *g = (const uint16_t *)got.data(), *w = (const uint16_t *)want.data();
        for (size_t i = 0; i < got.size() / 2; i++)
            if (std::abs((int)g[i] - (int)w[i]) > 1) return false;
        return true;
    }
    if (type == OR_TYPE_F32) {
        const float *g = (const float *)got.data(), *w = (const float *)want.data();
        for (size_t i = 0; i < got.size() / 4; i++)
            if (!(std::fabs(g[i] - w[i]) <= 2e-6f)) return false;
        return true;
    }
    // block types: the fp16 scale (and min) header, then the codes
    const int64_t bs = or_type_size(type), hdr = (type == OR_TYPE_Q4_1 || type == OR_TYPE_Q5_1) ? 4 : 2;
    const int64_t rb = or_row_size(type, e), rows = (int64_t)got.size() / rb;
    std::vector<float> dg((size_t)e), dw((size_t)e);
    for (int64_t r = 0; r < rows; r++) {
        const uint8_t *g = &got[(size_t)(r * rb)], *w = &want[(size_t)(r * rb)];
        or_dequantize_row(type, g, dg.data(), e);
        or_dequantize_row(type, w, dw.data(), e);
        for (int64_t b = 0; b < e / 32; b++) {
            if (std::memcmp(g + b * bs, w + b * bs, (size_t)hdr)) return false;
            uint16_t d16;
            std::memcpy(&d16, w + b * bs, 2);
            const float step = std::fabs(or_fp16_to_fp32(d16));
            for (int64_t i = 0; i < 32; i++)
                if (!(std::fabs(dg[(size_t)(b * 32 + i)] - dw[(size_t)(b * 32 + i)]) <= step + 1e-7f)) return false;
        }
    }
    return true;
}

// Device transposed V [max_seq, e, batch] f16: the first n tokens of each column, as transpose_f16.
std::vector<uint16_t> fetch_vt(const cvattn_tensor &cache, int64_t n) {
    const int64_t e = cache.ne[1], batch = cache.ne[2];
    std::vector<uint16_t> out((size_t)(batch * e * n));
    HIP_OK(hipMemcpy2D(out.data(), n * 2, cache.data, cache.nb[1], n * 2, (size_t)(e * batch), hipMemcpyDeviceToHost));
    return out;
}

// Fills every byte of a layer's cache tensors of the bound slot.
void clobber(cvattn::kv_cache &c, int layers, uint8_t byte) {
    for (int l = 0; l < layers; l++) {
        cvattn_tensor kc, vc;
        RC_OK(c.layer_tensors(l, 0, &kc, &vc, nullptr, nullptr), "layer_tensors");
        HIP_OK(hipMemset(kc.data, byte, kc.nb[2] * (size_t)kc.ne[2]));
        HIP_OK(hipMemset(vc.data, byte, vc.nb[2] * (size_t)vc.ne[2]));
    }
    HIP_OK(hipDeviceSynchronize());
}

// ------------------------------------------------------------------------------------------------
// LLM: prefill + decode + offload/load, one slot, batch 1
// ------------------------------------------------------------------------------------------------
void run_llm(int kt, int vt, bool fattn, hipStream_t st) {
    const int L = 2, D = 64, Hkv = 2, H = 14, E = D * Hkv;
    const uint32_t max_seq = 300;
    const float base = 1e6f;
    char name[96];
    std::snprintf(name, sizeof name, "llm %s k%d v%d", fattn ? "fa" : "nonfa", kt, vt);
    std::printf("case %s\n", name);
    std::fflush(stdout);
    std::mt19937 g(1234 + kt * 16 + vt + (fattn ? 0 : 100));

    cvattn::kv_cache c;
    RC_OK(c.build_kv_cache(L, D, D, Hkv, max_seq, kt, vt, 1, 1, 1, fattn), "build_kv_cache");
    check(c.can_reuse() == fattn, "can_reuse");
    std::vector<LayerMirror> mir(L);
    for (auto &m : mir) m.init(E, max_seq, 1);

    auto step = [&](uint32_t n, bool reuse, const char *tag) {
        const uint32_t t0 = c.cur_len, total = t0 + n;
        std::vector<int32_t> pos(n), pos_heads((size_t)n * Hkv);
        for (uint32_t i = 0; i < n; i++) {
            pos[i] = (int32_t)(t0 + i);
            for (int h = 0; h < Hkv; h++) pos_heads[(size_t)i * Hkv + h] = (int32_t)(t0 + i);
        }
        DevBuf dpos(4 * n);
        dpos.put(pos);
        const cvattn_tensor pid = tensor(dpos.p, CVATTN_TYPE_I32, {n, 1, 1, 1}, {4, 4 * n, 4 * n, 4 * n});
        if (!fattn) RC_OK(c.set_input_v_idxs((const int32_t *)dpos.p, n, n, st), "set_input_v_idxs");
        // causal mask [total, n] (src/cosyvoice-llm.cpp:101-107) for a prefill; none for one token
        std::vector<uint16_t> mask;
        DevBuf dmask(2 * (size_t)total * n);
        if (n > 1) {
            mask.resize((size_t)total * n);
            or_causal_mask(mask.data(), n, total);
            dmask.put(mask);
        }
        const cvattn_tensor mt = tensor(dmask.p, CVATTN_TYPE_F16, {total, n, 1, 1},
                                        {2, 2 * (size_t)total, 2 * (size_t)total * n, 2 * (size_t)total * n});
        for (int l = 0; l < L; l++) {
            std::vector<float> k = randn(g, (size_t)n * E), v = randn(g, (size_t)n * E), q = randn(g, (size_t)n * H * D);
            DevBuf dk(4 * k.size()), dv(4 * v.size()), dq(4 * q.size()), dout(4 * q.size());
            dk.put(k);
            dv.put(v);
            dq.put(q);
            cvattn_tensor kk = tensor(dk.p, CVATTN_TYPE_F32, {D, Hkv, n, 1}, {4, 4 * D, 4 * (size_t)E, 4 * (size_t)E * n});
            cvattn_tensor vv = tensor(dv.p, CVATTN_TYPE_F32, {D, Hkv, n, 1}, {4, 4 * D, 4 * (size_t)E, 4 * (size_t)E * n});
            RC_OK(c.update_cache_rope(kk, vv, pid, l, D, D, CVATTN_ROPE_NEOX, base, 1.0f, st), "update_cache_rope");
            check(kk.ne[1] == total && vv.ne[fattn ? 1 : 0] == total, "update_cache views span cur_len + n");
            // q [D, H, n] permuted to [D, n, H] (src/cosyvoice-llm.cpp:60)
            const cvattn_tensor qv = tensor(dq.p, CVATTN_TYPE_F32, {D, n, H, 1},
                                            {4, 4 * (size_t)H * D, 4 * D, 4 * (size_t)H * D * n});
            const cvattn_tensor dst = tensor(dout.p, CVATTN_TYPE_F32, {D, H, n, 1},
                                             {4, 4 * D, 4 * (size_t)H * D, 4 * (size_t)H * D * n});
            RC_OK(c.attention_forward(qv, kk, vv, n > 1 ? &mt : nullptr, dst, st), "attention_forward");
            HIP_OK(hipStreamSynchronize(st));
            std::vector<float> got(q.size());
            HIP_OK(hipMemcpy(got.data(), dout.p, 4 * got.size(), hipMemcpyDeviceToHost));

            // oracle: rotate K per head, record the rows, quantize, attend
            std::vector<float> kr(k.size());
            or_rope_f32(k.data(), kr.data(), D, (int64_t)n * Hkv, pos_heads.data(), D, OR_ROPE_NEOX, base, 1.0f);
            for (uint32_t i = 0; i < n; i++) {
                std::memcpy(mir[l].krow(0, t0 + i), &kr[(size_t)i * E], 4 * E);
                std::memcpy(mir[l].vrow(0, t0 + i), &v[(size_t)i * E], 4 * E);
            }
            cvattn_tensor kc, vc;
            RC_OK(c.layer_tensors(l, total, &kc, &vc, nullptr, nullptr), "layer_tensors");
            const std::vector<uint8_t> kq = quantize_rows(mir[l].k, kt, E, max_seq, 1, total);
            check(k_rows_close(kt, fetch_rows(kc, total), kq, E), std::string(name) + " " + tag + ": K cache rows");
            const int64_t rk = or_row_size(kt, E);
            const int64_t ks = or_type_size(kt);
            const int64_t kne[4] = {D, total, Hkv, 1};
            const size_t knb[4] = {(size_t)ks, (size_t)rk, (size_t)rk / Hkv, (size_t)rk * total};
            const or_tensor ok = otensor(kq.data(), kt, kne, knb);
            const int64_t qne[4] = {D, n, H, 1};
            const size_t qnb[4] = {4, 4 * (size_t)H * D, 4 * D, 4 * (size_t)H * D * n};
            const or_tensor oq = otensor(q.data(), OR_TYPE_F32, qne, qnb);
            const int64_t mne[4] = {total, n, 1, 1};
            const size_t mnb[4] = {2, 2 * (size_t)total, 2 * (size_t)total * n, 2 * (size_t)total * n};
            const or_tensor om = otensor(mask.data(), OR_TYPE_F16, mne, mnb);
            std::vector<float> want(q.size());
            if (fattn) {
                const std::vector<uint8_t> vq = quantize_rows(mir[l].v, vt, E, max_seq, 1, total);
                check(fetch_rows(vc, total) == vq, std::string(name) + " " + tag + ": V cache bytes");
                const int64_t rv = or_row_size(vt, E);
                const int64_t vne[4] = {D, total, Hkv, 1};
                const size_t vnb[4] = {(size_t)or_type_size(vt), (size_t)rv, (size_t)rv / Hkv, (size_t)rv * total};
                const or_tensor ov = otensor(vq.data(), vt, vne, vnb);
                or_flash_attn_ext_f64(&oq, &ok, &ov, n > 1 ? &om : nullptr, want.data(), 0.125f);
            } else {
                const std::vector<uint16_t> vth = transpose_f16(mir[l].v, E, max_seq, 1, total);
                check(fetch_vt(vc, total) == vth, std::string(name) + " " + tag + ": transposed V cache bytes");
                const int64_t vne[4] = {total, D, Hkv, 1};
                const size_t vnb[4] = {2, 2 * (size_t)total, 2 * (size_t)total * D, 2 * (size_t)total * E};
                const or_tensor ov = otensor(vth.data(), OR_TYPE_F16, vne, vnb);
                or_attn_nonfa_f64(&oq, &ok, &ov, n > 1 ? &om : nullptr, want.data(), 0.125f);
            }
            compare(got, want, std::string(name) + " " + tag + " layer " + std::to_string(l));
        }
        // the two ways the reference advances the cache (src/cosyvoice-llm.cpp:124,197,221,299)
        if (reuse)
            RC_OK(c.shift_kv_node_pos(n), "shift_kv_node_pos");
        else
            c.cur_len += n;
        check(c.cur_len == total, "cur_len advanced");
    };

    step(37, false, "prefill 37");
    step(1, false, "decode 38");
    step(1, fattn, "decode 39");
    step(1, fattn, "decode 40");
    if (!fattn) {
        check(c.shift_kv_node_pos(1) == CVATTN_ERR_UNSUPPORTED, "shift_kv_node_pos needs flash attention");
        check(c.slide_kv_slot() == CVATTN_ERR_UNSUPPORTED, "slide_kv_slot needs flash attention");
    }

    // offload the cache, clobber the device slot, load it back (src/cosyvoice-model.cpp:586-601)
    const uint32_t kept = c.cur_len;
    RC_OK(c.offload_cache(kept, st), "offload_cache");
    HIP_OK(hipStreamSynchronize(st));
    const size_t row_host = (size_t)L * ((size_t)or_row_size(kt, E) + (fattn ? (size_t)or_row_size(vt, E) : 2 * (size_t)E));
    check(c.get_offloaded_cache_size() == row_host * kept, "get_offloaded_cache_size");
    clobber(c, L, 0x7b);
    c.cur_len = 0;
    RC_OK(c.load_cache(st), "load_cache");
    HIP_OK(hipStreamSynchronize(st));
    check(c.cur_len == kept, "load_cache restores cur_len");
    step(1, false, "decode after load");
    step(3, fattn, "3 tokens after load");

    c.clear_offloaded_cache();
    check(c.get_offloaded_cache_size() == 0, "clear_offloaded_cache");
    RC_OK(c.load_cache(st), "load_cache after clear");
    check(c.cur_len == 0, "load after clear empties the cache");
    check(c.offload_slot(1, 4, st) == CVATTN_ERR_BAD_ARGS, "offload_slot past the host slots");
    check(!c.bind_slot(1), "bind_slot past the last slot");
}

// ------------------------------------------------------------------------------------------------
// DiT: streaming slots, batch 2, two chunks
// ------------------------------------------------------------------------------------------------
void run_dit(int kt, int vt, bool fattn, hipStream_t st) {
    const int L = 2, D = 64, H = 16, E = D * H, B = 2, S = 3;
    const uint32_t max_seq = 160, T1 = 60, T2 = 40;
    char name[96];
    std::snprintf(name, sizeof name, "dit %s k%d v%d", fattn ? "fa" : "nonfa", kt, vt);
    std::printf("case %s\n", name);
    std::fflush(stdout);
    std::mt19937 g(77 + kt * 16 + vt + (fattn ? 0 : 100));

    cvattn::kv_cache c;
    RC_OK(c.build_kv_cache(L, D, D, H, max_seq, kt, vt, B, S, 1, fattn), "build_kv_cache");
    std::vector<std::vector<LayerMirror>> mir(S, std::vector<LayerMirror>(L));
    for (auto &s : mir)
        for (auto &m : s) m.init(E, max_seq, B);

    // one ODE step of a chunk: the rows of every layer into the bound slot, then attention
    auto ode_step = [&](int slot, uint32_t T, const std::vector<uint32_t> &bounds, const std::string &tag) {
        check(c.slot() == slot, tag + ": bound slot");
        const uint32_t t0 = c.cur_len, total = t0 + T;
        // positions [T, B] = t0 + j (src/cosyvoice-token2wav.cpp:277-283); the rope takes them flat
        std::vector<int32_t> pos((size_t)T * B);
        for (int b = 0; b < B; b++)
            for (uint32_t j = 0; j < T; j++) pos[(size_t)b * T + j] = (int32_t)(t0 + j);
        DevBuf dpos(4 * pos.size());
        dpos.put(pos);
        const cvattn_tensor pid = tensor(dpos.p, CVATTN_TYPE_I32, {T, B, 1, 1}, {4, 4 * T, 4 * (size_t)T * B, 4 * (size_t)T * B});
        if (!fattn) RC_OK(c.set_input_v_idxs((const int32_t *)dpos.p, T * B, T, st), "set_input_v_idxs");
        // chunk mask over the new frames of a first chunk (src/cosyvoice-token2wav.cpp:285-298)
        std::vector<uint16_t> mask;
        const bool masked = !bounds.empty();
        DevBuf dmask(2 * (size_t)T * T);
        if (masked) {
            mask.resize((size_t)T * T);
            or_chunk_mask(mask.data(), T, bounds.data(), (int64_t)bounds.size());
            dmask.put(mask);
        }
        const cvattn_tensor mt = tensor(dmask.p, CVATTN_TYPE_F16, {T, T, 1, 1},
                                        {2, 2 * (size_t)T, 2 * (size_t)T * T, 2 * (size_t)T * T});
        for (int l = 0; l < L; l++) {
            const size_t nrow = (size_t)B * T * E;
            std::vector<float> k = randn(g, nrow), v = randn(g, nrow), q = randn(g, nrow);
            DevBuf dk(4 * nrow), dv(4 * nrow), dq(4 * nrow), dout(4 * nrow);
            dk.put(k);
            dv.put(v);
            dq.put(q);
            // [D, H, T, B] (src/cosyvoice-graph.cpp:357-359)
            cvattn_tensor kk = tensor(dk.p, CVATTN_TYPE_F32, {D, H, T, B}, {4, 4 * D, 4 * (size_t)E, 4 * (size_t)E * T});
            cvattn_tensor vv = tensor(dv.p, CVATTN_TYPE_F32, {D, H, T, B}, {4, 4 * D, 4 * (size_t)E, 4 * (size_t)E * T});
            RC_OK(c.update_cache_rope(kk, vv, pid, l, E, D, CVATTN_ROPE_NORMAL, 10000.0f, 1.0f, st), "update_cache_rope");
            const cvattn_tensor qv = tensor(dq.p, CVATTN_TYPE_F32, {D, T, H, B}, {4, 4 * (size_t)E, 4 * D, 4 * (size_t)E * T});
            const cvattn_tensor dst = tensor(dout.p, CVATTN_TYPE_F32, {D, H, T, B}, {4, 4 * D, 4 * (size_t)E, 4 * (size_t)E * T});
            RC_OK(c.attention_forward(qv, kk, vv, masked ? &mt : nullptr, dst, st), "attention_forward");
            HIP_OK(hipStreamSynchronize(st));
            std::vector<float> got(nrow);
            HIP_OK(hipMemcpy(got.data(), dout.p, 4 * nrow, hipMemcpyDeviceToHost));

            std::vector<float> kr(nrow);
            or_rope_f32(k.data(), kr.data(), E, (int64_t)T * B, pos.data(), D, OR_ROPE_NORMAL, 10000.0f, 1.0f);
            LayerMirror &m = mir[slot][l];
            for (int b = 0; b < B; b++)
                for (uint32_t j = 0; j < T; j++) {
                    std::memcpy(m.krow(b, t0 + j), &kr[((size_t)b * T + j) * E], 4 * E);
                    std::memcpy(m.vrow(b, t0 + j), &v[((size_t)b * T + j) * E], 4 * E);
                }
            cvattn_tensor kc, vc;
            RC_OK(c.layer_tensors(l, total, &kc, &vc, nullptr, nullptr), "layer_tensors");
            const std::vector<uint8_t> kq = quantize_rows(m.k, kt, E, max_seq, B, total);
            check(k_rows_close(kt, fetch_rows(kc, total), kq, E), name + (" " + tag) + ": K cache rows");
            const int64_t rk = or_row_size(kt, E);
            const int64_t kne[4] = {D, total, H, B};
            const size_t knb[4] = {(size_t)or_type_size(kt), (size_t)rk, (size_t)rk / H, (size_t)rk * total};
            const or_tensor ok = otensor(kq.data(), kt, kne, knb);
            const int64_t qne[4] = {D, T, H, B};
            const size_t qnb[4] = {4, 4 * (size_t)E, 4 * D, 4 * (size_t)E * T};
            const or_tensor oq = otensor(q.data(), OR_TYPE_F32, qne, qnb);
            const int64_t mne[4] = {T, T, 1, 1};
            const size_t mnb[4] = {2, 2 * (size_t)T, 2 * (size_t)T * T, 2 * (size_t)T * T};
            const or_tensor om = otensor(mask.data(), OR_TYPE_F16, mne, mnb);
            std::vector<float> want(nrow);
            if (fattn) {
                const std::vector<uint8_t> vq = quantize_rows(m.v, vt, E, max_seq, B, total);
                check(fetch_rows(vc, total) == vq, name + (" " + tag) + ": V cache bytes");
                const int64_t rv = or_row_size(vt, E);
                const int64_t vne[4] = {D, total, H, B};
                const size_t vnb[4] = {(size_t)or_type_size(vt), (size_t)rv, (size_t)rv / H, (size_t)rv * total};
                const or_tensor ov = otensor(vq.data(), vt, vne, vnb);
                or_flash_attn_ext_f64(&oq, &ok, &ov, masked ? &om : nullptr, want.data(), 0.125f);
            } else {
                const std::vector<uint16_t> vth = transpose_f16(m.v, E, max_seq, B, total);
                check(fetch_vt(vc, total) == vth, name + (" " + tag) + ": transposed V cache bytes");
                const int64_t vne[4] = {total, D, H, B};
                const size_t vnb[4] = {2, 2 * (size_t)total, 2 * (size_t)total * D, 2 * (size_t)total * E};
                const or_tensor ov = otensor(vth.data(), OR_TYPE_F16, vne, vnb);
                or_attn_nonfa_f64(&oq, &ok, &ov, masked ? &om : nullptr, want.data(), 0.125f);
            }
            compare(got, want, name + (" " + tag) + " layer " + std::to_string(l));
        }
    };

    // chunk 1: cur_len 0 for every step; slot 0 (staging) is offloaded after its step
    check(c.bind_slot(0), "bind_slot 0");
    ode_step(0, T1, {25, 50}, "chunk 1 step 0");
    RC_OK(c.offload_slot(0, c.cur_len + T1, st), "offload_slot");
    check(c.bind_slot(1), "bind_slot 1");
    ode_step(1, T1, {25, 50}, "chunk 1 step 1");
    if (fattn) {
        RC_OK(c.slide_kv_slot(), "slide_kv_slot");
    } else {
        check(c.slide_kv_slot() == CVATTN_ERR_UNSUPPORTED, "slide_kv_slot needs flash attention");
        check(c.bind_slot(2), "bind_slot 2");
    }
    ode_step(2, T1, {25, 50}, "chunk 1 step 2");
    check(c.slide_kv_slot() != CVATTN_OK, "no slot after the last");
    c.cur_len += T1; // the chunk's frames join the cache (src/cosyvoice-token2wav.cpp:466-468)

    // chunk 2: slot 0 is reused by another step in between, so it is loaded back first
    check(c.bind_slot(0), "bind_slot 0");
    clobber(c, L, 0x5a);
    const uint32_t kv_len = c.cur_len;
    RC_OK(c.load_slot(0, st), "load_slot");
    check(c.cur_len == T1, "load_slot sets the stored length");
    c.cur_len = kv_len; // src/cosyvoice-token2wav.cpp:316-318
    ode_step(0, T2, {}, "chunk 2 step 0");
    check(c.bind_slot(1), "bind_slot 1");
    ode_step(1, T2, {}, "chunk 2 step 1");
    check(c.bind_slot(2), "bind_slot 2");
    ode_step(2, T2, {}, "chunk 2 step 2");
}

// ------------------------------------------------------------------------------------------------
// Argument checks that need no device
// ------------------------------------------------------------------------------------------------
void run_no_gpu() {
    std::printf("case argument checks\n");
    cvattn::kv_cache c;
    check(c.build_kv_cache(2, 64, 128, 2, 100, CVATTN_TYPE_F16, CVATTN_TYPE_F16, 1, 1, 0, true) ==
              CVATTN_ERR_UNSUPPORTED, "unequal K/V head sizes");
    check(c.build_kv_cache(2, 64, 64, 2, 100, CVATTN_TYPE_Q8_0, CVATTN_TYPE_Q8_0, 1, 1, 0, false) ==
              CVATTN_ERR_UNSUPPORTED, "quantized transposed V");
    check(c.build_kv_cache(0, 64, 64, 2, 100, CVATTN_TYPE_F16, CVATTN_TYPE_F16, 1, 1, 0, true) == CVATTN_ERR_BAD_ARGS,
          "no layers");
    check(c.build_kv_cache(2, 64, 64, 2, 0, CVATTN_TYPE_F16, CVATTN_TYPE_F16, 1, 1, 0, true) == CVATTN_ERR_BAD_ARGS,
          "no rows");
    cvattn_tensor t = tensor(nullptr, CVATTN_TYPE_F32, {64, 2, 1, 1}, {4, 256, 512, 512});
    cvattn_tensor p = tensor(nullptr, CVATTN_TYPE_I32, {1, 1, 1, 1}, {4, 4, 4, 4});
    check(c.update_cache(t, t, p, 0, nullptr) == CVATTN_ERR_BAD_ARGS, "update_cache before build");
    check(c.attention_forward(t, t, t, nullptr, t, nullptr) == CVATTN_ERR_BAD_ARGS, "attention_forward before build");
    check(!c.bind_slot(0), "bind_slot before build");
    check(c.slot() == -1, "no slot before build");
    check(c.load_slot(0, nullptr) == CVATTN_ERR_BAD_ARGS, "load_slot before build");
    check(c.get_offloaded_cache_size() == 0, "nothing offloaded");
}

} // namespace

int main(int argc, char **argv) {
    const bool no_gpu = argc > 1 && std::strcmp(argv[1], "--no-gpu") == 0;
    run_no_gpu();
    if (!no_gpu) {
        hipStream_t st;
        HIP_OK(hipStreamCreate(&st));
        run_llm(CVATTN_TYPE_Q8_0, CVATTN_TYPE_Q4_0, true, st);
        run_llm(CVATTN_TYPE_F16, CVATTN_TYPE_F16, true, st);
        run_llm(CVATTN_TYPE_Q8_0, CVATTN_TYPE_F16, false, st);
        run_dit(CVATTN_TYPE_Q8_0, CVATTN_TYPE_Q4_0, true, st);
        run_dit(CVATTN_TYPE_F16, CVATTN_TYPE_F16, false, st);
        HIP_OK(hipStreamDestroy(st));
    }
    std::printf(g_fail ? "FAILED %d check(s)\n" : "ALL PASSED\n", g_fail);
    return g_fail ? 1 : 0;
}
