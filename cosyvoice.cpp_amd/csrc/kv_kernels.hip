// kv_kernels.hip -- KV-cache block formats on gfx950:
//   * dequantize: the test entry for the in-register unpacking the attention kernels use
//     (same raw8_load/raw8_unpack path), bit-exact to ggml's dequantize_row_*;
//   * set_rows: the quantize-on-write KV update of cosyvoice_kv_cache::update_cache
//     (src/cosyvoice-kv-cache.cpp:316,322), bit-exact to ggml's quantize_row_*_ref, optionally
//     with the K rotary embedding of the same layer fused in front (src/cosyvoice-llm.cpp:57,
//     src/cosyvoice-graph.cpp:352);
//   * rope: ggml_rope_ext for the query side (src/cosyvoice-llm.cpp:56,
//     src/cosyvoice-graph.cpp:351);
//   * cvt_f16: the one-time fp16 copy of fp32 K/V views that many row groups read (the DiT
//     call without cache, src/cosyvoice-graph.cpp:370-376).
#include "cvattn_device.h"
#include "cvattn_launch.h"

namespace cvattn {

// One thread per 8 elements of a 32-element block (f16 shares the 32-element grouping).
template <int T>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *src, float *dst, int64_t n_groups) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gid >> 2;
    if (blk >= n_groups) return;
    const int c = (int)(gid & 3);
    const int64_t row_bytes = T == T_F16 ? 64 : type_bytes(T);
    Raw8<T> r;
    raw8_load<T>(gptr(src) + blk * row_bytes, 0, c, r);
    uint32_t o[4];
    raw8_unpack<T>(r, c, o);
    float rd, rm;
    raw8_scales<T>(r, rd, rm);
    constexpr float bias = stage_bias<T>();
    float y[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const h2 h = as_h2(o[i]);
#pragma unroll
        for (int s = 0; s < 2; s++) {
            if constexpr (is_quant(T)) {
                // (code)*d is exact in fp32; only "+ m" rounds, as in ggml's dequantizers
                const float code = (float)h[s] - bias;
                y[2 * i + s] = has_min(T) ? code * rd + rm : code * rd;
            } else {
                y[2 * i + s] = (float)h[s];
            }
        }
    }
    float *out = dst + blk * 32 + 8 * c;
#pragma unroll
    for (int i = 0; i < 8; i++) out[i] = y[i];
}

__global__ __launch_bounds__(256) void copy_f32_kernel(const float *src, float *dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void f16_to_f32_kernel(const _Float16 *src, float *dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = (float)src[i];
}

// One thread per 8 halfs of a destination row; blocks [0, blocks0) copy view 0, the rest view 1
// (the K and V copies of one call share a launch).  Indices are 32-bit (total < 2^31).  VEC: the
// source rows are 16-byte aligned and ne0 is a multiple of 8, so a chunk is two 16-byte loads
// (plain loads: non-temporal ones made the T=1500 DiT call ~3 us slower).
struct CvtF16Pair {
    CvtF16Args v[2];
    uint32_t blocks0;
};
template <bool VEC>
__global__ __launch_bounds__(256) void cvt_f16_kernel(CvtF16Pair p) {
    const bool second = blockIdx.x >= p.blocks0;
    const CvtF16Args &a = second ? p.v[1] : p.v[0];
    const uint32_t t = (blockIdx.x - (second ? p.blocks0 : 0u)) * 256u + threadIdx.x;
    if (t >= (uint32_t)a.total) return;
    const uint32_t r = fdiv(t, a.div_chunks), i0 = 8u * (t - r * (uint32_t)a.chunks);
    const uint32_t r2 = fdiv(r, a.div_ne1), i1 = r - r2 * (uint32_t)a.ne1;
    const uint32_t i3 = fdiv(r2, a.div_ne2), i2 = r2 - i3 * (uint32_t)a.ne2;
    const float *row = (const float *)(a.src + (int64_t)i1 * a.nb1 + (int64_t)i2 * a.nb2 + (int64_t)i3 * a.nb3);
    float x[8];
    if constexpr (VEC) {
        const f4 lo = *(const f4 *)(row + i0);
        const f4 hi = *(const f4 *)(row + i0 + 4);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            x[j] = lo[j];
            x[4 + j] = hi[j];
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) x[j] = i0 + j < (uint32_t)a.ne0 ? row[i0 + j] : 0.0f;
    }
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) o[j] = __builtin_bit_cast(uint32_t, h2{(_Float16)x[2 * j], (_Float16)x[2 * j + 1]});
    *(u4 *)(a.dst + (int64_t)r * a.dst_row + i0) = u4{o[0], o[1], o[2], o[3]};
}

// ------------------------------------------------------------------------------------------
// ggml quantize_row_*_ref, one 32-element block per thread.  Contraction is disabled so each
// multiply/add rounds exactly like the reference C (x*id then +8.5f are separate roundings).
// ------------------------------------------------------------------------------------------
// fp32 -> fp16 (round to nearest even).  The sign bit is taken from the fp32 value: the
// backend may fold "x * c -> fp16" into an fma with a +0 addend, which turns -0 into +0
// (q4_0/q5_0 blocks of zeros have d = 0 / -8 = -0, and ggml stores that sign).
__device__ __forceinline__ void st_half(uint8_t *p, float f) {
    const _Float16 h = (_Float16)f;
    uint16_t bits = __builtin_bit_cast(uint16_t, h);
    bits = (uint16_t)((bits & 0x7fffu) | ((__builtin_bit_cast(uint32_t, f) >> 16) & 0x8000u));
    __builtin_memcpy(p, &bits, 2);
}

template <int T>
__device__ void quantize_block_ref(const float *x, uint8_t *y) {
#pragma clang fp contract(off)
    if constexpr (T == T_Q8_0) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        st_half(y, d);
        for (int j = 0; j < 32; j++) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
    } else if constexpr (T == T_Q4_0 || T == T_Q5_0) {
        constexpr float nlev = T == T_Q4_0 ? -8.0f : -16.0f;
        constexpr float off = T == T_Q4_0 ? 8.5f : 16.5f;
        constexpr int qmax = T == T_Q4_0 ? 15 : 31;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float v = x[j];
            if (amax < fabsf(v)) {
                amax = fabsf(v);
                max = v;
            }
        }
        const float d = max / nlev;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        st_half(y, d);
        uint32_t qh = 0;
        const int qs_off = T == T_Q4_0 ? 2 : 6;
        for (int j = 0; j < 16; j++) {
            const float x0 = x[j] * id;
            const float x1 = x[j + 16] * id;
            const int q0 = min(qmax, (int)(int8_t)(int)(x0 + off));
            const int q1 = min(qmax, (int)(int8_t)(int)(x1 + off));
            const uint8_t u0 = (uint8_t)q0, u1 = (uint8_t)q1;
            y[qs_off + j] = (uint8_t)((u0 & 0x0f) | ((u1 & 0x0f) << 4));
            qh |= ((uint32_t)(u0 & 0x10u) >> 4) << j;
            qh |= ((uint32_t)(u1 & 0x10u) >> 4) << (j + 16);
        }
        if constexpr (T == T_Q5_0) __builtin_memcpy(y + 2, &qh, 4);
    } else if constexpr (T == T_Q4_1 || T == T_Q5_1) {
        constexpr float nlev = T == T_Q4_1 ? 15.0f : 31.0f;
        float mn = 3.402823466e+38f, mx = -3.402823466e+38f;
        for (int j = 0; j < 32; j++) {
            const float v = x[j];
            if (v < mn) mn = v;
            if (v > mx) mx = v;
        }
        const float d = (mx - mn) / nlev;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        st_half(y, d);
        st_half(y + 2, mn);
        uint32_t qh = 0;
        const int qs_off = T == T_Q4_1 ? 4 : 8;
        for (int j = 0; j < 16; j++) {
            const float x0 = (x[j] - mn) * id;
            const float x1 = (x[j + 16] - mn) * id;
            uint8_t u0, u1;
            if constexpr (T == T_Q4_1) {
                u0 = (uint8_t)min(15, (int)(int8_t)(int)(x0 + 0.5f));
                u1 = (uint8_t)min(15, (int)(int8_t)(int)(x1 + 0.5f));
            } else {
                u0 = (uint8_t)(int)(x0 + 0.5f);
                u1 = (uint8_t)(int)(x1 + 0.5f);
            }
            y[qs_off + j] = (uint8_t)((u0 & 0x0f) | ((u1 & 0x0f) << 4));
            qh |= ((uint32_t)(u0 & 0x10u) >> 4) << j;
            qh |= ((uint32_t)(u1 & 0x10u) >> 4) << (j + 16);
        }
        if constexpr (T == T_Q5_1) __builtin_memcpy(y + 4, &qh, 4);
    }
}

// ------------------------------------------------------------------------------------------
// RoPE as ggml's CPU backend forms it (ggml_rope_ext, ext_factor 0, attn_factor 1): the angle of
// pair k is p times theta_scale k times (one float multiply per pair, in order), times
// freq_scale; cos/sin of that; x0*c - x1*s and x0*s + x1*c rounded product by product.
// ------------------------------------------------------------------------------------------
struct RopeAngle {
    float p, ts, fs, th;
    int k;  // pair whose angle th holds
    int kc; // pair whose cos/sin are held
    float c, s;
    __device__ void init(float pos, float theta_scale, float freq_scale) {
        p = pos;
        ts = theta_scale;
        fs = freq_scale;
        th = pos;
        k = 0;
        kc = -1;
    }
    // walks forward from the last pair asked for (from pair 0 when k goes back)
    __device__ void at(int kk) {
        if (kk == kc) return;
        if (kk < k) {
            th = p;
            k = 0;
        }
        while (k < kk) {
            th = th * ts;
            k++;
        }
        sincosf(fs * th, &s, &c);
        kc = kk;
    }
};

// Element i (< seg) of rope(x) for one rope input x[0..seg).
__device__ __forceinline__ float rope_value(const float *x, int i, int dims, bool neox, RopeAngle &A) {
#pragma clang fp contract(off)
    if (i >= dims) return x[i];
    int k, a, b;
    bool second;
    if (neox) {
        const int half = dims >> 1;
        second = i >= half;
        k = second ? i - half : i;
        a = k;
        b = k + half;
    } else {
        k = i >> 1;
        a = 2 * k;
        b = a + 1;
        second = (i & 1) != 0;
    }
    A.at(k);
    const float x0 = x[a], x1 = x[b];
    return second ? x0 * A.s + x1 * A.c : x0 * A.c - x1 * A.s;
}

// One thread per unit of two elements: rotated pair k (k < dims/2), or two copied tail elements.
// Every element is read and written by one thread, so dst may alias src.
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
#pragma clang fp contract(off)
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t units = a.ne0 >> 1;
    if (gid >= a.total / 2) return;
    const int64_t u = gid % units;
    int64_t r = gid / units;
    const int64_t i1 = r % a.ne1;
    r /= a.ne1;
    const int64_t i2 = r % a.ne2;
    const int64_t i3 = r / a.ne2;
    const float *x = (const float *)((const uint8_t *)a.src + i1 * a.src_nb1 + i2 * a.src_nb2 + i3 * a.src_nb3);
    float *y = (float *)((uint8_t *)a.dst + i1 * a.dst_nb1 + i2 * a.dst_nb2 + i3 * a.dst_nb3);
    const int half = a.rope_dims >> 1;
    if (u < half) {
        const int k = (int)u;
        const int ia = a.rope_neox ? k : 2 * k;
        const int ib = a.rope_neox ? k + half : 2 * k + 1;
        RopeAngle A;
        A.init((float)a.pos[i2], a.theta_scale, a.freq_scale);
        A.at(k);
        const float x0 = x[ia], x1 = x[ib];
        const float y0 = x0 * A.c - x1 * A.s;
        const float y1 = x0 * A.s + x1 * A.c;
        y[ia] = y0;
        y[ib] = y1;
    } else {
        const int64_t i = a.rope_dims + 2 * (u - half);
        const float x0 = x[i], x1 = x[i + 1];
        y[i] = x0;
        y[i + 1] = x1;
    }
}

template <int T, bool ROPE>
__global__ __launch_bounds__(256) void set_rows_kernel(SetRowsArgs a) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= a.total) return;
    constexpr int per = is_quant(T) ? 32 : 1;
    const int64_t units_per_row = a.ne0 / per;
    const int64_t e = gid % units_per_row;
    int64_t r = gid / units_per_row;
    const int64_t i01 = r % a.n_rows;
    r /= a.n_rows;
    const int64_t i02 = r % a.ne2;
    const int64_t i03 = r / a.ne2;
    const uint8_t *ip = a.idx + i01 * a.idx_nb0 + (i02 % a.idx_ne1) * a.idx_nb1 + (i03 % a.idx_ne2) * a.idx_nb2;
    int64_t i1;
    if (a.idx_i64) {
        __builtin_memcpy(&i1, ip, 8);
    } else {
        int32_t v;
        __builtin_memcpy(&v, ip, 4);
        i1 = v;
    }
    if (i1 < 0 || i1 >= a.dst_rows) return; // out-of-range positions write nothing
    const float *row = (const float *)(a.src + i01 * a.src_nb1 + i02 * a.src_nb2 + i03 * a.src_nb3);
    const float *x = row + e * per;
    uint8_t *y = a.dst + i1 * a.dst_nb1 + i02 * a.dst_nb2 + i03 * a.dst_nb3 + e * type_bytes(T);
    float xb[per];
    if constexpr (ROPE) {
        // the per elements of this unit, rotated within their rope input (head) of the row
        RopeAngle A;
        A.init((float)a.pos[i01 + a.n_rows * (i02 + a.ne2 * i03)], a.theta_scale, a.freq_scale);
        for (int j = 0; j < per; j++) {
            const int64_t c = e * per + j;
            const int64_t seg = c / a.rope_seg;
            xb[j] = rope_value(row + seg * a.rope_seg, (int)(c - seg * a.rope_seg), a.rope_dims, a.rope_neox != 0, A);
        }
    } else {
        for (int j = 0; j < per; j++) xb[j] = x[j];
    }
    if constexpr (T == T_F32) {
        __builtin_memcpy(y, &xb[0], 4);
    } else if constexpr (T == T_F16) {
        st_half(y, xb[0]);
    } else {
        quantize_block_ref<T>(xb, y);
    }
}

// ------------------------------------------------------------------------------------------
// DiT step inputs (src/cosyvoice-token2wav.cpp:273-302, src/cosyvoice-kv-cache.cpp:357-377).
// ------------------------------------------------------------------------------------------
// One workgroup per mask row: the row's block end is the first chunk boundary above it (the
// bounds are sorted; every thread scans them from the kernel arguments), then the row is filled
// with 0 before it and fp16 -inf from it on.
__global__ __launch_bounds__(256) void chunk_mask_kernel(ChunkMaskArgs a) {
    const int i = blockIdx.x;
    int end = a.n_cols;
    for (int b = 0; b < a.n_bounds; b++)
        if (a.bounds[b] > (uint32_t)i) {
            end = (int)min((uint32_t)a.n_cols, a.bounds[b]);
            break;
        }
    uint16_t *row = (uint16_t *)(a.mask + (int64_t)i * a.nb1);
    for (int j = threadIdx.x; j < a.n_cols; j += blockDim.x) row[j] = j < end ? (uint16_t)0 : (uint16_t)0xFC00;
}

__global__ __launch_bounds__(256) void fill_positions_kernel(int32_t *pos, int64_t n, int64_t total, int64_t nb1,
                                                            int32_t base) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    const int64_t j = gid % n, b = gid / n;
    *(int32_t *)((uint8_t *)pos + b * nb1 + 4 * j) = (int32_t)j + base;
}

// idx[i * n_embd + j] = (i / n_per_batch) * max_seq * n_embd + pos[i % n_per_batch] + j * max_seq,
// in 32-bit arithmetic as the host loop forms it.
__global__ __launch_bounds__(256) void v_idxs_kernel(int32_t *idx, const int32_t *pos, uint32_t n_tokens,
                                                    uint32_t n_per_batch, uint32_t n_embd, uint32_t max_seq) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (int64_t)n_tokens * n_embd) return;
    const uint32_t i = (uint32_t)(gid / n_embd), j = (uint32_t)(gid % n_embd);
    const int32_t base = (int32_t)((i / n_per_batch) * max_seq * n_embd) + pos[i % n_per_batch];
    idx[gid] = base + (int32_t)(j * max_seq);
}

// n_kv[i] += delta for i < n: the device-side length update of plans prepared with a device n_kv
// (the counterpart of shift_kv_node_pos, src/cosyvoice-kv-cache.cpp:398-408, inside a captured
// graph).
// Mask tile classes: one wave per (problem, row group, key tile); lane i reads query row q0+i of
// the block (row r of the kernel is query r / G, so a 64-row group spans at most 64 query rows).
// The block is all zero (+0 or -0), all -inf, prefix-shaped (each row 0 up to some key, -inf
// from there on; the lane writes its row's prefix length) or none of these, over the keys below
// n_kv (a tile the sequence ends inside is classified over its valid keys).  Only masks shared
// by every head and sequence are classified (plane 0).
// One block (row group rg, key tile kt) of a problem: lane i reads query row q0+i (64 keys as
// eight 16-byte pieces, all in flight at once).  A row of only +-0 or only -inf is told by two OR
// reductions over its 32 words; only rows with both (the edges of the visible region) are
// scanned key by key.  Writes the class byte and, for a prefix-shaped block, the 64 prefix
// lengths.
__device__ __forceinline__ void classify_block(const void *mask, int64_t m_nb1, int rg, int kt, int n_kv, int n_rows,
                                               int G, uint8_t *cls_out, uint8_t *bnd, int lane) {
    const int r0 = rg * 64, r1 = min(n_rows, r0 + 64) - 1;
    const int q0 = r0 / G, q1 = r1 / G;
    const int k0 = kt * 64;
    const int nv = min(64, n_kv - k0); // valid keys of the tile
    const int q = q0 + lane;
    const bool row = q <= q1 && nv > 0;
    bool any_nonzero = false, any_finite = false, bad = false; // bad: not prefix-shaped
    int first_inf = max(nv, 0);
    if (row) {
        gu8 *m = gptr(mask) + (int64_t)q * m_nb1 + (int64_t)k0 * 2;
        // whole pieces below n_kv as 16-byte loads, the piece n_kv ends inside key by key; keys
        // past n_kv are neither read nor counted (they read as -inf here, and the scan stops at
        // nv).  The piece conditions are uniform, and every load is issued before any use.
        u4 w[8];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            if (8 * c + 8 <= nv) {
                w[c] = ldg_u128(m + 16 * c);
            } else if (8 * c < nv) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int kk = 8 * c + 2 * i;
                    const uint32_t lo = kk < nv ? (uint32_t)ldg_u16(m + 2 * kk) : 0xfc00u;
                    const uint32_t hi = kk + 1 < nv ? (uint32_t)ldg_u16(m + 2 * kk + 2) : 0xfc00u;
                    w[c][i] = lo | (hi << 16);
                }
            } else {
                w[c] = u4{0xfc00fc00u, 0xfc00fc00u, 0xfc00fc00u, 0xfc00fc00u};
            }
        }
        uint32_t orz = 0, orn = 0; // OR of the magnitudes / of the differences from -inf
#pragma unroll
        for (int c = 0; c < 8; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                orz |= w[c][i] & 0x7fff7fffu;
                orn |= w[c][i] ^ 0xfc00fc00u;
            }
        if (nv == 64 && orz == 0) { // every key +-0
            any_finite = true;
        } else if (nv == 64 && orn == 0) { // every key -inf
            any_nonzero = true;
            first_inf = 0;
        } else {
            // an edge row: its first -inf key f, then one check that keys below f are +-0 and
            // keys from f on (below nv) are -inf; pieces and halves are compile-time indexes and
            // the bounds are compares, not branches
            int f = nv;
#pragma unroll
            for (int c = 0; c < 8; c++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t x = w[c][i];
                    const int k = 8 * c + 2 * i;
                    const int fk = (x & 0xffffu) == 0xfc00u ? k : (x >> 16) == 0xfc00u ? k + 1 : 64;
                    f = min(f, fk);
                }
            bool ok = true, nz = false, fin = false;
#pragma unroll
            for (int c = 0; c < 8; c++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t x = w[c][i];
                    const int k = 8 * c + 2 * i;
                    const uint32_t lo = x & 0xffffu, hi = x >> 16;
                    const bool lz = (lo & 0x7fffu) == 0u, hz = (hi & 0x7fffu) == 0u;
                    const bool li = lo == 0xfc00u, hi_i = hi == 0xfc00u;
                    // keys past nv read as -inf and count as neither
                    ok &= k >= nv || (k < f ? lz : li);
                    ok &= k + 1 >= nv || (k + 1 < f ? hz : hi_i);
                    nz |= (k < nv && !lz) || (k + 1 < nv && !hz);
                    fin |= (k < nv && !li) || (k + 1 < nv && !hi_i);
                }
            any_nonzero = nz;
            any_finite = fin;
            bad = !ok;
            first_inf = f;
        }
    }
    int cls = MCLS_MIXED;
    if (nv > 0) {
        const bool nz = __builtin_amdgcn_ballot_w64(any_nonzero) != 0;
        const bool fin = __builtin_amdgcn_ballot_w64(any_finite) != 0;
        const bool nonprefix = __builtin_amdgcn_ballot_w64(row && bad) != 0;
        cls = !nz ? MCLS_ZERO : !fin ? MCLS_OFF : !nonprefix ? MCLS_PREFIX : MCLS_MIXED;
        if (cls == MCLS_PREFIX) {
            // four lanes' lengths a dword (the table is 64-byte aligned): one 64-byte store, not
            // 64 byte stores
            const uint32_t b = (uint32_t)first_inf & 0xffu;
            const uint32_t b1 = __shfl_down(b, 1), b2 = __shfl_down(b, 2), b3 = __shfl_down(b, 3);
            if ((lane & 3) == 0) ((uint32_t *)bnd)[lane >> 2] = b | (b1 << 8) | (b2 << 16) | (b3 << 24);
        }
    }
    if (lane == 0) *cls_out = (uint8_t)cls;
}

template <bool BATCH>
__global__ __launch_bounds__(256) void mask_classify_kernel(FaArgs a) {
    const int lane = threadIdx.x & 63;
    // the wave's block (uniform: the problem lookup and its fields stay on the scalar unit)
    const int64_t blk = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (blk >= a.u.mcls_blocks) return;
    FaProblem P;
    if (!BATCH || a.u.n_problems == 1) {
        P = a.p0;
    } else {
        // the last problem whose first block is <= blk
        int lo = 0, hi = a.u.n_problems - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (a.table[mid].mcls_begin <= blk) lo = mid;
            else hi = mid - 1;
        }
        P = a.table[__builtin_amdgcn_readfirstlane(lo)];
    }
    const int nkt = P.mcls_ld;
    const int64_t local = blk - P.mcls_begin;
    const int rg = (int)(local / nkt), kt = (int)(local - (int64_t)rg * nkt);
    int n_kv = P.n_kv;
    if (P.n_kv_dev) n_kv = min(max(*P.n_kv_dev, 0), n_kv);
    classify_block(P.mask, P.m_nb1, rg, kt, n_kv, a.u.n_rows, a.u.G, P.mcls + local, mcls_bounds(P, a.u.mcls_blocks, local), lane);
}

// The one-problem launch with a host-set n_kv (every DiT call): its few arguments are scalars in
// the first kernel-argument dwords, which the compiled kernel receives in SGPRs (kernarg
// preloading takes scalar arguments, not aggregates), so a wave reads no argument memory before
// its mask loads: the kernel is two memory round trips (mask, class stores) instead of four.
__global__ __launch_bounds__(256) void mask_classify_one(const void *mask, uint8_t *mcls, int32_t m_nb1, int32_t nkt,
                                                         int32_t blocks, int32_t n_kv, int32_t n_rows, int32_t G) {
    const int lane = threadIdx.x & 63;
    const int blk = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (blk >= blocks) return;
    const int rg = blk / nkt, kt = blk - rg * nkt;
    classify_block(mask, m_nb1, rg, kt, n_kv, n_rows, G, mcls + blk, mcls + (blocks + 63) / 64 * 64 + (int64_t)blk * 64, lane);
}

hipError_t mask_classify_launch(const FaArgs &a, bool batch, hipStream_t st) {
    if (a.u.mcls_blocks <= 0) return hipSuccess;
    const unsigned grid = (unsigned)((a.u.mcls_blocks + 3) / 4);
    const FaProblem &p = a.p0;
    if ((!batch || a.u.n_problems == 1) && !p.n_kv_dev && p.m_nb1 <= INT32_MAX && a.u.mcls_blocks <= INT32_MAX / 64) {
        hipLaunchKernelGGL(mask_classify_one, dim3(grid), dim3(256), 0, st, (const void *)p.mask, p.mcls, (int32_t)p.m_nb1,
                           p.mcls_ld, (int32_t)a.u.mcls_blocks, p.n_kv, a.u.n_rows, a.u.G);
    } else if (batch) {
        hipLaunchKernelGGL(mask_classify_kernel<true>, dim3(grid), dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL(mask_classify_kernel<false>, dim3(grid), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void shift_n_kv_kernel(int32_t *n_kv, int32_t n, int32_t delta) {
    const int32_t i = (int32_t)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) n_kv[i] += delta;
}

// ------------------------------------------------------------------------------------------
// Host launchers.
// ------------------------------------------------------------------------------------------
hipError_t shift_n_kv_launch(int32_t *n_kv, int32_t n, int32_t delta, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(shift_n_kv_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, n_kv, n, delta);
    return hipGetLastError();
}

hipError_t chunk_mask_launch(const ChunkMaskArgs &a, hipStream_t st) {
    if (a.n_rows <= 0 || a.n_cols <= 0) return hipSuccess;
    hipLaunchKernelGGL(chunk_mask_kernel, dim3((unsigned)a.n_rows), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t fill_positions_launch(int32_t *pos, int64_t n, int64_t batch, int64_t nb1, int32_t base, hipStream_t st) {
    const int64_t total = n * batch;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_positions_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, pos, n, total,
                       nb1, base);
    return hipGetLastError();
}

hipError_t v_idxs_launch(int32_t *idx, const int32_t *pos, uint32_t n_tokens, uint32_t n_per_batch, uint32_t n_embd,
                         uint32_t max_seq, hipStream_t st) {
    const int64_t total = (int64_t)n_tokens * n_embd;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(v_idxs_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, idx, pos, n_tokens,
                       n_per_batch, n_embd, max_seq);
    return hipGetLastError();
}
hipError_t dequant_launch(int type, const void *src, float *dst, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    if (type == T_F32) {
        hipLaunchKernelGGL(copy_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           (const float *)src, dst, n);
        return hipGetLastError();
    }
    if (type == T_F16 && (n % 32) != 0) {
        hipLaunchKernelGGL(f16_to_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           (const _Float16 *)src, dst, n);
        return hipGetLastError();
    }
    const int64_t groups = n / 32;
    const unsigned grid = (unsigned)((groups * 4 + 255) / 256);
    const uint8_t *s = (const uint8_t *)src;
    switch (type) {
    case T_F16: hipLaunchKernelGGL(dequant_kernel<T_F16>, dim3(grid), dim3(256), 0, st, s, dst, groups); break;
    case T_Q8_0: hipLaunchKernelGGL(dequant_kernel<T_Q8_0>, dim3(grid), dim3(256), 0, st, s, dst, groups); break;
    case T_Q4_0: hipLaunchKernelGGL(dequant_kernel<T_Q4_0>, dim3(grid), dim3(256), 0, st, s, dst, groups); break;
    case T_Q4_1: hipLaunchKernelGGL(dequant_kernel<T_Q4_1>, dim3(grid), dim3(256), 0, st, s, dst, groups); break;
    case T_Q5_0: hipLaunchKernelGGL(dequant_kernel<T_Q5_0>, dim3(grid), dim3(256), 0, st, s, dst, groups); break;
    case T_Q5_1: hipLaunchKernelGGL(dequant_kernel<T_Q5_1>, dim3(grid), dim3(256), 0, st, s, dst, groups); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool ROPE>
static hipError_t set_rows_launch_t(int type, const SetRowsArgs &a, hipStream_t st) {
    const dim3 grid((unsigned)((a.total + 255) / 256)), block(256);
    switch (type) {
    case T_F32: hipLaunchKernelGGL((set_rows_kernel<T_F32, ROPE>), grid, block, 0, st, a); break;
    case T_F16: hipLaunchKernelGGL((set_rows_kernel<T_F16, ROPE>), grid, block, 0, st, a); break;
    case T_Q8_0: hipLaunchKernelGGL((set_rows_kernel<T_Q8_0, ROPE>), grid, block, 0, st, a); break;
    case T_Q4_0: hipLaunchKernelGGL((set_rows_kernel<T_Q4_0, ROPE>), grid, block, 0, st, a); break;
    case T_Q4_1: hipLaunchKernelGGL((set_rows_kernel<T_Q4_1, ROPE>), grid, block, 0, st, a); break;
    case T_Q5_0: hipLaunchKernelGGL((set_rows_kernel<T_Q5_0, ROPE>), grid, block, 0, st, a); break;
    case T_Q5_1: hipLaunchKernelGGL((set_rows_kernel<T_Q5_1, ROPE>), grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t set_rows_launch(int type, const SetRowsArgs &a, hipStream_t st) {
    if (a.total <= 0) return hipSuccess;
    return a.rope_dims > 0 ? set_rows_launch_t<true>(type, a, st) : set_rows_launch_t<false>(type, a, st);
}

hipError_t cvt_f16_launch(CvtF16Args *a, int n, hipStream_t st) {
    if (n < 1 || n > 2) return hipErrorInvalidValue;
    CvtF16Pair p;
    bool vec = true;
    int64_t blocks[2] = {0, 0};
    for (int i = 0; i < n; i++) {
        CvtF16Args &c = a[i];
        if (c.total < 0 || c.total > kCvtMaxChunks || c.dst_row % 8 || c.chunks * 8 != c.dst_row || c.ne0 > c.dst_row ||
            c.ne1 <= 0 || c.ne2 <= 0)
            return hipErrorInvalidValue;
        c.div_chunks = make_fastdiv((uint32_t)c.chunks);
        c.div_ne1 = make_fastdiv((uint32_t)c.ne1);
        c.div_ne2 = make_fastdiv((uint32_t)c.ne2);
        vec = vec && c.ne0 % 8 == 0 && (((uintptr_t)c.src | (uintptr_t)c.nb1 | (uintptr_t)c.nb2 | (uintptr_t)c.nb3) & 15) == 0;
        blocks[i] = (c.total + 255) / 256;
        p.v[i] = c;
    }
    if (n == 1) p.v[1] = p.v[0];
    p.blocks0 = (uint32_t)blocks[0];
    const int64_t grid = blocks[0] + blocks[1];
    if (grid == 0) return hipSuccess;
    if (vec) hipLaunchKernelGGL(cvt_f16_kernel<true>, dim3((unsigned)grid), dim3(256), 0, st, p);
    else hipLaunchKernelGGL(cvt_f16_kernel<false>, dim3((unsigned)grid), dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t rope_launch(const RopeArgs &a, hipStream_t st) {
    if (a.total <= 0) return hipSuccess;
    const int64_t units = a.total / 2;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, st, a);
    return hipGetLastError();
}

} // namespace cvattn
