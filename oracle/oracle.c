/*
 * oracle.c -- CPU restatement of the attention-path arithmetic (TEST INFRASTRUCTURE ONLY;
 * see oracle.h for what each function restates and how it is pinned).
 *
 * The ggml pieces (block layouts, *_ref quantizers, dequantizers, CPU vec-dot and the CPU
 * flash-attention loop) are restated from ggml's published algorithm.  ggml itself is not in
 * /root/reference: cosyvoice.cpp fetches it at configure time (cmake/Dependencies.cmake:98-106,
 * unpinned master for non-Metal builds).  Call sites that fix the semantics:
 *   src/cosyvoice-kv-cache.cpp:104-119  cache tensors [H_kv*D, max_seq, batch] of k_type/v_type
 *   src/cosyvoice-kv-cache.cpp:309-324  set_rows write + [D, n_kv, H_kv, B] permuted views
 *   src/cosyvoice-kv-cache.cpp:379-396  ggml_flash_attn_ext(q,k,v,mask,1/sqrt(D),0,0), prec F32;
 *                                       non-FA: mul_mat -> soft_max_ext -> mul_mat(V^T)
 *   src/cosyvoice-graph.cpp:357-377     DiT q/k/v views and the FA call
 *   src/cosyvoice-llm.cpp:20-29         causal mask; src/cosyvoice-token2wav.cpp:285-298 chunk mask
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------
 * IEEE binary16 <-> binary32, round to nearest even (what ggml's x86 F16C path does).
 * ---------------------------------------------------------------------------------------- */
uint16_t or_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) { /* inf or nan */
        if (a == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x1ffu));
    }
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (a >= 0x38800000u) {                                 /* normal half */
        const uint32_t mant = a & 0x7fffffu;
        const uint32_t e = (a >> 23) - 127u + 15u;
        uint32_t h = (e << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (a <= 0x33000000u) return (uint16_t)sign; /* <= 2^-25: rounds to (signed) zero */
    {
        /* subnormal half: units of 2^-24 */
        const uint32_t m = (a & 0x7fffffu) | 0x800000u;
        const uint32_t e = a >> 23;
        const uint32_t s = 126u - e; /* 14..24 */
        uint32_t h = m >> s;
        const uint32_t rem = m & ((1u << s) - 1u);
        const uint32_t half = 1u << (s - 1u);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
}

float or_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0x1fu) {
        x = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        x = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        x = sign;
    } else { /* subnormal: normalise */
        uint32_t ee = 113u;
        while (!(m & 0x400u)) {
            m <<= 1;
            ee--;
        }
        x = sign | (ee << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void or_fp32_to_fp16_row(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = or_fp32_to_fp16(x[i]);
}
void or_fp16_to_fp32_row(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = or_fp16_to_fp32(x[i]);
}

/* ------------------------------------------------------------------------------------------
 * Block layouts (ggml-common.h): 32 elements per block, little-endian, packed.
 *   q8_0 {half d; int8 qs[32]}                 34 B
 *   q8_1 {half d; half s; int8 qs[32]}         36 B   (vec-dot type only)
 *   q4_0 {half d; uint8 qs[16]}                18 B
 *   q4_1 {half d; half m; uint8 qs[16]}        20 B
 *   q5_0 {half d; uint8 qh[4]; uint8 qs[16]}   22 B
 *   q5_1 {half d; half m; uint8 qh[4]; uint8 qs[16]} 24 B
 * ---------------------------------------------------------------------------------------- */
#define QK 32

int64_t or_block_size(int type) {
    switch (type) {
    case OR_TYPE_F32:
    case OR_TYPE_F16: return 1;
    case OR_TYPE_Q4_0:
    case OR_TYPE_Q4_1:
    case OR_TYPE_Q5_0:
    case OR_TYPE_Q5_1:
    case OR_TYPE_Q8_0:
    case OR_TYPE_Q8_1: return QK;
    default: return 0;
    }
}

int64_t or_type_size(int type) {
    switch (type) {
    case OR_TYPE_F32: return 4;
    case OR_TYPE_F16: return 2;
    case OR_TYPE_Q4_0: return 18;
    case OR_TYPE_Q4_1: return 20;
    case OR_TYPE_Q5_0: return 22;
    case OR_TYPE_Q5_1: return 24;
    case OR_TYPE_Q8_0: return 34;
    case OR_TYPE_Q8_1: return 36;
    default: return 0;
    }
}

int64_t or_row_size(int type, int64_t n) {
    const int64_t bs = or_block_size(type);
    if (bs == 0 || n % bs) return -1;
    return n / bs * or_type_size(type);
}

static void put_half(uint8_t *p, float f) {
    const uint16_t h = or_fp32_to_fp16(f);
    p[0] = (uint8_t)(h & 0xff);
    p[1] = (uint8_t)(h >> 8);
}
static float get_half(const uint8_t *p) {
    return or_fp16_to_fp32((uint16_t)(p[0] | (p[1] << 8)));
}

/* quantize_row_q8_0_ref: d = amax/127, id = 1/d, q = roundf(x*id) (ties away from zero). */
static void quant_q8_0_ref(const float *x, uint8_t *y) {
    float amax = 0.0f;
    for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put_half(y, d);
    for (int j = 0; j < QK; j++) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

/* quantize_row_q4_0_ref: the signed element of largest magnitude (first on ties) maps to -8. */
static void quant_q4_0_ref(const float *x, uint8_t *y) {
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < QK; j++) {
        if (amax < fabsf(x[j])) {
            amax = fabsf(x[j]);
            max = x[j];
        }
    }
    const float d = max / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put_half(y, d);
    for (int j = 0; j < QK / 2; j++) {
        const float x0 = x[j] * id;
        const float x1 = x[j + QK / 2] * id;
        int q0 = (int8_t)(x0 + 8.5f);
        int q1 = (int8_t)(x1 + 8.5f);
        if (q0 > 15) q0 = 15;
        if (q1 > 15) q1 = 15;
        y[2 + j] = (uint8_t)((q0 & 0xff) | ((q1 & 0xff) << 4));
    }
}

/* quantize_row_q4_1_ref: d = (max-min)/15, m = min, q = min(15, (int8)((x-min)*id + 0.5)). */
static void quant_q4_1_ref(const float *x, uint8_t *y) {
    float min = FLT_MAX, max = -FLT_MAX;
    for (int j = 0; j < QK; j++) {
        if (x[j] < min) min = x[j];
        if (x[j] > max) max = x[j];
    }
    const float d = (max - min) / 15.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put_half(y, d);
    put_half(y + 2, min);
    for (int j = 0; j < QK / 2; j++) {
        const float x0 = (x[j] - min) * id;
        const float x1 = (x[j + QK / 2] - min) * id;
        int q0 = (int8_t)(x0 + 0.5f);
        int q1 = (int8_t)(x1 + 0.5f);
        if (q0 > 15) q0 = 15;
        if (q1 > 15) q1 = 15;
        y[4 + j] = (uint8_t)((q0 & 0xff) | ((q1 & 0xff) << 4));
    }
}

/* quantize_row_q5_0_ref: like q4_0 with 5 bits; the 5th bit of element j goes to qh bit j. */
static void quant_q5_0_ref(const float *x, uint8_t *y) {
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < QK; j++) {
        if (amax < fabsf(x[j])) {
            amax = fabsf(x[j]);
            max = x[j];
        }
    }
    const float d = max / -16.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put_half(y, d);
    uint32_t qh = 0;
    for (int j = 0; j < QK / 2; j++) {
        const float x0 = x[j] * id;
        const float x1 = x[j + QK / 2] * id;
        int q0 = (int8_t)(x0 + 16.5f);
        int q1 = (int8_t)(x1 + 16.5f);
        if (q0 > 31) q0 = 31;
        if (q1 > 31) q1 = 31;
        const uint8_t u0 = (uint8_t)q0, u1 = (uint8_t)q1;
        y[6 + j] = (uint8_t)((u0 & 0x0f) | ((u1 & 0x0f) << 4));
        qh |= ((uint32_t)(u0 & 0x10u) >> 4) << j;
        qh |= ((uint32_t)(u1 & 0x10u) >> 4) << (j + QK / 2);
    }
    memcpy(y + 2, &qh, 4);
}

/* quantize_row_q5_1_ref: d = (max-min)/31, m = min, q = (uint8)((x-min)*id + 0.5). */
static void quant_q5_1_ref(const float *x, uint8_t *y) {
    float min = FLT_MAX, max = -FLT_MAX;
    for (int j = 0; j < QK; j++) {
        if (x[j] < min) min = x[j];
        if (x[j] > max) max = x[j];
    }
    const float d = (max - min) / 31.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put_half(y, d);
    put_half(y + 2, min);
    uint32_t qh = 0;
    for (int j = 0; j < QK / 2; j++) {
        const float x0 = (x[j] - min) * id;
        const float x1 = (x[j + QK / 2] - min) * id;
        const uint8_t u0 = (uint8_t)(x0 + 0.5f);
        const uint8_t u1 = (uint8_t)(x1 + 0.5f);
        y[8 + j] = (uint8_t)((u0 & 0x0f) | ((u1 & 0x0f) << 4));
        qh |= ((uint32_t)(u0 & 0x10u) >> 4) << j;
        qh |= ((uint32_t)(u1 & 0x10u) >> 4) << (j + QK / 2);
    }
    memcpy(y + 4, &qh, 4);
}

int or_quantize_row(int type, const float *x, void *vy, int64_t k) {
    uint8_t *y = (uint8_t *)vy;
    const int64_t bs = or_block_size(type), ts = or_type_size(type);
    if (bs == 0 || k % bs) return -1;
    if (type == OR_TYPE_F32) {
        memcpy(y, x, (size_t)k * 4);
        return 0;
    }
    if (type == OR_TYPE_F16) {
        for (int64_t i = 0; i < k; i++) put_half(y + 2 * i, x[i]);
        return 0;
    }
    for (int64_t b = 0; b < k / QK; b++) {
        const float *xb = x + b * QK;
        uint8_t *yb = y + b * ts;
        switch (type) {
        case OR_TYPE_Q8_0: quant_q8_0_ref(xb, yb); break;
        case OR_TYPE_Q4_0: quant_q4_0_ref(xb, yb); break;
        case OR_TYPE_Q4_1: quant_q4_1_ref(xb, yb); break;
        case OR_TYPE_Q5_0: quant_q5_0_ref(xb, yb); break;
        case OR_TYPE_Q5_1: quant_q5_1_ref(xb, yb); break;
        default: return -1;
        }
    }
    return 0;
}

/* Dequantizers: y = code*d (+ m).  Every int*half product is exact in fp32; only "+m" rounds. */
int or_dequantize_row(int type, const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    const int64_t bs = or_block_size(type), ts = or_type_size(type);
    if (bs == 0 || k % bs) return -1;
    if (type == OR_TYPE_F32) {
        memcpy(y, x, (size_t)k * 4);
        return 0;
    }
    if (type == OR_TYPE_F16) {
        for (int64_t i = 0; i < k; i++) y[i] = get_half(x + 2 * i);
        return 0;
    }
    for (int64_t b = 0; b < k / QK; b++) {
        const uint8_t *xb = x + b * ts;
        float *yb = y + b * QK;
        const float d = get_half(xb);
        switch (type) {
        case OR_TYPE_Q8_0:
            for (int j = 0; j < QK; j++) yb[j] = (float)(int8_t)xb[2 + j] * d;
            break;
        case OR_TYPE_Q8_1:
            for (int j = 0; j < QK; j++) yb[j] = (float)(int8_t)xb[4 + j] * d;
            break;
        case OR_TYPE_Q4_0:
            for (int j = 0; j < QK / 2; j++) {
                yb[j] = (float)((xb[2 + j] & 0x0f) - 8) * d;
                yb[j + QK / 2] = (float)((xb[2 + j] >> 4) - 8) * d;
            }
            break;
        case OR_TYPE_Q4_1: {
            const float m = get_half(xb + 2);
            for (int j = 0; j < QK / 2; j++) {
                yb[j] = (float)(xb[4 + j] & 0x0f) * d + m;
                yb[j + QK / 2] = (float)(xb[4 + j] >> 4) * d + m;
            }
            break;
        }
        case OR_TYPE_Q5_0: {
            uint32_t qh;
            memcpy(&qh, xb + 2, 4);
            for (int j = 0; j < QK / 2; j++) {
                const int h0 = (int)((qh >> j) << 4) & 0x10;
                const int h1 = (int)(qh >> (j + 12)) & 0x10;
                yb[j] = (float)(((xb[6 + j] & 0x0f) | h0) - 16) * d;
                yb[j + QK / 2] = (float)(((xb[6 + j] >> 4) | h1) - 16) * d;
            }
            break;
        }
        case OR_TYPE_Q5_1: {
            const float m = get_half(xb + 2);
            uint32_t qh;
            memcpy(&qh, xb + 4, 4);
            for (int j = 0; j < QK / 2; j++) {
                const int h0 = (int)((qh >> j) << 4) & 0x10;
                const int h1 = (int)(qh >> (j + 12)) & 0x10;
                yb[j] = (float)((xb[8 + j] & 0x0f) | h0) * d + m;
                yb[j + QK / 2] = (float)((xb[8 + j] >> 4) | h1) * d + m;
            }
            break;
        }
        default: return -1;
        }
    }
    return 0;
}

/* ggml's x86 quantize_row_q8_0 / q8_1 (the CPU from_float of the vec-dot type): the
 * multiplier is 127/amax and rounding is to nearest even; q8_1 also stores s = d*sum(q). */
static float round_half_even(float v) {
    return nearbyintf(v); /* default FP environment rounds to nearest even */
}

void or_quantize_row_q8_0_cpu(const float *x, void *vy, int64_t k) {
    uint8_t *y = (uint8_t *)vy;
    for (int64_t b = 0; b < k / QK; b++) {
        const float *xb = x + b * QK;
        uint8_t *yb = y + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        put_half(yb, d);
        for (int j = 0; j < QK; j++) yb[2 + j] = (uint8_t)(int8_t)round_half_even(xb[j] * id);
    }
}

void or_quantize_row_q8_1_cpu(const float *x, void *vy, int64_t k) {
    uint8_t *y = (uint8_t *)vy;
    for (int64_t b = 0; b < k / QK; b++) {
        const float *xb = x + b * QK;
        uint8_t *yb = y + b * 36;
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        int sum = 0;
        put_half(yb, d);
        for (int j = 0; j < QK; j++) {
            const int q = (int)round_half_even(xb[j] * id);
            yb[4 + j] = (uint8_t)(int8_t)q;
            sum += q;
        }
        put_half(yb + 2, d * (float)sum);
    }
}

/* ------------------------------------------------------------------------------------------
 * Tensor access helpers.
 * ---------------------------------------------------------------------------------------- */
static const uint8_t *elem_ptr(const or_tensor *t, int64_t i1, int64_t i2, int64_t i3) {
    return (const uint8_t *)t->data + i1 * t->nb[1] + i2 * t->nb[2] + i3 * t->nb[3];
}

/* Row of ne0 elements at (i1,i2,i3) as fp32; rows of block types are contiguous blocks. */
static int load_row_f32(const or_tensor *t, int64_t i1, int64_t i2, int64_t i3, float *out) {
    const uint8_t *p = elem_ptr(t, i1, i2, i3);
    const int64_t n = t->ne[0];
    if (t->type == OR_TYPE_F32) {
        for (int64_t d = 0; d < n; d++) memcpy(&out[d], p + d * t->nb[0], 4);
        return 0;
    }
    if (t->type == OR_TYPE_F16) {
        for (int64_t d = 0; d < n; d++) out[d] = get_half(p + d * t->nb[0]);
        return 0;
    }
    return or_dequantize_row(t->type, p, out, n);
}

static float mask_value(const or_tensor *mask, int64_t j, int64_t i, int64_t h, int64_t b) {
    const uint8_t *mp = (const uint8_t *)mask->data + i * mask->nb[1] +
                        (h % mask->ne[2]) * mask->nb[2] + (b % mask->ne[3]) * mask->nb[3];
    return get_half(mp + j * 2);
}

static int check_fa_shapes(const or_tensor *q, const or_tensor *k, const or_tensor *v,
                           const or_tensor *mask) {
    if (q->ne[0] != k->ne[0]) return -1;
    if (k->ne[1] != v->ne[1]) return -1;
    if (k->ne[2] <= 0 || q->ne[2] % k->ne[2] || q->ne[2] % v->ne[2]) return -1;
    if (q->ne[3] % k->ne[3] || q->ne[3] % v->ne[3]) return -1;
    if (mask && (mask->ne[0] < k->ne[1] || mask->ne[1] < q->ne[1])) return -1;
    return 0;
}

/* ------------------------------------------------------------------------------------------
 * fp64 textbook attention with the ggml_flash_attn_ext contract:
 *   q [D, n_q, H, B], k [D, n_kv, H_kv, B], v [Dv, n_kv, H_kv, B], mask f16 [n_kv, >=n_q, 1|H, 1|B]
 *   kv head = h / (H/H_kv); -inf mask entries drop the key; a row with no key left -> 0;
 *   dst f32 [Dv, H, n_q, B] contiguous.
 * ---------------------------------------------------------------------------------------- */
int or_flash_attn_ext_f64(const or_tensor *q, const or_tensor *k, const or_tensor *v,
                          const or_tensor *mask, float *dst, float scale) {
    if (check_fa_shapes(q, k, v, mask)) return -1;
    const int64_t D = q->ne[0], nq = q->ne[1], H = q->ne[2], B = q->ne[3];
    const int64_t nkv = k->ne[1], Dv = v->ne[0];
    const int64_t rk2 = H / k->ne[2], rv2 = H / v->ne[2];
    const int64_t rk3 = B / k->ne[3], rv3 = B / v->ne[3];
    float *qrow = malloc(sizeof(float) * D);
    float *kf = malloc(sizeof(float) * D * (nkv ? nkv : 1));
    float *vf = malloc(sizeof(float) * Dv * (nkv ? nkv : 1));
    double *s = malloc(sizeof(double) * (nkv ? nkv : 1));
    double *acc = malloc(sizeof(double) * Dv);
    int rc = 0;
    for (int64_t b = 0; b < B && !rc; b++) {
        for (int64_t h = 0; h < H && !rc; h++) {
            const int64_t hk = h / rk2, hv = h / rv2;
            for (int64_t j = 0; j < nkv && !rc; j++) {
                rc |= load_row_f32(k, j, hk, b / rk3, kf + j * D);
                rc |= load_row_f32(v, j, hv, b / rv3, vf + j * Dv);
            }
            for (int64_t i = 0; i < nq && !rc; i++) {
                rc |= load_row_f32(q, i, h, b, qrow);
                double mx = -INFINITY;
                for (int64_t j = 0; j < nkv; j++) {
                    const double mv = mask ? (double)mask_value(mask, j, i, h, b) : 0.0;
                    if (mv == -INFINITY) {
                        s[j] = -INFINITY;
                        continue;
                    }
                    double dot = 0.0;
                    for (int64_t d = 0; d < D; d++) dot += (double)qrow[d] * (double)kf[j * D + d];
                    s[j] = dot * (double)scale + mv;
                    if (s[j] > mx) mx = s[j];
                }
                for (int64_t d = 0; d < Dv; d++) acc[d] = 0.0;
                double l = 0.0;
                if (mx != -INFINITY) {
                    for (int64_t j = 0; j < nkv; j++) {
                        if (s[j] == -INFINITY) continue;
                        const double p = exp(s[j] - mx);
                        l += p;
                        for (int64_t d = 0; d < Dv; d++) acc[d] += p * (double)vf[j * Dv + d];
                    }
                }
                float *o = dst + ((b * nq + i) * H + h) * Dv;
                for (int64_t d = 0; d < Dv; d++) o[d] = l > 0.0 ? (float)(acc[d] / l) : 0.0f;
            }
        }
    }
    free(qrow);
    free(kf);
    free(vf);
    free(s);
    free(acc);
    return rc;
}

/* ------------------------------------------------------------------------------------------
 * ggml CPU flash-attention loop, restated (ggml-cpu/ops.cpp,
 * ggml_compute_forward_flash_attn_ext_f16_one_chunk):
 *   Q is converted to K's vec-dot type (f16 for f16 K; q8_0 for q8_0/q4_0/q5_0 K; q8_1 for
 *   q4_1/q5_1 K; f32 stays f32), each key's score is vec_dot(K_j, Qc)*scale + mask, keys whose
 *   mask is -inf are skipped, and one online-softmax pass keeps M, S and an accumulator that is
 *   fp16 when V is f16 (fp32 otherwise).  The row result is acc * (S == 0 ? 0 : 1/S).
 * ---------------------------------------------------------------------------------------- */
static int vec_dot_type(int ktype) {
    switch (ktype) {
    case OR_TYPE_F32: return OR_TYPE_F32;
    case OR_TYPE_F16: return OR_TYPE_F16;
    case OR_TYPE_Q8_0:
    case OR_TYPE_Q4_0:
    case OR_TYPE_Q5_0: return OR_TYPE_Q8_0;
    case OR_TYPE_Q4_1:
    case OR_TYPE_Q5_1: return OR_TYPE_Q8_1;
    default: return -1;
    }
}

/* Integer codes of one 32-block (offset removed for _0 types, raw for _1 types). */
static void block_codes(int type, const uint8_t *xb, int32_t *c, float *d, float *m) {
    *d = get_half(xb);
    *m = 0.0f;
    switch (type) {
    case OR_TYPE_Q8_0:
        for (int j = 0; j < QK; j++) c[j] = (int8_t)xb[2 + j];
        break;
    case OR_TYPE_Q4_0:
        for (int j = 0; j < QK / 2; j++) {
            c[j] = (xb[2 + j] & 0x0f) - 8;
            c[j + 16] = (xb[2 + j] >> 4) - 8;
        }
        break;
    case OR_TYPE_Q4_1:
        *m = get_half(xb + 2);
        for (int j = 0; j < QK / 2; j++) {
            c[j] = xb[4 + j] & 0x0f;
            c[j + 16] = xb[4 + j] >> 4;
        }
        break;
    case OR_TYPE_Q5_0: {
        uint32_t qh;
        memcpy(&qh, xb + 2, 4);
        for (int j = 0; j < QK / 2; j++) {
            c[j] = ((xb[6 + j] & 0x0f) | ((int)((qh >> j) << 4) & 0x10)) - 16;
            c[j + 16] = ((xb[6 + j] >> 4) | ((int)(qh >> (j + 12)) & 0x10)) - 16;
        }
        break;
    }
    case OR_TYPE_Q5_1: {
        uint32_t qh;
        *m = get_half(xb + 2);
        memcpy(&qh, xb + 4, 4);
        for (int j = 0; j < QK / 2; j++) {
            c[j] = (xb[8 + j] & 0x0f) | ((int)((qh >> j) << 4) & 0x10);
            c[j + 16] = (xb[8 + j] >> 4) | ((int)(qh >> (j + 12)) & 0x10);
        }
        break;
    }
    default: break;
    }
}

/* vec_dot(K row, converted Q): quantized K against q8_0/q8_1 Q, f16 against f16, f32. */
static float vec_dot_k_q(int ktype, const uint8_t *krow, int64_t knb0, const void *qc, int64_t D) {
    if (ktype == OR_TYPE_F32) {
        const float *qf = (const float *)qc;
        float sum = 0.0f;
        for (int64_t d = 0; d < D; d++) {
            float kv;
            memcpy(&kv, krow + d * knb0, 4);
            sum += kv * qf[d];
        }
        return sum;
    }
    if (ktype == OR_TYPE_F16) {
        const uint16_t *qh = (const uint16_t *)qc;
        float sum = 0.0f;
        for (int64_t d = 0; d < D; d++) sum += get_half(krow + d * knb0) * or_fp16_to_fp32(qh[d]);
        return sum;
    }
    const int64_t ts = or_type_size(ktype);
    const uint8_t *qb = (const uint8_t *)qc;
    const int qts = vec_dot_type(ktype) == OR_TYPE_Q8_1 ? 36 : 34;
    const int qoff = qts == 36 ? 4 : 2;
    float sum = 0.0f;
    for (int64_t b = 0; b < D / QK; b++) {
        int32_t c[QK];
        float dk, mk;
        block_codes(ktype, krow + b * ts, c, &dk, &mk);
        const uint8_t *yb = qb + b * qts;
        const float dq = get_half(yb);
        int32_t isum = 0;
        for (int j = 0; j < QK; j++) isum += c[j] * (int8_t)yb[qoff + j];
        sum += dk * dq * (float)isum;
        if (qts == 36) sum += mk * get_half(yb + 2);
    }
    return sum;
}

typedef struct {
    const or_tensor *q, *k, *v, *mask;
    float *dst;
    float scale;
    int64_t row_begin, row_end;
    int rc;
} cpu_fa_job;

static void *cpu_fa_worker(void *arg) {
    cpu_fa_job *job = (cpu_fa_job *)arg;
    const or_tensor *q = job->q, *k = job->k, *v = job->v, *mask = job->mask;
    const int64_t D = q->ne[0], nq = q->ne[1], H = q->ne[2], B = q->ne[3];
    const int64_t nkv = k->ne[1], Dv = v->ne[0];
    const int64_t rk2 = H / k->ne[2], rv2 = H / v->ne[2];
    const int64_t rk3 = B / k->ne[3], rv3 = B / v->ne[3];
    const int vdt = vec_dot_type(k->type);
    float *qf = malloc(sizeof(float) * D);
    uint8_t *qc = malloc((size_t)(D * 4 + 64));
    float *acc32 = malloc(sizeof(float) * Dv);
    uint16_t *acc16 = malloc(sizeof(uint16_t) * Dv);
    float *v32 = malloc(sizeof(float) * Dv);
    for (int64_t r = job->row_begin; r < job->row_end; r++) {
        /* row order: query i fastest over heads? ggml iterates ir -> (iq1, iq2, iq3) with
         * iq1 (query) fastest; the split only changes which thread computes a row. */
        const int64_t i = r % nq, h = (r / nq) % H, b = r / (nq * H);
        if (load_row_f32(q, i, h, b, qf)) {
            job->rc = -1;
            break;
        }
        if (vdt == OR_TYPE_F32) {
            memcpy(qc, qf, sizeof(float) * D);
        } else if (vdt == OR_TYPE_F16) {
            or_fp32_to_fp16_row(qf, (uint16_t *)qc, D);
        } else if (vdt == OR_TYPE_Q8_0) {
            or_quantize_row_q8_0_cpu(qf, qc, D);
        } else {
            or_quantize_row_q8_1_cpu(qf, qc, D);
        }
        float S = 0.0f, M = -INFINITY;
        for (int64_t d = 0; d < Dv; d++) {
            acc32[d] = 0.0f;
            acc16[d] = 0;
        }
        const int64_t hk = h / rk2, hv = h / rv2;
        for (int64_t j = 0; j < nkv; j++) {
            const float mv = mask ? mask_value(mask, j, i, h, b) : 0.0f;
            if (mv == -INFINITY) continue;
            const uint8_t *krow = elem_ptr(k, j, hk, b / rk3);
            float s = vec_dot_k_q(k->type, krow, (int64_t)k->nb[0], qc, D);
            s = s * job->scale + mv;
            const float Mold = M;
            float ms = 1.0f, vs = 1.0f;
            const uint8_t *vrow = elem_ptr(v, j, hv, b / rv3);
            if (v->type == OR_TYPE_F16) {
                if (s > M) {
                    M = s;
                    ms = expf(Mold - M);
                    for (int64_t d = 0; d < Dv; d++)
                        acc16[d] = or_fp32_to_fp16(or_fp16_to_fp32(acc16[d]) * ms);
                } else {
                    vs = expf(s - M);
                }
                for (int64_t d = 0; d < Dv; d++)
                    acc16[d] = or_fp32_to_fp16(
                        fmaf(get_half(vrow + d * v->nb[0]), vs, or_fp16_to_fp32(acc16[d])));
            } else {
                if (s > M) {
                    M = s;
                    ms = expf(Mold - M);
                    for (int64_t d = 0; d < Dv; d++) acc32[d] *= ms;
                } else {
                    vs = expf(s - M);
                }
                if (load_row_f32(v, j, hv, b / rv3, v32)) {
                    job->rc = -1;
                    break;
                }
                for (int64_t d = 0; d < Dv; d++) acc32[d] = fmaf(v32[d], vs, acc32[d]);
            }
            S = S * ms + vs;
        }
        if (v->type == OR_TYPE_F16)
            for (int64_t d = 0; d < Dv; d++) acc32[d] = or_fp16_to_fp32(acc16[d]);
        const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
        float *o = job->dst + ((b * nq + i) * H + h) * Dv;
        for (int64_t d = 0; d < Dv; d++) o[d] = acc32[d] * S_inv;
    }
    free(qf);
    free(qc);
    free(acc32);
    free(acc16);
    free(v32);
    return NULL;
}

int or_flash_attn_ext_ggml_cpu(const or_tensor *q, const or_tensor *k, const or_tensor *v,
                               const or_tensor *mask, float *dst, float scale, int n_threads) {
    if (check_fa_shapes(q, k, v, mask)) return -1;
    if (vec_dot_type(k->type) < 0) return -1;
    if (or_block_size(k->type) > 1 && q->ne[0] % QK) return -1;
    const int64_t rows = q->ne[1] * q->ne[2] * q->ne[3];
    if (n_threads < 1) n_threads = 1;
    if (n_threads > rows) n_threads = (int)(rows > 0 ? rows : 1);
    cpu_fa_job *jobs = calloc((size_t)n_threads, sizeof(cpu_fa_job));
    pthread_t *th = calloc((size_t)n_threads, sizeof(pthread_t));
    const int64_t per = (rows + n_threads - 1) / n_threads;
    for (int t = 0; t < n_threads; t++) {
        jobs[t].q = q;
        jobs[t].k = k;
        jobs[t].v = v;
        jobs[t].mask = mask;
        jobs[t].dst = dst;
        jobs[t].scale = scale;
        jobs[t].row_begin = t * per < rows ? t * per : rows;
        jobs[t].row_end = (t + 1) * per < rows ? (t + 1) * per : rows;
        if (t > 0) pthread_create(&th[t], NULL, cpu_fa_worker, &jobs[t]);
    }
    cpu_fa_worker(&jobs[0]);
    int rc = jobs[0].rc;
    for (int t = 1; t < n_threads; t++) {
        pthread_join(th[t], NULL);
        rc |= jobs[t].rc;
    }
    free(jobs);
    free(th);
    return rc;
}

/* ------------------------------------------------------------------------------------------
 * Non-flash attention (src/cosyvoice-kv-cache.cpp:387-395, src/cosyvoice-graph.cpp:378-388):
 *   scores = mul_mat(K, Q) [n_kv, n_q, H, B]; W = soft_max_ext(scores, mask, scale);
 *   out = permute(mul_mat(V^T, W)) -> [Dv, H, n_q, B].  vt is the transposed-V view
 *   [n_kv, Dv, H_kv, B] (element (j, d) at j*nb0 + d*nb1), f32 or f16.
 * soft_max_ext takes the max over all keys including -inf ones; a fully masked row gives NaN
 * in ggml's CPU kernel; here it is reported as NaN as well.
 * ---------------------------------------------------------------------------------------- */
int or_attn_nonfa_f64(const or_tensor *q, const or_tensor *k, const or_tensor *vt,
                      const or_tensor *mask, float *dst, float scale) {
    const int64_t D = q->ne[0], nq = q->ne[1], H = q->ne[2], B = q->ne[3];
    const int64_t nkv = k->ne[1], Dv = vt->ne[1];
    if (vt->ne[0] != nkv || q->ne[0] != k->ne[0]) return -1;
    if (vt->type != OR_TYPE_F32 && vt->type != OR_TYPE_F16) return -1;
    const int64_t rk2 = H / k->ne[2], rv2 = H / vt->ne[2];
    const int64_t rk3 = B / k->ne[3], rv3 = B / vt->ne[3];
    float *qrow = malloc(sizeof(float) * D);
    float *kf = malloc(sizeof(float) * D);
    double *s = malloc(sizeof(double) * (nkv ? nkv : 1));
    int rc = 0;
    for (int64_t b = 0; b < B && !rc; b++)
        for (int64_t h = 0; h < H && !rc; h++)
            for (int64_t i = 0; i < nq && !rc; i++) {
                rc |= load_row_f32(q, i, h, b, qrow);
                double mx = -INFINITY;
                for (int64_t j = 0; j < nkv; j++) {
                    rc |= load_row_f32(k, j, h / rk2, b / rk3, kf);
                    double dot = 0.0;
                    for (int64_t d = 0; d < D; d++) dot += (double)qrow[d] * (double)kf[d];
                    const double mv = mask ? (double)mask_value(mask, j, i, h, b) : 0.0;
                    s[j] = dot * (double)scale + mv;
                    if (s[j] > mx) mx = s[j];
                }
                double l = 0.0;
                for (int64_t j = 0; j < nkv; j++) {
                    s[j] = exp(s[j] - mx);
                    l += s[j];
                }
                float *o = dst + ((b * nq + i) * H + h) * Dv;
                for (int64_t d = 0; d < Dv; d++) {
                    double acc = 0.0;
                    for (int64_t j = 0; j < nkv; j++) {
                        const uint8_t *p = (const uint8_t *)vt->data + j * vt->nb[0] +
                                           d * vt->nb[1] + (h / rv2) * vt->nb[2] +
                                           (b / rv3) * vt->nb[3];
                        float vv;
                        if (vt->type == OR_TYPE_F32)
                            memcpy(&vv, p, 4);
                        else
                            vv = get_half(p);
                        acc += s[j] * (double)vv;
                    }
                    o[d] = (float)(acc / l);
                }
            }
    free(qrow);
    free(kf);
    free(s);
    return rc;
}

/* ------------------------------------------------------------------------------------------
 * Masks and the KV write.
 * ---------------------------------------------------------------------------------------- */
/* src/cosyvoice-llm.cpp:20-29: row i of n_batch new tokens sees keys j <= seq_len-n_batch+i. */
void or_causal_mask(uint16_t *mask, uint32_t n_batch, uint32_t seq_len) {
    for (uint32_t i = 0; i < n_batch; i++)
        for (uint32_t j = 0; j < seq_len; j++)
            mask[(size_t)i * seq_len + j] = (j > seq_len - n_batch + i) ? 0xFC00u : 0u;
}

/* src/cosyvoice-token2wav.cpp:285-298: row i sees keys before the first chunk boundary > i
 * (or all n keys when no boundary exceeds i). */
void or_chunk_mask(uint16_t *mask, int64_t n, const uint32_t *bounds, int64_t n_bounds) {
    for (int64_t i = 0; i < n; i++) {
        int64_t end = n;
        for (int64_t t = 0; t < n_bounds; t++) {
            if ((int64_t)bounds[t] > i) {
                end = bounds[t];
                break;
            }
        }
        for (int64_t j = 0; j < n; j++) mask[i * n + j] = j < end ? 0u : 0xFC00u;
    }
}

int or_set_rows(void *dst, int dst_type, size_t dst_nb1, int64_t dst_rows, const float *src,
                size_t src_nb1, int64_t ne0, const int32_t *idx, int64_t n_rows) {
    if (or_row_size(dst_type, ne0) < 0) return -1;
    for (int64_t r = 0; r < n_rows; r++) {
        if (idx[r] < 0 || idx[r] >= dst_rows) return -1;
        const float *x = (const float *)((const uint8_t *)src + r * src_nb1);
        if (or_quantize_row(dst_type, x, (uint8_t *)dst + (size_t)idx[r] * dst_nb1, ne0)) return -1;
    }
    return 0;
}

/* ggml_rope_ext (ggml-cpu/ops.cpp rope_f32 with rope_cache_init / rope_yarn; not vendored), for
 * freq_factors NULL, ext_factor 0, attn_factor 1: the cache of (cos, sin) per pair is filled
 * from theta = p, multiplied by theta_scale after each pair; rope_yarn then takes
 * theta * freq_scale and cosf/sinf of it.  NORMAL rotates (x[2k], x[2k+1]); NEOX rotates
 * (x[k], x[k + n_dims/2]).  Called at src/cosyvoice-llm.cpp:56-57 and
 * src/cosyvoice-graph.cpp:351-352. */
int or_rope_f32(const float *src, float *dst, int64_t ne0, int64_t n_rows, const int32_t *pos, int n_dims,
                int mode, float freq_base, float freq_scale) {
    if (n_dims <= 0 || (n_dims & 1) || n_dims > ne0 || (ne0 & 1)) return -1;
    if (mode != OR_ROPE_NORMAL && mode != OR_ROPE_NEOX) return -1;
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    float *cs = (float *)malloc(sizeof(float) * (size_t)n_dims);
    if (!cs) return -1;
    for (int64_t r = 0; r < n_rows; r++) {
        const float *x = src + r * ne0;
        float *y = dst + r * ne0;
        float theta = (float)pos[r];
        for (int i0 = 0; i0 < n_dims; i0 += 2) {
            const float t = freq_scale * theta;
            cs[i0] = cosf(t);
            cs[i0 + 1] = sinf(t);
            theta *= theta_scale;
        }
        const int half = n_dims / 2;
        for (int i0 = 0; i0 < n_dims; i0 += 2) {
            const int a = mode == OR_ROPE_NEOX ? i0 / 2 : i0;
            const int b = mode == OR_ROPE_NEOX ? i0 / 2 + half : i0 + 1;
            const float c = cs[i0], sn = cs[i0 + 1];
            const float x0 = x[a], x1 = x[b];
            y[a] = x0 * c - x1 * sn;
            y[b] = x0 * sn + x1 * c;
        }
        for (int64_t i = n_dims; i < ne0; i++) y[i] = x[i];
    }
    free(cs);
    return 0;
}
