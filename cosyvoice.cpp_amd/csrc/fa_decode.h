// fa_decode.h -- decode-shaped flash attention for gfx950: at most 16 query rows per kv head
// (GQA decode over the LLM KV cache: the 7 q heads of a Qwen2-0.5B kv head times a few query
// tokens), the GGML_OP_FLASH_ATTN_EXT node of src/cosyvoice-kv-cache.cpp:383-384 in decode.
//
// The KV cache is streamed once.  A workgroup is 4 waves sharing the 16 query rows of one
// (batch, kv head); each wave owns a run of WLEN tokens and walks it in 64-token steps.  At the
// first step every load of the step is issued before any use; later steps are prefetched one
// step ahead.  K/V are read with bounds-checked buffer loads (rows past n_kv read as zeros).
//
// Per 16-token tile (v_mfma_f32_16x16x32_f16 with A = K rows, B = Q^T, see fa_impl.h for the
// operand layouts): the K A-operand (8 consecutive dims of one token) is loaded straight into
// registers and unpacked there; only the block scales go through LDS to reach the accumulator
// layout.  V is staged transposed in wave-private LDS for the P.V MFMA.  Softmax is base 2 with
// a lazily raised reference maximum (the O accumulators are rescaled only when a row's maximum
// grows by more than 2^8, so P stays <= 256 and fits fp16).
//
// Token splits: the waves of a workgroup merge their states in LDS; several workgroups of one
// (batch, kv head) write partials that the last one to arrive merges (prepared batches) or that
// fa_combine_kernel merges (single calls).
#pragma once

#include "fa_impl.h"

namespace cvattn {

constexpr int DEC_NW = 4;      // waves per workgroup
constexpr int DEC_TS = 64;     // tokens per wave step
constexpr int DEC_VSTR = 68;   // halfs per staged V^T row (64 tokens + pad)
constexpr float DEC_RESCALE_LOG2 = 8.0f;
constexpr int DEC_MERGE_CHUNK = 16; // split partials loaded together by the merging workgroup

// Buffer resource over [base, base + bytes); loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(gu8 *base, int64_t bytes) {
    const int32_t n = bytes > 0x7fffffff ? 0x7fffffff : (int32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, n, 0x00020000);
}

__device__ __forceinline__ uint32_t bld_u32(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ u2 bld_u64(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ u4 bld_u128(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t bld_u16(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// raw8_load through a buffer resource: dims [32*b + 8*c, +8) of the head row at byte `row`.
template <int T>
__device__ __forceinline__ void raw8_bload(__amdgpu_buffer_rsrc_t rs, int row, int b, int c, Raw8<T> &r) {
    r.dm = 0u;
    if constexpr (T == T_F32) {
        const u4 a = bld_u128(rs, row + (32 * b + 8 * c) * 4);
        const u4 e = bld_u128(rs, row + (32 * b + 8 * c) * 4 + 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            r.w[i] = a[i];
            r.w[4 + i] = e[i];
        }
    } else if constexpr (T == T_F16) {
        const u4 a = bld_u128(rs, row + (32 * b + 8 * c) * 2);
#pragma unroll
        for (int i = 0; i < 4; i++) r.w[i] = a[i];
    } else {
        const int blk = row + b * type_bytes(T);
        r.dm = has_min(T) ? bld_u32(rs, blk) : bld_u16(rs, blk);
        constexpr int qs_off = T == T_Q8_0 ? 2 : T == T_Q4_0 ? 2 : T == T_Q4_1 ? 4 : T == T_Q5_0 ? 6 : 8;
        const u2 q = bld_u64(rs, blk + qs_off + (T == T_Q8_0 ? 8 * c : 8 * (c & 1)));
        r.w[0] = q[0];
        r.w[1] = q[1];
        if constexpr (T == T_Q5_0 || T == T_Q5_1) r.w[2] = bld_u32(rs, blk + (T == T_Q5_0 ? 2 : 4));
    }
}

template <int KT, int VT>
struct DecRegs {
    Raw8<KT> k[4][2]; // K A-operand words: tile x block (this lane's token, dims 8g..8g+7)
    Raw8<VT> v[2][4]; // V staging items x 4 tokens
};

template <int KT>
__device__ __forceinline__ void dec_load_k(__amdgpu_buffer_rsrc_t rk, int64_t nb1, int t0, int t16, int g,
                                           Raw8<KT> (&k)[4][2]) {
#pragma unroll
    for (int tt = 0; tt < 4; tt++)
#pragma unroll
        for (int b = 0; b < 2; b++) raw8_bload<KT>(rk, (int)((t0 + 16 * tt + t16) * nb1), b, g, k[tt][b]);
}

template <int VT>
__device__ __forceinline__ void dec_load_v(__amdgpu_buffer_rsrc_t rv, int64_t nb1, int t0, int lane,
                                           Raw8<VT> (&v)[2][4]) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const Item it = item_of(lane + 64 * i);
#pragma unroll
        for (int j = 0; j < 4; j++) raw8_bload<VT>(rv, (int)((t0 + 4 * it.tq + j) * nb1), it.b, it.c, v[i][j]);
    }
}

template <int KT, int VT, bool MASK, bool BATCH>
__global__ __launch_bounds__(64 * DEC_NW) void fa_decode_kernel(FaArgs args) {
    __shared__ __attribute__((aligned(16))) _Float16 sV[DEC_NW][HEAD * DEC_VSTR];
    __shared__ __attribute__((aligned(16))) float sKd[DEC_NW][2][DEC_TS];
    __shared__ __attribute__((aligned(16))) float sKm[DEC_NW][2][DEC_TS];
    __shared__ __attribute__((aligned(16))) float sVd[DEC_NW][2][DEC_TS];
    __shared__ __attribute__((aligned(16))) float sVm[DEC_NW][2][DEC_TS];
    __shared__ uint32_t s_last;

    const FaUniform &U = args.u;
    FaProblem P;
    // consecutive units (the kv heads of one token range, whose rows share cache lines) run on
    // one XCD so each line is fetched into one L2 only
    const UnitPos pos = locate_unit<BATCH>(args, xcd_unit(blockIdx.x, gridDim.x), P);
    const int kh = pos.kh, rg = pos.rg, split = pos.split, bq = pos.bq;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int col = lane & 15, g = lane >> 4;

    const int t_begin = split * P.split_len;
    const int t_end = min(P.n_kv, t_begin + P.split_len);
    const int wlen = P.split_len / DEC_NW;
    const int w_begin = t_begin + wv * wlen;
    const int w_end = min(t_end, w_begin + wlen);
    const int nsteps = (min(wlen, max(0, t_end - t_begin)) + DEC_TS - 1) / DEC_TS; // uniform

    gu8 *kbase = gptr(P.k) + (int64_t)kh * P.k_nb2 + (int64_t)(bq / P.rk3) * P.k_nb3;
    gu8 *vbase = gptr(P.v) + (int64_t)kh * P.v_nb2 + (int64_t)(bq / P.rv3) * P.v_nb3;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, (int64_t)P.n_kv * P.k_nb1);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase, (int64_t)P.n_kv * P.v_nb1);

    // issue the first step's K/V loads before anything else
    DecRegs<KT, VT> R;
    if (nsteps > 0) {
        dec_load_k<KT>(rk, P.k_nb1, w_begin, col, g, R.k);
        dec_load_v<VT>(rv, P.v_nb1, w_begin, lane, R.v);
    }

    // ---- this lane's query row and its Q operand (hi + lo fp16) ----
    const int row = rg * 16 + col;
    const bool row_ok = row < U.n_rows;
    const int iq = row_ok ? row / U.G : 0;
    const int hq = kh * U.G + (row_ok ? row % U.G : 0);
    h8 qhi[2], qlo[2];
    float qsum[2];
    bool need_lo = false;
    {
        gu8 *qp = gptr(P.q) + (int64_t)iq * P.q_nb1 + (int64_t)hq * P.q_nb2 + (int64_t)bq * P.q_nb3;
        float x[2][8];
        if (U.q_f16) {
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int j = 0; j < 8; j++) x[b][j] = ldg_half(qp + 2 * (32 * b + 8 * g + j));
        } else {
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int j = 0; j < 8; j++) x[b][j] = as_f32(ldg_u32(qp + 4 * (32 * b + 8 * g + j)));
        }
#pragma unroll
        for (int b = 0; b < 2; b++) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float xs = row_ok ? x[b][j] * U.scale_log2 : 0.0f;
                const _Float16 hx = (_Float16)xs;
                const _Float16 lx = (_Float16)(xs - (float)hx);
                qhi[b][j] = hx;
                qlo[b][j] = lx;
                need_lo |= lx != (_Float16)0.0f;
                s += (float)hx + (float)lx;
            }
            qsum[b] = wave_sum16x4(s);
        }
    }
    need_lo = __syncthreads_or(need_lo) != 0;
    constexpr float kbias = stage_bias<KT>();
    const f4 cinit0 = {-kbias * qsum[0], -kbias * qsum[0], -kbias * qsum[0], -kbias * qsum[0]};
    const f4 cinit1 = {-kbias * qsum[1], -kbias * qsum[1], -kbias * qsum[1], -kbias * qsum[1]};

    gu8 *mrow = nullptr;
    if constexpr (MASK)
        mrow = gptr(P.mask) + (int64_t)iq * P.m_nb1 + (int64_t)(hq % P.m_ne2) * P.m_nb2 +
               (int64_t)(bq % P.m_ne3) * P.m_nb3;

    float m_ref = -INFINITY; // reference maximum (base 2) of this lane's row
    float l_run = 0.0f;
    float corr[2] = {0.0f, 0.0f};
    f4 oacc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) oacc[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    _Float16 *cV = sV[wv];
    for (int step = 0; step < nsteps; step++) {
        const int t0 = w_begin + step * DEC_TS;
        // ---- stage V^T and the block scales of K and V ----
#pragma unroll
        for (int i = 0; i < 2; i++) {
            Stage4<VT> s4;
#pragma unroll
            for (int j = 0; j < 4; j++) s4.r[j] = R.v[i][j];
            s4.valid = 0xfu; // rows past n_kv were read as zeros; past w_end they are masked
            stage_store_v<VT, DEC_VSTR, DEC_TS>(s4, item_of(lane + 64 * i), cV, sVd[wv], sVm[wv]);
        }
        if constexpr (is_quant(KT)) {
            if (g < 2) {
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    float d0, m0, d1, m1; // (select, not R.k[tt][g]: a lane-dependent index would
                    raw8_scales<KT>(R.k[tt][0], d0, m0); // move the array to scratch memory)
                    raw8_scales<KT>(R.k[tt][1], d1, m1);
                    const float d = g == 0 ? d0 : d1, m = g == 0 ? m0 : m1;
                    sKd[wv][g][16 * tt + col] = d;
                    if constexpr (has_min(KT)) sKm[wv][g][16 * tt + col] = m;
                }
            }
        }
        __syncthreads();
        if (step + 1 < nsteps) dec_load_v<VT>(rv, P.v_nb1, t0 + DEC_TS, lane, R.v);

        // ---- S^T = K Q^T for the four 16-token tiles ----
        f4 s[4];
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
            uint32_t a0w[4], a1w[4];
            raw8_unpack<KT>(R.k[tt][0], g, a0w);
            raw8_unpack<KT>(R.k[tt][1], g, a1w);
            const h8 a0 = as_h8(u4{a0w[0], a0w[1], a0w[2], a0w[3]});
            const h8 a1 = as_h8(u4{a1w[0], a1w[1], a1w[2], a1w[3]});
            f4 acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qhi[0], cinit0, 0, 0, 0);
            f4 acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qhi[1], cinit1, 0, 0, 0);
            if (need_lo) {
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qlo[0], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qlo[1], acc1, 0, 0, 0);
            }
            if constexpr (is_quant(KT)) {
                const f4 d0 = *(const f4 *)&sKd[wv][0][16 * tt + 4 * g];
                const f4 d1 = *(const f4 *)&sKd[wv][1][16 * tt + 4 * g];
                f4 v = d0 * acc0 + d1 * acc1;
                if constexpr (has_min(KT)) {
                    const f4 m0 = *(const f4 *)&sKm[wv][0][16 * tt + 4 * g];
                    const f4 m1 = *(const f4 *)&sKm[wv][1][16 * tt + 4 * g];
                    v += m0 * qsum[0] + m1 * qsum[1];
                }
                s[tt] = v;
            } else {
                s[tt] = acc0 + acc1;
            }
        }
        if (step + 1 < nsteps) dec_load_k<KT>(rk, P.k_nb1, t0 + DEC_TS, col, g, R.k);

        // ---- mask, range, softmax with a lazily raised reference maximum ----
        const bool full = t0 + DEC_TS <= w_end; // uniform
        float mx = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
            const int tb = t0 + 16 * tt + 4 * g;
            if constexpr (MASK) {
                if (full) {
                    const u2 mw = ldg_u64(mrow + (int64_t)tb * 2);
                    const h2 a = as_h2(mw[0]), c2 = as_h2(mw[1]);
                    s[tt][0] += (float)a[0] * 1.4426950408889634f;
                    s[tt][1] += (float)a[1] * 1.4426950408889634f;
                    s[tt][2] += (float)c2[0] * 1.4426950408889634f;
                    s[tt][3] += (float)c2[1] * 1.4426950408889634f;
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int t = tb + j;
                        const float mv = ldg_half(mrow + (int64_t)min(t, P.n_kv - 1) * 2);
                        s[tt][j] = t < w_end ? s[tt][j] + mv * 1.4426950408889634f : -INFINITY;
                    }
                }
            } else if (!full) {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (tb + j >= w_end) s[tt][j] = -INFINITY;
            }
#pragma unroll
            for (int j = 0; j < 4; j++) mx = fmaxf(mx, s[tt][j]);
        }
        mx = wave_max16x4(mx);
        // raise the reference only when the row maximum outgrows it by 2^8
        const bool raise = mx > m_ref + DEC_RESCALE_LOG2;
        const float m_new = raise ? mx : m_ref;
        if (__builtin_amdgcn_ballot_w64(raise && m_ref != -INFINITY)) { // uniform
            const float alpha = fast_exp2(m_ref - m_new);
            l_run *= alpha;
            corr[0] *= alpha;
            corr[1] *= alpha;
#pragma unroll
            for (int i = 0; i < 4; i++) oacc[i] *= alpha;
        }
        m_ref = m_new;
        const float m_use = m_ref == -INFINITY ? 0.0f : m_ref;
#pragma unroll
        for (int tt = 0; tt < 4; tt++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float p = fast_exp2(s[tt][j] - m_use);
                s[tt][j] = p;
                l_run += p;
            }

        // ---- O^T += V^T P^T ----
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            const f4 plo = s[2 * kb], phi = s[2 * kb + 1];
            h8 pb[2];
#pragma unroll
            for (int b = 0; b < 2; b++) {
                f4 xlo = plo, xhi = phi;
                if constexpr (is_quant(VT)) {
                    xlo = plo * *(const f4 *)&sVd[wv][b][32 * kb + 4 * g];
                    xhi = phi * *(const f4 *)&sVd[wv][b][32 * kb + 16 + 4 * g];
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    pb[b][j] = (_Float16)xlo[j];
                    pb[b][4 + j] = (_Float16)xhi[j];
                }
                if constexpr (has_min(VT)) {
                    const f4 mlo = *(const f4 *)&sVm[wv][b][32 * kb + 4 * g];
                    const f4 mhi = *(const f4 *)&sVm[wv][b][32 * kb + 16 + 4 * g];
                    const f4 t = plo * mlo + phi * mhi;
                    corr[b] += t[0] + t[1] + t[2] + t[3];
                }
                if constexpr (!is_quant(VT)) break;
            }
            if constexpr (!is_quant(VT)) pb[1] = pb[0];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int dim = 16 * i + col;
                const h4 va = *(const h4 *)&cV[dim * DEC_VSTR + 32 * kb + 4 * g];
                const h4 vb = *(const h4 *)&cV[dim * DEC_VSTR + 32 * kb + 16 + 4 * g];
                const h8 a = {va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
                oacc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb[i >> 1], oacc[i], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // ---------------- epilogue: merge the 4 waves (same rows, disjoint tokens) ----------------
    l_run = wave_sum16x4(l_run);
    if constexpr (has_min(VT)) {
        corr[0] = wave_sum16x4(corr[0]);
        corr[1] = wave_sum16x4(corr[1]);
#pragma unroll
        for (int i = 0; i < 4; i++) oacc[i] += corr[i >> 1];
    }
    float *xo = (float *)&sV[0][0];                  // [4][64 dims][16 rows]
    float *xm = (float *)&sKd[0][0][0];              // [4][16] m, then [4][16] l
    static_assert(sizeof(sV) >= DEC_NW * 64 * 16 * sizeof(float), "merge buffer");
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) xo[(wv * 64 + 16 * i + 4 * g + j) * 16 + col] = oacc[i][j];
    if (g == 0) {
        xm[wv * 16 + col] = m_ref;
        xm[DEC_NW * 16 + wv * 16 + col] = l_run;
    }
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < DEC_NW; w++) M = fmaxf(M, xm[w * 16 + col]);
    const float Mu = M == -INFINITY ? 0.0f : M;
    float L = 0.0f;
    f4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < DEC_NW; w++) {
        const float f = fast_exp2(xm[w * 16 + col] - Mu);
        L += xm[DEC_NW * 16 + w * 16 + col] * f;
#pragma unroll
        for (int j = 0; j < 4; j++) o[j] += xo[(w * 64 + 16 * wv + 4 * g + j) * 16 + col] * f;
    }
    // wave wv now owns dims 16*wv + 4g + j of row `col`
    const int ns = P.n_splits;
    const int64_t slot0 = P.part_begin + (((int64_t)bq * U.H_kv + kh) * U.n_rowgroups + rg) * 16 * ns;
    if (ns == 1) {
        if (row_ok) {
            const float inv = L > 0.0f ? 1.0f / L : 0.0f;
            float *out = P.dst + (((int64_t)bq * U.n_q + iq) * U.H + hq) * HEAD;
            *(f4 *)&out[16 * wv + 4 * g] = o * inv;
        }
        return;
    }
    if constexpr (!BATCH) {
        float *part = U.partials + (slot0 + (int64_t)col * ns + split) * PART_STRIDE;
        if (row_ok) {
            *(f4 *)&part[16 * wv + 4 * g] = o;
            if (wv == 0 && g == 0) {
                part[64] = M;
                part[65] = L;
            }
        }
        return;
    } else {
        // Partials of this (batch, kv head, row group): [16 rows][ns splits][PART_STRIDE floats],
        // written and read with agent-coherent (sc1) buffer accesses, the form the compiler gives
        // agent-scope atomic loads and stores, but vectorised and all in flight at once.
        constexpr int SC1 = 16;
        const __amdgpu_buffer_rsrc_t rp =
            make_rsrc((gu8 *)(U.partials + slot0 * PART_STRIDE), (int64_t)16 * ns * PART_STRIDE * 4);
        if (row_ok) {
            const int base = (col * ns + split) * PART_STRIDE * 4;
            __builtin_amdgcn_raw_buffer_store_b128(as_u4(o), rp, base + (16 * wv + 4 * g) * 4, 0, SC1);
            if (wv == 0 && g == 0)
                __builtin_amdgcn_raw_buffer_store_b64(u2{as_u32(M), as_u32(L)}, rp, base + 64 * 4, 0, SC1);
        }
        // once the partials have completed, the arrival count publishes them (a device-wide
        // fence would write back the whole L2)
        wait_memory();
        __syncthreads();
        if (tid == 0) {
            uint32_t *cnt = U.counters + P.cnt_begin + ((int64_t)bq * U.H_kv + kh) * U.n_rowgroups + rg;
            const uint32_t prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = prev == (uint32_t)(ns - 1);
            if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last ? 1u : 0u;
        }
        __syncthreads();
        if (!s_last) return;
        // last arrival: merge every split of its 16 rows; thread = (row, 4 dims); the loads of
        // up to DEC_MERGE_CHUNK splits are issued together
        const int r = tid >> 4, d0 = (tid & 15) * 4;
        const int rrow = rg * 16 + r;
        if (rrow >= U.n_rows) return;
        float Mm = -INFINITY, Ll = 0.0f;
        f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int c0 = 0; c0 < ns; c0 += DEC_MERGE_CHUNK) {
            u2 ml[DEC_MERGE_CHUNK];
            u4 ov[DEC_MERGE_CHUNK];
#pragma unroll
            for (int j = 0; j < DEC_MERGE_CHUNK; j++) {
                const int sp = min(c0 + j, ns - 1);
                const int base = (r * ns + sp) * PART_STRIDE * 4;
                ml[j] = __builtin_amdgcn_raw_buffer_load_b64(rp, base + 64 * 4, 0, SC1);
                ov[j] = __builtin_amdgcn_raw_buffer_load_b128(rp, base + d0 * 4, 0, SC1);
            }
            float cm = Mm;
#pragma unroll
            for (int j = 0; j < DEC_MERGE_CHUNK; j++)
                if (c0 + j < ns) cm = fmaxf(cm, as_f32(ml[j][0]));
            if (cm == -INFINITY) continue; // every row of these splits is fully masked so far
            const float a = fast_exp2(Mm - cm);
            Ll *= a;
            acc *= a;
#pragma unroll
            for (int j = 0; j < DEC_MERGE_CHUNK; j++) {
                if (c0 + j < ns) {
                    const float f = fast_exp2(as_f32(ml[j][0]) - cm);
                    Ll += as_f32(ml[j][1]) * f;
                    acc += as_f4(ov[j]) * f;
                }
            }
            Mm = cm;
        }
        const float inv = Ll > 0.0f ? 1.0f / Ll : 0.0f;
        const int riq = rrow / U.G, rhq = kh * U.G + rrow % U.G;
        *(f4 *)&P.dst[(((int64_t)bq * U.n_q + riq) * U.H + rhq) * HEAD + d0] = acc * inv;
    }
}

} // namespace cvattn
