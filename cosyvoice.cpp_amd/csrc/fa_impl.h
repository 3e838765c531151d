// fa_impl.h -- flash attention for gfx950 (the GGML_OP_FLASH_ATTN_EXT node of
// src/cosyvoice-kv-cache.cpp:383-384 and src/cosyvoice-graph.cpp:375-376).
//
// Rows.  For one (batch b, kv head kh) the rows are the n_q * G query rows sharing kh
// (G = H / H_kv), ordered r = i * G + g (query i, q head kh*G + g).  A wave owns 16 rows: the 16
// columns of its MFMA tiles.  For GQA decode the 7 q heads of a kv head are rows of one wave, so
// every K/V byte is read once for all of them.
//
// Two workgroup shapes (template WSPLIT):
//   WSPLIT (decode, <= 16 rows):  NW waves share one row group and split the workgroup's token
//       range; each wave stages its own 32-token tiles; the waves' softmax states are merged in
//       LDS at the end, so a workgroup writes one result (or one split partial).
//   rows   (prefill / DiT):       NW waves own 16 rows each (64 rows per workgroup) and share
//       64-token K/V tiles staged once in LDS.
// Token splits beyond one workgroup are merged by fa_combine_kernel.
//
// Per wave and 16-token tile (v_mfma_f32_16x16x32_f16, two 32-dim K halves):
//   S^T[t][r] = K[t][:] . Q[r][:]     A = K rows from LDS (natural layout), B = Q^T (registers)
// Q is pre-scaled by scale*log2(e), so softmax runs in base 2.  Quantized K is staged as fp16
// "1024 + u" codes; the MFMA accumulator starts at -(1024 + off)*sum(Q) so it ends as
// sum(code*Q), and the block scale d (and min m) are applied per token afterwards.
// The C layout of S^T (lane l: row l%16, tokens 4*(l/16)+j) is exactly the B layout of P^T for
//   O^T[dim][r] += V^T[dim][t] . P^T[t][r]   A = V^T from LDS (staged transposed), B = P^T
// when the 8 k-slots of lane group g are tokens {4g..4g+3} of one 16-token tile and
// {16+4g..16+4g+3} of the next.  V codes are staged exactly (fp16 small integers); the V block
// scale is folded into P (one B operand per 32-dim block) and the V min into a per-row term.
//
// Pipelining: the global loads of step s+1 are issued into registers before step s computes.
#pragma once

#include "cvattn_device.h"
#include "cvattn_launch.h"

namespace cvattn {

template <int NW, bool WSPLIT>
struct FaCfg {
    static constexpr int TSTEP = WSPLIT ? 32 : 64;  // tokens per staged tile
    static constexpr int NTILE = TSTEP / 16;         // 16-token S tiles per step
    static constexpr int NKB = TSTEP / 32;           // 32-token PV k-blocks per step
    static constexpr int KSTR = 72;                  // halfs per staged K row (64 + pad)
    static constexpr int VSTR = TSTEP + 4;           // halfs per staged V^T row (+ pad)
    static constexpr int NITEM = TSTEP * 2;          // staging items per tensor per tile
    static constexpr int NSTAGE = WSPLIT ? NW : 1;   // independent tile buffers
    static constexpr int ROWS = WSPLIT ? 16 : 16 * NW; // query rows per workgroup
    static constexpr int THREADS = 64 * NW;
    // staging items handled per thread per step (K and V counted together)
    static constexpr int ITEMS_PER_THREAD = WSPLIT ? 2 : (2 * NITEM) / THREADS;
};

// Index of the problem owning `key` in a table sorted by `field` (binary search; uniform).
template <int64_t FaProblem::*field>
__device__ __forceinline__ int find_problem(const FaProblem *table, int n, int64_t key) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (table[mid].*field <= key)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

// Staging item: 4 consecutive tokens x 8 consecutive dims of one 32-dim block.
struct Item {
    int c, b, tq;
};
__device__ __forceinline__ Item item_of(int it) { return Item{it & 3, (it >> 2) & 1, it >> 3}; }

template <int T>
struct Stage4 {
    Raw8 r[4];
};

template <int T>
__device__ __forceinline__ void stage_load(const uint8_t *base, int64_t nb1, int t0, int t_lim, Item it, Stage4<T> &s) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int t = t0 + 4 * it.tq + j;
        if (t < t_lim) {
            raw8_load<T>(base + (int64_t)t * nb1, it.b, it.c, s.r[j]);
        } else {
#pragma unroll
            for (int w = 0; w < 8; w++) s.r[j].w[w] = 0u;
            s.r[j].d = 0.0f;
            s.r[j].m = 0.0f;
        }
    }
}

// K tile: natural layout sK[t][dim], scales sKd/sKm[b][t].
template <int T, int KSTR, int TSTEP>
__device__ __forceinline__ void stage_store_k(const Stage4<T> &s, Item it, _Float16 *sK, float (*sKd)[TSTEP],
                                              float (*sKm)[TSTEP]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t o[4];
        raw8_unpack<T>(s.r[j], it.c, o);
        *(u4 *)&sK[(4 * it.tq + j) * KSTR + 32 * it.b + 8 * it.c] = u4{o[0], o[1], o[2], o[3]};
    }
    if constexpr (is_quant(T)) {
        if (it.c == 0) {
            *(f4 *)&sKd[it.b][4 * it.tq] = f4{s.r[0].d, s.r[1].d, s.r[2].d, s.r[3].d};
            if constexpr (has_min(T)) *(f4 *)&sKm[it.b][4 * it.tq] = f4{s.r[0].m, s.r[1].m, s.r[2].m, s.r[3].m};
        }
    }
}

// V tile: transposed sV[dim][t] holding the exact code (or value) as fp16, scales sVd/sVm[b][t].
template <int T, int VSTR, int TSTEP>
__device__ __forceinline__ void stage_store_v(const Stage4<T> &s, Item it, _Float16 *sV, float (*sVd)[TSTEP],
                                              float (*sVm)[TSTEP]) {
    constexpr float bias = stage_bias<T>();
    const h2 nb2 = {(_Float16)(-bias), (_Float16)(-bias)};
    h2 hv[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t o[4];
        raw8_unpack<T>(s.r[j], it.c, o);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            h2 x = __builtin_bit_cast(h2, o[i]);
            if constexpr (is_quant(T)) x = x + nb2;
            hv[j][i] = x;
        }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int i = e >> 1, k = e & 1;
        const h4 col4 = {hv[0][i][k], hv[1][i][k], hv[2][i][k], hv[3][i][k]};
        *(h4 *)&sV[(32 * it.b + 8 * it.c + e) * VSTR + 4 * it.tq] = col4;
    }
    if constexpr (is_quant(T)) {
        if (it.c == 0) {
            *(f4 *)&sVd[it.b][4 * it.tq] = f4{s.r[0].d, s.r[1].d, s.r[2].d, s.r[3].d};
            if constexpr (has_min(T)) *(f4 *)&sVm[it.b][4 * it.tq] = f4{s.r[0].m, s.r[1].m, s.r[2].m, s.r[3].m};
        }
    }
}

// Last-arriving workgroup of a split row group merges all split partials of its rows
// (prepared batches: no separate combine launch).  Returns true if this workgroup merged.
template <int ROWS, int THREADS>
__device__ __forceinline__ void merge_splits(const FaUniform &U, const FaProblem &P, int bq, int kh, int rg,
                                             int64_t slot0, int tid) {
    // slot of (row r, split s) = slot0 + r * n_splits + s
    constexpr int PER = ROWS * HEAD / THREADS; // outputs per thread
    static_assert(PER * THREADS == ROWS * HEAD, "merge tiling");
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int idx = tid + e * THREADS;
        const int r = idx / HEAD, d = idx % HEAD;
        const int row = rg * ROWS + r;
        if (row >= U.n_rows) continue;
        const float *part = U.partials + (slot0 + (int64_t)r * P.n_splits) * PART_STRIDE;
        float M = -INFINITY;
        for (int s = 0; s < P.n_splits; s++) M = fmaxf(M, part[s * PART_STRIDE + 64]);
        float L = 0.0f, acc = 0.0f;
        if (M != -INFINITY) {
            for (int s = 0; s < P.n_splits; s++) {
                const float *ps = part + s * PART_STRIDE;
                const float w = fast_exp2(ps[64] - M);
                L += ps[65] * w;
                acc += ps[d] * w;
            }
        }
        const int iq = row / U.G, hq = kh * U.G + row % U.G;
        P.dst[(((int64_t)bq * U.n_q + iq) * U.H + hq) * HEAD + d] = L > 0.0f ? acc / L : 0.0f;
    }
}

template <int NW, bool WSPLIT, int KT, int VT, bool MASK, bool BATCH>
__global__ __launch_bounds__(64 * NW) void fa_fwd_kernel(FaArgs args) {
    using C = FaCfg<NW, WSPLIT>;
    constexpr int TSTEP = C::TSTEP, NTILE = C::NTILE, NKB = C::NKB;
    constexpr int KSTR = C::KSTR, VSTR = C::VSTR, NITEM = C::NITEM, NSTAGE = C::NSTAGE;

    __shared__ __attribute__((aligned(16))) _Float16 sK[NSTAGE][TSTEP * KSTR];
    __shared__ __attribute__((aligned(16))) _Float16 sV[NSTAGE][HEAD * VSTR];
    __shared__ __attribute__((aligned(16))) float sKd[NSTAGE][2][TSTEP];
    __shared__ __attribute__((aligned(16))) float sKm[NSTAGE][2][TSTEP];
    __shared__ __attribute__((aligned(16))) float sVd[NSTAGE][2][TSTEP];
    __shared__ __attribute__((aligned(16))) float sVm[NSTAGE][2][TSTEP];

    const FaUniform &U = args.u;
    const int64_t unit = xcd_unit(blockIdx.x, gridDim.x);
    FaProblem P;
    if constexpr (BATCH)
        P = args.table[find_problem<&FaProblem::unit_begin>(args.table, U.n_problems, unit)];
    else
        P = args.p0;

    int64_t ul = unit - P.unit_begin;
    const int kh = (int)(ul % U.H_kv);
    ul /= U.H_kv;
    const int rg = (int)(ul % U.n_rowgroups);
    ul /= U.n_rowgroups;
    const int split = (int)(ul % P.n_splits);
    const int bq = (int)(ul / P.n_splits);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const int col = lane & 15; // MFMA column (query row) / A-operand row (token or dim)
    const int g = lane >> 4;   // lane group: k-slots 8g..8g+7, C rows 4g..4g+3
    const int st = WSPLIT ? wv : 0;

    // token range of this workgroup, and of this wave's tiles
    const int t_begin = split * P.split_len;
    const int t_end = min(P.n_kv, t_begin + P.split_len);
    const int wlen = WSPLIT ? P.split_len / NW : P.split_len;
    const int w_begin = WSPLIT ? t_begin + wv * wlen : t_begin;
    const int w_end = WSPLIT ? min(t_end, w_begin + wlen) : t_end;
    const int nsteps = (min(wlen, max(0, t_end - t_begin)) + TSTEP - 1) / TSTEP; // uniform in the workgroup

    const uint8_t *kbase = (const uint8_t *)P.k + (int64_t)kh * P.k_nb2 + (int64_t)(bq / P.rk3) * P.k_nb3;
    const uint8_t *vbase = (const uint8_t *)P.v + (int64_t)kh * P.v_nb2 + (int64_t)(bq / P.rv3) * P.v_nb3;

    // ---- this lane's query row and its Q operand (B of the S^T MFMA) ----
    const int row = rg * C::ROWS + (WSPLIT ? 0 : wv * 16) + col;
    const bool row_ok = row < U.n_rows;
    const int iq = row_ok ? row / U.G : 0;
    const int hq = kh * U.G + (row_ok ? row % U.G : 0);
    h8 qop[2];
    float qsum[2];
    {
        const uint8_t *qp = (const uint8_t *)P.q + (int64_t)iq * P.q_nb1 + (int64_t)hq * P.q_nb2 +
                            (int64_t)bq * P.q_nb3;
#pragma unroll
        for (int b = 0; b < 2; b++) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int d = 32 * b + 8 * g + j;
                float x = 0.0f;
                if (row_ok) x = U.q_f16 ? ldg_half(qp + 2 * d) : __builtin_bit_cast(float, ldg_u32(qp + 4 * d));
                const _Float16 hx = (_Float16)(x * U.scale_log2);
                qop[b][j] = hx;
                s += (float)hx;
            }
            qsum[b] = wave_sum16x4(s);
        }
    }
    constexpr float kbias = stage_bias<KT>();
    const f4 cinit0 = {-kbias * qsum[0], -kbias * qsum[0], -kbias * qsum[0], -kbias * qsum[0]};
    const f4 cinit1 = {-kbias * qsum[1], -kbias * qsum[1], -kbias * qsum[1], -kbias * qsum[1]};

    const uint8_t *mrow = nullptr;
    if constexpr (MASK) {
        mrow = (const uint8_t *)P.mask + (int64_t)iq * P.m_nb1 + (int64_t)(hq % P.m_ne2) * P.m_nb2 +
               (int64_t)(bq % P.m_ne3) * P.m_nb3;
    }

    float m_run = -INFINITY;
    float l_run = 0.0f;
    float corr[2] = {0.0f, 0.0f};
    f4 oacc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) oacc[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // ---- staging assignment ----
    // WSPLIT: every lane of a wave stages K item `lane` and V item `lane` of its own tile.
    // rows:   thread t < NITEM stages K item t, else V item t - NITEM (uniform per wave).
    const bool do_k = WSPLIT || tid < NITEM;
    const bool do_v = WSPLIT || tid >= NITEM;
    const Item itk = item_of(WSPLIT ? lane : tid);
    const Item itv = item_of(WSPLIT ? lane : tid - NITEM);
    Stage4<KT> rk;
    Stage4<VT> rv;
    if (nsteps > 0) {
        if (do_k) stage_load<KT>(kbase, P.k_nb1, w_begin, w_end, itk, rk);
        if (do_v) stage_load<VT>(vbase, P.v_nb1, w_begin, w_end, itv, rv);
    }

    for (int step = 0; step < nsteps; step++) {
        const int t0 = w_begin + step * TSTEP;
        if (do_k) stage_store_k<KT, KSTR, TSTEP>(rk, itk, sK[st], sKd[st], sKm[st]);
        if (do_v) stage_store_v<VT, VSTR, TSTEP>(rv, itv, sV[st], sVd[st], sVm[st]);
        __syncthreads();
        if (step + 1 < nsteps) { // next tile's loads fly while this one computes
            if (do_k) stage_load<KT>(kbase, P.k_nb1, t0 + TSTEP, w_end, itk, rk);
            if (do_v) stage_load<VT>(vbase, P.v_nb1, t0 + TSTEP, w_end, itv, rv);
        }

        // ---------------- S^T = K Q^T, tile by tile ----------------
        const _Float16 *cK = sK[st];
        f4 s[NTILE];
#pragma unroll
        for (int tt = 0; tt < NTILE; tt++) {
            const h8 a0 = *(const h8 *)&cK[(16 * tt + col) * KSTR + 8 * g];
            const h8 a1 = *(const h8 *)&cK[(16 * tt + col) * KSTR + 32 + 8 * g];
            const f4 acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qop[0], cinit0, 0, 0, 0);
            const f4 acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qop[1], cinit1, 0, 0, 0);
            if constexpr (is_quant(KT)) {
                const f4 d0 = *(const f4 *)&sKd[st][0][16 * tt + 4 * g];
                const f4 d1 = *(const f4 *)&sKd[st][1][16 * tt + 4 * g];
                f4 v = d0 * acc0 + d1 * acc1;
                if constexpr (has_min(KT)) {
                    const f4 m0 = *(const f4 *)&sKm[st][0][16 * tt + 4 * g];
                    const f4 m1 = *(const f4 *)&sKm[st][1][16 * tt + 4 * g];
                    v += m0 * qsum[0] + m1 * qsum[1];
                }
                s[tt] = v;
            } else {
                s[tt] = acc0 + acc1;
            }
        }

        // ---------------- mask, bounds, online softmax (base 2) ----------------
        float mx = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < NTILE; tt++) {
            const int tb = t0 + 16 * tt + 4 * g;
            if constexpr (MASK) {
                if (tb + 3 < w_end) {
                    const uint8_t *mp = mrow + (int64_t)tb * 2;
                    const h2 a = __builtin_bit_cast(h2, ldg_u32(mp));
                    const h2 c2 = __builtin_bit_cast(h2, ldg_u32(mp + 4));
                    s[tt][0] += (float)a[0] * 1.4426950408889634f;
                    s[tt][1] += (float)a[1] * 1.4426950408889634f;
                    s[tt][2] += (float)c2[0] * 1.4426950408889634f;
                    s[tt][3] += (float)c2[1] * 1.4426950408889634f;
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        s[tt][j] = tb + j < w_end ? s[tt][j] + ldg_half(mrow + (int64_t)(tb + j) * 2) * 1.4426950408889634f
                                                  : -INFINITY;
                }
            } else {
                if (tb + 3 >= w_end) {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if (tb + j >= w_end) s[tt][j] = -INFINITY;
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) mx = fmaxf(mx, s[tt][j]);
        }
        mx = wave_max16x4(mx);
        const float m_new = fmaxf(m_run, mx);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = fast_exp2(m_run - m_use);
        m_run = m_new;
        float psum = 0.0f;
#pragma unroll
        for (int tt = 0; tt < NTILE; tt++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float p = fast_exp2(s[tt][j] - m_use);
                s[tt][j] = p;
                psum += p;
            }
        l_run = l_run * alpha + psum;
        corr[0] *= alpha;
        corr[1] *= alpha;
#pragma unroll
        for (int i = 0; i < 4; i++) oacc[i] *= alpha;

        // ---------------- O^T += V^T P^T ----------------
        const _Float16 *cV = sV[st];
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const f4 plo = s[2 * kb], phi = s[2 * kb + 1];
            h8 pb[2];
#pragma unroll
            for (int b = 0; b < 2; b++) {
                f4 xlo = plo, xhi = phi;
                if constexpr (is_quant(VT)) {
                    xlo = plo * *(const f4 *)&sVd[st][b][32 * kb + 4 * g];
                    xhi = phi * *(const f4 *)&sVd[st][b][32 * kb + 16 + 4 * g];
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    pb[b][j] = (_Float16)xlo[j];
                    pb[b][4 + j] = (_Float16)xhi[j];
                }
                if constexpr (has_min(VT)) {
                    const f4 mlo = *(const f4 *)&sVm[st][b][32 * kb + 4 * g];
                    const f4 mhi = *(const f4 *)&sVm[st][b][32 * kb + 16 + 4 * g];
                    const f4 t = plo * mlo + phi * mhi;
                    corr[b] += t[0] + t[1] + t[2] + t[3];
                }
                if constexpr (!is_quant(VT)) break; // one B operand serves both blocks
            }
            if constexpr (!is_quant(VT)) pb[1] = pb[0];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int dim = 16 * i + col;
                const h4 va = *(const h4 *)&cV[dim * VSTR + 32 * kb + 4 * g];
                const h4 vb = *(const h4 *)&cV[dim * VSTR + 32 * kb + 16 + 4 * g];
                const h8 a = {va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
                oacc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb[i >> 1], oacc[i], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // ---------------- epilogue ----------------
    // partial slot of (row r of this row group, split s) = slot0 + r * n_splits + s
    const int64_t slot0 = P.part_begin + (((int64_t)bq * U.H_kv + kh) * U.n_rowgroups + rg) * C::ROWS * P.n_splits;
    l_run = wave_sum16x4(l_run);
    if constexpr (has_min(VT)) {
        corr[0] = wave_sum16x4(corr[0]);
        corr[1] = wave_sum16x4(corr[1]);
#pragma unroll
        for (int i = 0; i < 4; i++) oacc[i] += corr[i >> 1];
    }

    if constexpr (WSPLIT && NW > 1) {
        // merge the NW waves' states (same rows, disjoint tokens) through LDS
        float *xo = (float *)&sK[0][0];                    // [NW][64 dims][16 rows]
        float *xm = (float *)&sV[0][0];                    // [NW][16] m then [NW][16] l
        static_assert(sizeof(sK) >= NW * 64 * 16 * sizeof(float), "merge buffer");
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) xo[(wv * 64 + 16 * i + 4 * g + j) * 16 + col] = oacc[i][j];
        if (g == 0) {
            xm[wv * 16 + col] = m_run;
            xm[NW * 16 + wv * 16 + col] = l_run;
        }
        __syncthreads();
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, xm[w * 16 + col]);
        const float Mu = M == -INFINITY ? 0.0f : M;
        float L = 0.0f;
        f4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = fast_exp2(xm[w * 16 + col] - Mu);
            L += xm[NW * 16 + w * 16 + col] * f;
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] += xo[(w * 64 + 16 * wv + 4 * g + j) * 16 + col] * f;
        }
        // wave wv now owns dims 16*wv + 4g + j of row `col`
        if (row_ok) {
            if (P.n_splits == 1) {
                const float inv = L > 0.0f ? 1.0f / L : 0.0f;
                float *out = P.dst + (((int64_t)bq * U.n_q + iq) * U.H + hq) * HEAD;
                *(f4 *)&out[16 * wv + 4 * g] = o * inv;
            } else {
                float *out = U.partials + (slot0 + (int64_t)col * P.n_splits + split) * PART_STRIDE;
                *(f4 *)&out[16 * wv + 4 * g] = o;
                if (wv == 0 && g == 0) {
                    out[64] = M;
                    out[65] = L;
                }
            }
        }
    } else {
        if (row_ok) {
            if (P.n_splits == 1) {
                const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
                float *o = P.dst + (((int64_t)bq * U.n_q + iq) * U.H + hq) * HEAD;
#pragma unroll
                for (int i = 0; i < 4; i++) *(f4 *)&o[16 * i + 4 * g] = oacc[i] * inv;
            } else {
                float *o = U.partials + (slot0 + (int64_t)(row - rg * C::ROWS) * P.n_splits + split) * PART_STRIDE;
#pragma unroll
                for (int i = 0; i < 4; i++) *(f4 *)&o[16 * i + 4 * g] = oacc[i];
                if (g == 0) {
                    o[64] = m_run;
                    o[65] = l_run;
                }
            }
        }
    }

    // prepared batches: the last split of a row group to arrive merges the partials
    if constexpr (BATCH) {
        if (P.n_splits > 1) {
            __shared__ uint32_t s_last;
            __threadfence();
            __syncthreads();
            if (tid == 0) {
                uint32_t *cnt = U.counters + P.cnt_begin + ((int64_t)bq * U.H_kv + kh) * U.n_rowgroups + rg;
                const uint32_t prev = atomicAdd(cnt, 1u);
                const bool last = prev == (uint32_t)(P.n_splits - 1);
                if (last) atomicExch(cnt, 0u); // leave the counter zeroed for the next launch
                s_last = last ? 1u : 0u;
            }
            __syncthreads();
            if (s_last) {
                __threadfence();
                merge_splits<C::ROWS, C::THREADS>(U, P, bq, kh, rg, slot0, tid);
            }
        }
    }
}

// Merge split partials: one wave per output row (b, i, h); lane = output dim.
template <int ROWS, bool BATCH>
__global__ __launch_bounds__(64) void fa_combine_kernel(FaArgs args) {
    const FaUniform &U = args.u;
    const int64_t row = blockIdx.x;
    FaProblem P;
    if constexpr (BATCH)
        P = args.table[find_problem<&FaProblem::row_begin>(args.table, U.n_problems, row)];
    else
        P = args.p0;
    if (P.n_splits == 1) return;
    int64_t rl = row - P.row_begin;
    const int hq = (int)(rl % U.H);
    rl /= U.H;
    const int iq = (int)(rl % U.n_q);
    const int bq = (int)(rl / U.n_q);
    const int kh = hq / U.G;
    const int r = iq * U.G + hq % U.G;
    const int rg = r / ROWS, rr = r % ROWS;
    const int64_t slot0 = P.part_begin + ((((int64_t)bq * U.H_kv + kh) * U.n_rowgroups + rg) * ROWS + rr) * P.n_splits;
    const float *part = U.partials + slot0 * PART_STRIDE;
    const int d = threadIdx.x;
    float M = -INFINITY;
    for (int s = 0; s < P.n_splits; s++) M = fmaxf(M, part[s * PART_STRIDE + 64]);
    float L = 0.0f, acc = 0.0f;
    if (M != -INFINITY) {
        for (int s = 0; s < P.n_splits; s++) {
            const float *ps = part + s * PART_STRIDE;
            const float w = fast_exp2(ps[64] - M);
            L += ps[65] * w;
            acc += ps[d] * w;
        }
    }
    P.dst[(((int64_t)bq * U.n_q + iq) * U.H + hq) * HEAD + d] = L > 0.0f ? acc / L : 0.0f;
}

using FaLaunchFn = hipError_t (*)(const FaArgs &, hipStream_t);

template <int NW, bool WSPLIT, int KT, int VT, bool MASK, bool BATCH>
hipError_t launch_fa(const FaArgs &a, hipStream_t st) {
    if (a.u.total_units <= 0) return hipSuccess;
    hipLaunchKernelGGL((fa_fwd_kernel<NW, WSPLIT, KT, VT, MASK, BATCH>), dim3((unsigned)a.u.total_units),
                       dim3(64 * NW), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // single calls merge split partials with a second launch; prepared batches merge in-kernel
    if (!BATCH && a.p0.n_splits > 1 && a.u.total_rows > 0) {
        hipLaunchKernelGGL((fa_combine_kernel<FaCfg<NW, WSPLIT>::ROWS, BATCH>), dim3((unsigned)a.u.total_rows),
                           dim3(64), 0, st, a);
        e = hipGetLastError();
    }
    return e;
}

// Launch table [mask][batch][k type index][v type index]; index order f32 f16 q8_0 q4_0 q4_1 q5_0 q5_1.
#define CVATTN_V_ROW(NW, WS, KT, MASK, BATCH)                                                       \
    {launch_fa<NW, WS, KT, T_F32, MASK, BATCH>, launch_fa<NW, WS, KT, T_F16, MASK, BATCH>,          \
     launch_fa<NW, WS, KT, T_Q8_0, MASK, BATCH>, launch_fa<NW, WS, KT, T_Q4_0, MASK, BATCH>,        \
     launch_fa<NW, WS, KT, T_Q4_1, MASK, BATCH>, launch_fa<NW, WS, KT, T_Q5_0, MASK, BATCH>,        \
     launch_fa<NW, WS, KT, T_Q5_1, MASK, BATCH>}
#define CVATTN_TABLE(NW, WS, MASK, BATCH)                                                            \
    {CVATTN_V_ROW(NW, WS, T_F32, MASK, BATCH), CVATTN_V_ROW(NW, WS, T_F16, MASK, BATCH),            \
     CVATTN_V_ROW(NW, WS, T_Q8_0, MASK, BATCH), CVATTN_V_ROW(NW, WS, T_Q4_0, MASK, BATCH),          \
     CVATTN_V_ROW(NW, WS, T_Q4_1, MASK, BATCH), CVATTN_V_ROW(NW, WS, T_Q5_0, MASK, BATCH),          \
     CVATTN_V_ROW(NW, WS, T_Q5_1, MASK, BATCH)}

} // namespace cvattn
