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
    // the K tile buffers double as the split-merge scratch
    static constexpr int MERGE_MAX_SPLITS = (NSTAGE * TSTEP * KSTR * 2 / 4) / (2 * ROWS);
};

// Index of the problem owning `key` in a table sorted by `field`: start at the proportional
// guess (exact when all problems have the same size) and walk; uniform across the workgroup.
template <int64_t FaProblem::*field>
__device__ __forceinline__ int find_problem(const FaProblem *table, int n, int64_t key, int64_t total) {
    int i = total > 0 ? (int)min<int64_t>(n - 1, key * n / total) : 0;
    while (i > 0 && table[i].*field > key) i--;
    while (i + 1 < n && table[i + 1].*field <= key) i++;
    return i;
}

// Problem of workgroup unit `unit` in a table whose unit_begin values ascend: each lane of the
// wave compares one entry, so 64 problems cost one round trip.  Uniform across the workgroup.
__device__ __forceinline__ int find_problem_wave(const FaProblem *table, int n, uint32_t unit) {
    int cnt = 0;
    for (int c0 = 0; c0 < n; c0 += 64) {
        const int i = c0 + (int)(threadIdx.x & 63);
        const bool le = i < n && table[i].unit_begin <= (int64_t)unit;
        cnt += __popcll(__builtin_amdgcn_ballot_w64(le));
    }
    return cnt - 1;
}

// Position of a workgroup unit inside its problem: unit = ((bq*n_splits + split)*n_khg + khg)*
// n_rowgroups + rg, counted from the problem's unit_begin (khg: kv-head group, one kv head
// unless the decode kernel pairs heads).  Row groups are innermost so that the units of one XCD
// (see xcd_unit) share the K/V of few heads in that XCD's L2.
struct UnitPos {
    int kh, rg, split, bq;
};
template <bool BATCH>
__device__ __forceinline__ UnitPos locate_unit(const FaArgs &args, uint32_t unit, FaProblem &P) {
    const FaUniform &U = args.u;
    uint32_t ul = unit;
    if (!BATCH || U.n_problems == 1) {
        P = args.p0;
    } else if (U.units_per_problem > 0) {
        const uint32_t pi = fdiv(unit, U.div_upp);
        P = args.table[pi];
        ul = unit - pi * (uint32_t)U.units_per_problem;
    } else {
        P = args.table[find_problem_wave(args.table, U.n_problems, unit)];
        ul = unit - (uint32_t)P.unit_begin;
    }
    UnitPos r;
    uint32_t t = fdiv(ul, U.div_rowgroups);
    r.rg = (int)(ul - t * (uint32_t)U.n_rowgroups);
    ul = t;
    t = fdiv(ul, U.div_khg);
    r.kh = (int)(ul - t * (uint32_t)U.n_khg);
    ul = t;
    t = fdiv(ul, P.div_splits);
    r.split = (int)(ul - t * (uint32_t)P.n_splits);
    r.bq = (int)t;
    return r;
}

// Staging item: 4 consecutive tokens x 8 consecutive dims of one 32-dim block.
struct Item {
    int c, b, tq;
};
__device__ __forceinline__ Item item_of(int it) { return Item{it & 3, (it >> 2) & 1, it >> 3}; }

template <int T>
struct Stage4 {
    Raw8<T> r[4];
    uint32_t valid; // bit j: token j of the item is inside the wave's range
};

// Issue the loads of one staging item.  Rows past `t_lim` read row min(t, n_kv-1) (always in
// bounds) and are zeroed when stored; nothing here touches the loaded registers, so the loads
// stay in flight while the current tile computes.
template <int T>
__device__ __forceinline__ void stage_load(gu8 *base, int64_t nb1, int t0, int t_lim, int n_kv, Item it,
                                           Stage4<T> &s) {
    s.valid = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int t = t0 + 4 * it.tq + j;
        raw8_load<T>(base + (int64_t)min(t, n_kv - 1) * nb1, it.b, it.c, s.r[j]);
        s.valid |= (t < t_lim ? 1u : 0u) << j;
    }
}

template <int T>
__device__ __forceinline__ void stage_unpack(const Stage4<T> &s, int j, int c, uint32_t o[4], float &d, float &m) {
    const bool ok = (s.valid >> j) & 1u;
    raw8_unpack<T>(s.r[j], c, o);
    if (!ok) {
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = is_quant(T) ? 0x64006400u : 0u; // code 0 / value 0
    }
    raw8_scales<T>(s.r[j], d, m);
    d = ok ? d : 0.0f;
    m = ok ? m : 0.0f;
}

// K tile: natural layout sK[t][dim], scales sKd/sKm[b][t].
template <int T, int KSTR, int TSTEP>
__device__ __forceinline__ void stage_store_k(const Stage4<T> &s, Item it, _Float16 *sK, float (*sKd)[TSTEP],
                                              float (*sKm)[TSTEP]) {
    float d[4], m[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t o[4];
        stage_unpack<T>(s, j, it.c, o, d[j], m[j]);
        *(u4 *)&sK[(4 * it.tq + j) * KSTR + 32 * it.b + 8 * it.c] = u4{o[0], o[1], o[2], o[3]};
    }
    if constexpr (is_quant(T)) {
        if (it.c == 0) {
            *(f4 *)&sKd[it.b][4 * it.tq] = f4{d[0], d[1], d[2], d[3]};
            if constexpr (has_min(T)) *(f4 *)&sKm[it.b][4 * it.tq] = f4{m[0], m[1], m[2], m[3]};
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
    float d[4], m[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t o[4];
        stage_unpack<T>(s, j, it.c, o, d[j], m[j]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            h2 x = as_h2(o[i]);
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
            *(f4 *)&sVd[it.b][4 * it.tq] = f4{d[0], d[1], d[2], d[3]};
            if constexpr (has_min(T)) *(f4 *)&sVm[it.b][4 * it.tq] = f4{m[0], m[1], m[2], m[3]};
        }
    }
}

// Last-arriving workgroup of a split row group merges all split partials of its rows
// (prepared batches: no separate combine launch).  Three phases so the global loads run in
// parallel: (1) every split's (m, l) of every row into LDS, (2) one thread per row turns them
// into normalised split weights, (3) each thread sums its outputs over the splits.
// `scratch` holds 2 * ROWS * n_splits floats (n_splits <= MERGE_MAX_SPLITS).
template <int ROWS, int THREADS>
__device__ __forceinline__ void merge_splits(const FaUniform &U, const FaProblem &P, int bq, int kh, int rg,
                                             int64_t slot0, int tid, float *scratch) {
    const int ns = P.n_splits;
    float *sm = scratch;             // [ROWS][ns] m, then normalised weights
    float *sl = scratch + ROWS * ns; // [ROWS][ns] l
    for (int idx = tid; idx < ROWS * ns; idx += THREADS) {
        const float *ps = U.partials + (slot0 + idx) * PART_STRIDE; // slot0 + r*ns + s == slot0 + idx
        sm[idx] = ld_agent(ps + 64);
        sl[idx] = ld_agent(ps + 65);
    }
    __syncthreads();
    if (tid < ROWS) {
        float M = -INFINITY;
        for (int s = 0; s < ns; s++) M = fmaxf(M, sm[tid * ns + s]);
        float L = 0.0f;
        if (M != -INFINITY)
            for (int s = 0; s < ns; s++) {
                const float w = fast_exp2(sm[tid * ns + s] - M);
                sm[tid * ns + s] = w;
                L += sl[tid * ns + s] * w;
            }
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        for (int s = 0; s < ns; s++) sm[tid * ns + s] = M != -INFINITY ? sm[tid * ns + s] * inv : 0.0f;
    }
    __syncthreads();
    constexpr int PER = ROWS * HEAD / THREADS; // outputs per thread
    static_assert(PER * THREADS == ROWS * HEAD, "merge tiling");
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int idx = tid + e * THREADS;
        const int r = idx / HEAD, d = idx % HEAD;
        const int row = rg * ROWS + r;
        if (row >= U.n_rows) continue;
        const float *part = U.partials + (slot0 + (int64_t)r * ns) * PART_STRIDE + d;
        float acc = 0.0f;
#pragma unroll 8
        for (int s = 0; s < ns; s++) acc += sm[r * ns + s] * ld_agent(part + (int64_t)s * PART_STRIDE);
        const int iq = row / U.G, hq = kh * U.G + row % U.G;
        P.dst[(((int64_t)bq * U.n_q + iq) * U.H + hq) * HEAD + d] = acc;
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
    FaProblem P;
    const UnitPos pos = locate_unit<BATCH>(args, xcd_unit(blockIdx.x, gridDim.x), P);
    const int kh = pos.kh, rg = pos.rg, split = pos.split, bq = pos.bq;

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

    gu8 *kbase = gptr(P.k) + (int64_t)kh * P.k_nb2 + (int64_t)(bq / P.rk3) * P.k_nb3;
    gu8 *vbase = gptr(P.v) + (int64_t)kh * P.v_nb2 + (int64_t)(bq / P.rv3) * P.v_nb3;

    // ---- this lane's query row and its Q operand (B of the S^T MFMA) ----
    const int row = rg * C::ROWS + (WSPLIT ? 0 : wv * 16) + col;
    const bool row_ok = row < U.n_rows;
    const int iq = row_ok ? row / U.G : 0;
    const int hq = kh * U.G + (row_ok ? row % U.G : 0);
    // Q*scale*log2(e) = hi + lo, both fp16: two MFMAs make the QK products fp32-accurate
    // (lo is zero when Q is f16 and the scale is a power of two, and its MFMA is skipped then).
    h8 qhi[2], qlo[2];
    float qsum[2];
    bool need_lo = false;
    {
        gu8 *qp = gptr(P.q) + (int64_t)iq * P.q_nb1 + (int64_t)hq * P.q_nb2 + (int64_t)bq * P.q_nb3;
        // independent scalar loads, all issued before any use (16-byte vector loads of Q were
        // miscompiled here by the ROCm 7.2 compiler: only two lanes of each load survived)
        float x[2][8];
        if (U.q_f16) { // uniform
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int j = 0; j < 8; j++) x[b][j] = ldg_half(qp + 2 * (32 * b + 8 * g + j));
        } else {
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int j = 0; j < 8; j++)
                    x[b][j] = as_f32(ldg_u32(qp + 4 * (32 * b + 8 * g + j)));
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
    if constexpr (MASK) {
        mrow = gptr(P.mask) + (int64_t)iq * P.m_nb1 + (int64_t)(hq % P.m_ne2) * P.m_nb2 +
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
        if (do_k) stage_load<KT>(kbase, P.k_nb1, w_begin, w_end, P.n_kv, itk, rk);
        if (do_v) stage_load<VT>(vbase, P.v_nb1, w_begin, w_end, P.n_kv, itv, rv);
    }

    for (int step = 0; step < nsteps; step++) {
        const int t0 = w_begin + step * TSTEP;
        if (do_k) stage_store_k<KT, KSTR, TSTEP>(rk, itk, sK[st], sKd[st], sKm[st]);
        if (do_v) stage_store_v<VT, VSTR, TSTEP>(rv, itv, sV[st], sVd[st], sVm[st]);
        __syncthreads();
        if (step + 1 < nsteps) { // next tile's loads fly while this one computes
            if (do_k) stage_load<KT>(kbase, P.k_nb1, t0 + TSTEP, w_end, P.n_kv, itk, rk);
            if (do_v) stage_load<VT>(vbase, P.v_nb1, t0 + TSTEP, w_end, P.n_kv, itv, rv);
        }

        // ---------------- S^T = K Q^T, tile by tile ----------------
        const _Float16 *cK = sK[st];
        f4 s[NTILE];
#pragma unroll
        for (int tt = 0; tt < NTILE; tt++) {
            const h8 a0 = *(const h8 *)&cK[(16 * tt + col) * KSTR + 8 * g];
            const h8 a1 = *(const h8 *)&cK[(16 * tt + col) * KSTR + 32 + 8 * g];
            f4 acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qhi[0], cinit0, 0, 0, 0);
            f4 acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qhi[1], cinit1, 0, 0, 0);
            if (need_lo) {
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qlo[0], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qlo[1], acc1, 0, 0, 0);
            }
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
        const bool full = t0 + TSTEP <= w_end; // uniform: the whole tile is in range
#pragma unroll
        for (int tt = 0; tt < NTILE; tt++) {
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
            } else {
                if (!full) {
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
                if constexpr (BATCH) {
#pragma unroll
                    for (int j = 0; j < 4; j++) st_agent(&out[16 * wv + 4 * g + j], o[j]);
                    if (wv == 0 && g == 0) {
                        st_agent(&out[64], M);
                        st_agent(&out[65], L);
                    }
                } else {
                    *(f4 *)&out[16 * wv + 4 * g] = o;
                    if (wv == 0 && g == 0) {
                        out[64] = M;
                        out[65] = L;
                    }
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
                if constexpr (BATCH) {
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int j = 0; j < 4; j++) st_agent(&o[16 * i + 4 * g + j], oacc[i][j]);
                    if (g == 0) {
                        st_agent(&o[64], m_run);
                        st_agent(&o[65], l_run);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++) *(f4 *)&o[16 * i + 4 * g] = oacc[i];
                    if (g == 0) {
                        o[64] = m_run;
                        o[65] = l_run;
                    }
                }
            }
        }
    }

    // prepared batches: the last split of a row group to arrive merges the partials
    if constexpr (BATCH) {
        if (P.n_splits > 1) {
            // partials were stored with agent-scope stores; once they have completed, the
            // arrival count publishes them (no device-wide fence, which would flush the L2)
            __shared__ uint32_t s_last;
            wait_memory();
            __syncthreads();
            if (tid == 0) {
                uint32_t *cnt = U.counters + P.cnt_begin + ((int64_t)bq * U.H_kv + kh) * U.n_rowgroups + rg;
                const uint32_t prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const bool last = prev == (uint32_t)(P.n_splits - 1);
                // the last arrival leaves the counter zeroed for the next launch
                if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_last = last ? 1u : 0u;
            }
            __syncthreads();
            if (s_last) merge_splits<C::ROWS, C::THREADS>(U, P, bq, kh, rg, slot0, tid, (float *)&sK[0][0]);
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
        P = args.table[find_problem<&FaProblem::row_begin>(args.table, U.n_problems, row, U.total_rows)];
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
    const int ns = P.n_splits;
    float M = -INFINITY;
#pragma unroll 8
    for (int s = 0; s < ns; s++) M = fmaxf(M, part[s * PART_STRIDE + 64]);
    float L = 0.0f, acc = 0.0f;
    if (M != -INFINITY) {
#pragma unroll 8
        for (int s = 0; s < ns; s++) {
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
