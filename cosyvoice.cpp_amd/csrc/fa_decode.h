// fa_decode.h -- decode-shaped flash attention for gfx950: at most 64 query rows per kv head, in
// row groups of 16 (GQA decode over the LLM KV cache: the 7 q heads of a Qwen2-0.5B kv head times
// a few query tokens, or the 50-row chunk of a DiT streaming step), the GGML_OP_FLASH_ATTN_EXT
// node of src/cosyvoice-kv-cache.cpp:383-384 in decode.
//
// The KV cache is streamed once, in whole ggml blocks.  A workgroup is 4 independent waves on
// one (batch, kv head, row group, token split); each wave walks its own run of tokens in steps
// of 32 and never waits for the other waves until the end.
//
// Per wave step:
//   * every lane loads one 32-dim block of K and one of V (16-byte buffer loads of whole blocks;
//     64 lanes cover 32 consecutive tokens of the head, so a wave's loads are contiguous runs),
//     PD steps ahead of use;
//   * the lane unpacks its blocks into a wave-private LDS tile of fp16 rows [token][64 dims]
//     (K codes as "1024 + u", V codes exact) plus fp32 block scales;
//   * S^T = K Q^T with v_mfma_f32_16x16x32_f16 (A = K rows read from the tile, B = Q^T in
//     registers, split into fp16 hi + lo parts for fp32-accurate scores);
//   * softmax in base 2 with a lazily raised reference maximum;
//   * O^T += V^T P^T with v_mfma_f32_16x16x16_f16: the S^T accumulator of a 16-token tile is
//     already the B operand of P^T, and ds_read_b64_tr_b16 reads V^T straight from the
//     token-major V tile.
//
// Token splits: the waves of a workgroup merge their states in LDS; several workgroups of one
// group write partials that the last one to arrive merges (prepared batches) or that
// dec_combine_kernel merges (single calls).
#pragma once

#include "fa_impl.h"

namespace cvattn {

constexpr int DEC_NW = 4;      // waves per workgroup
constexpr int DEC_RS = 72;     // halfs per canonical LDS row (64 dims + pad): 144 B
constexpr float DEC_RESCALE_LOG2 = 8.0f;
// Token splits per merge round of the last-arriving workgroup: all loads of a round are issued
// at once.  Past 16 splits a second round costs more than the streaming it shortens for 4096-token
// sequences (the 24-layer q8_0/q4_0 step and the one-layer launch both measured best at 16), so
// the planner goes to two rounds (DEC_MAX_SPLITS) only for sequences long enough that 16 splits
// would leave a workgroup more than DEC_LONG_SPLIT tokens.
constexpr int DEC_MERGE_CHUNK = 16;
constexpr int DEC_MAX_SPLITS = 2 * DEC_MERGE_CHUNK;
constexpr int DEC_LONG_SPLIT = 256;

// Steps whose raw blocks are in flight at once (register budget per type pair).
template <int KT, int VT>
__host__ __device__ constexpr int dec_prefetch() {
    return blk_words<KT>() + blk_words<VT>() <= 16 ? 3 : blk_words<KT>() + blk_words<VT>() <= 32 ? 2 : 1;
}

// Query row of row slot `slot` (0..15) of a (kv head, row group); false if unused.
__device__ __forceinline__ bool dec_row(const FaUniform &U, int kh, int rg, int slot, int &iq, int &hq) {
    const int rr = rg * 16 + slot;
    const bool ok = rr < U.n_rows;
    const int r = ok ? rr : 0;
    iq = r / U.G;
    hq = kh * U.G + r % U.G;
    return ok;
}

// Split partials of one (batch, kv head, row group): O[ns][16 row slots][64] (a split's rows are
// one contiguous store run, and a merge load of one split covers 16 consecutive 256-byte rows)
// followed by (m, l)[16 row slots][nsp][2] with nsp = ns rounded up to even (16-byte rows); this
// fits in the 16 * ns * PART_STRIDE floats the host reserves per group.
__device__ __forceinline__ int dec_ml_offset(int ns) { return 16 * ns * 64; }
__device__ __forceinline__ int dec_nsp(int ns) { return (ns + 1) & ~1; }

// Merge the ns (<= DEC_MAX_SPLITS) split partials of one group's 16 row slots into dst; thread =
// (slot, 4 dims).  Splits are merged in rounds of DEC_MERGE_CHUNK: every load of a round is
// issued before any is used, and every lane of a row loads all of the round's (m, l) pairs of the
// row (the same bytes for the row's 16 lanes), so the weights need no cross-lane exchange.  A
// second round rescales the running sum to the new maximum.
// SC1: the partials were written by other workgroups of the same launch (agent-coherent loads).
template <bool SC1>
__device__ __forceinline__ void dec_merge(const FaUniform &U, float *dst, float *part0, int ns, int kh, int rg,
                                          int bq) {
    const int tid = threadIdx.x;
    const int r = tid >> 4, q = tid & 15, d0 = 4 * q;
    int iq, hq;
    const bool ok = dec_row(U, kh, rg, r, iq, hq); // uniform over the row's 16 lanes
    constexpr int AUX = SC1 ? 16 : 0;
    const int nsp = dec_nsp(ns);
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc((gu8 *)part0, (int64_t)(dec_ml_offset(ns) + 16 * nsp * 2) * 4);
    // Loads of row slots past the group's rows (never written) and of splits past ns point
    // outside the resource: they return 0 without a memory access, and need no branch.
    constexpr int kOutside = 0x7ffffff0;
    float M = -INFINITY, L = 0.0f;
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c0 = 0; c0 < ns; c0 += DEC_MERGE_CHUNK) { // one round, or two (uniform)
        u4 ov[DEC_MERGE_CHUNK];
        u4 ml[DEC_MERGE_CHUNK / 2]; // (m, l) of splits c0+2j and c0+2j+1
#pragma unroll
        for (int j = 0; j < DEC_MERGE_CHUNK; j++)
            ov[j] = __builtin_amdgcn_raw_buffer_load_b128(
                rp, ok && c0 + j < ns ? (((c0 + j) * 16 + r) * 64 + d0) * 4 : kOutside, 0, AUX);
#pragma unroll
        for (int j = 0; j < DEC_MERGE_CHUNK / 2; j++)
            ml[j] = __builtin_amdgcn_raw_buffer_load_b128(
                rp, ok && c0 + 2 * j < ns ? (dec_ml_offset(ns) + (r * nsp + c0 + 2 * j) * 2) * 4 : kOutside, 0, AUX);
        if (!ok) continue;
        float Mc = M;
#pragma unroll
        for (int j = 0; j < DEC_MERGE_CHUNK; j++)
            if (c0 + j < ns) Mc = fmaxf(Mc, as_f32(ml[j >> 1][2 * (j & 1)]));
        const float Mu = Mc == -INFINITY ? 0.0f : Mc;
        if (M != -INFINITY && Mc != M) { // a later round raised the maximum: rescale what is summed
            const float s = fast_exp2(M - Mu);
            L *= s;
            acc *= s;
        }
#pragma unroll
        for (int j = 0; j < DEC_MERGE_CHUNK; j++)
            if (c0 + j < ns) {
                const float m = as_f32(ml[j >> 1][2 * (j & 1)]);
                const float w = m == -INFINITY ? 0.0f : fast_exp2(m - Mu);
                L += as_f32(ml[j >> 1][2 * (j & 1) + 1]) * w;
                acc += as_f4(ov[j]) * w;
            }
        M = Mc;
    }
    if (!ok) return;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    *(f4 *)&dst[(((int64_t)bq * U.n_q + iq) * U.H + hq) * HEAD + d0] = acc * inv;
}

// The kernel's leading arguments are the DecPre words (cvattn_common.h), preloaded into scalar
// registers at wave launch (the decode translation units are built with
// -amdgpu-kernarg-preload-count=11); `args` is read from memory as usual.
template <int KT, int VT, bool MASK, bool BATCH>
__global__ __launch_bounds__(64 * DEC_NW) void fa_decode_kernel(const uint8_t *pre_k, const uint8_t *pre_v,
                                                                 const uint8_t *pre_q, int32_t pre_k_ps,
                                                                 int32_t pre_v_ps, int32_t pre_q_ps, uint32_t pre_kv,
                                                                 uint32_t pre_lens, uint32_t pre_shape,
                                                                 uint32_t pre_units, float pre_scale_log2,
                                                                 FaArgs args) {
    constexpr int TS = 32;                     // tokens per wave step
    constexpr int NT = 2;                      // 16-token score tiles per step
    constexpr int PD = dec_prefetch<KT, VT>(); // steps in flight
    __shared__ __attribute__((aligned(16))) _Float16 sK[DEC_NW][32 * DEC_RS];
    __shared__ __attribute__((aligned(16))) _Float16 sV[DEC_NW][32 * DEC_RS];
    __shared__ __attribute__((aligned(16))) float sS[DEC_NW][4][2][32]; // {kd, km, vd, vm} x block x row
    __shared__ uint32_t s_last;

    const FaUniform &U = args.u;
    FaProblem P;
    // the wave index is uniform per wave: readfirstlane lets the token range, step loop and
    // buffer soffsets live in scalar registers
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, g = lane >> 4;

    // ---- the workgroup's unit and the addressing of its loads ----
    // Consecutive units (the kv heads of one token range, whose rows share cache lines) run on
    // one XCD so each line is fetched into one L2 only.
    UnitPos pos;
    gu8 *kbase, *vbase;
    int n_kv, split_len, k_nb1, v_nb1;
    // the epilogue's view of the problem: output, split count, first partial slot and counter
    float *dst = nullptr;
    int ns;
    int64_t part_begin, cnt_begin;
    uint32_t fast_p = 0; // the problem index on the preloaded path
    int iq, hq;
    bool row_ok;
    gu8 *qp;
    const bool fast = !MASK && (pre_shape >> 24) != 0; // uniform
    if (fast) {
        // everything from the preloaded words: no memory access before the loads are issued
        const uint32_t hkv = (pre_shape >> 16) & 0xffu, G = pre_shape >> 24;
        const uint32_t upp = (pre_kv >> 24) * hkv; // units per problem: splits x kv heads
        const uint32_t unit = xcd_unit(blockIdx.x, pre_units);
        const uint32_t p = __builtin_amdgcn_readfirstlane(unit / upp);
        const uint32_t ul = unit - p * upp;
        const uint32_t sp = __builtin_amdgcn_readfirstlane(ul / hkv);
        pos.kh = (int)(ul - sp * hkv);
        pos.split = (int)sp;
        pos.rg = 0;
        pos.bq = 0;
        k_nb1 = (int)(pre_lens >> 16);
        v_nb1 = (int)(pre_shape & 0xffffu);
        const int k_nb2 = __builtin_amdgcn_readfirstlane(k_nb1 / (int)hkv);
        const int v_nb2 = __builtin_amdgcn_readfirstlane(v_nb1 / (int)hkv);
        kbase = gptr(pre_k) + (int64_t)p * pre_k_ps + (int64_t)pos.kh * k_nb2;
        vbase = gptr(pre_v) + (int64_t)p * pre_v_ps + (int64_t)pos.kh * v_nb2;
        n_kv = (int)(pre_kv & 0xffffffu);
        split_len = (int)(pre_lens & 0xffffu);
        // one query token: row `col` of the kv head is q head kh*G + col, contiguous f32 heads
        row_ok = col < (int)G;
        iq = 0;
        hq = pos.kh * (int)G + (row_ok ? col : 0);
        qp = gptr(pre_q) + (int64_t)p * pre_q_ps + (int64_t)hq * (HEAD * 4);
        // the problems of a uniform launch follow each other in the output, the partial slots and
        // the arrival counters (H_kv groups of 16 row slots per problem)
        ns = (int)(pre_kv >> 24);
        fast_p = p; // the output pointer comes from the kernel arguments, in the epilogue
        part_begin = ns > 1 ? (int64_t)p * hkv * 16 * ns : 0;
        cnt_begin = (int64_t)p * hkv;
    } else {
        pos = locate_unit<BATCH>(args, xcd_unit(blockIdx.x, gridDim.x), P);
        resolve_n_kv<BATCH>(P);
        kbase = gptr(P.k) + (int64_t)pos.kh * P.k_nb2 + (int64_t)(pos.bq / P.rk3) * P.k_nb3;
        vbase = gptr(P.v) + (int64_t)pos.kh * P.v_nb2 + (int64_t)(pos.bq / P.rv3) * P.v_nb3;
        n_kv = P.n_kv;
        split_len = P.split_len;
        k_nb1 = (int)P.k_nb1;
        v_nb1 = (int)P.v_nb1;
        row_ok = dec_row(U, pos.kh, pos.rg, col, iq, hq);
        qp = gptr(P.q) + (int64_t)iq * P.q_nb1 + (int64_t)hq * P.q_nb2 + (int64_t)pos.bq * P.q_nb3;
        dst = P.dst;
        ns = P.n_splits;
        part_begin = P.part_begin;
        cnt_begin = P.cnt_begin;
    }
    const int kh = pos.kh, rg = pos.rg, split = pos.split, bq = pos.bq;

    const int t_begin = split * split_len;
    const int t_end = min(n_kv, t_begin + split_len);
    const int wlen = split_len / DEC_NW;
    const int w_begin = t_begin + wv * wlen;
    const int w_end = min(t_end, w_begin + wlen);
    const int nsteps = (max(0, w_end - w_begin) + TS - 1) / TS; // per wave

    // this lane's block in every step: token lt of the step (tile row lrow), 32-dim block lb
    const int lt = lane >> 1;
    const int lb = lane & 1;
    const int lrow = lt;
    // the head rows this workgroup reads: loads of tokens >= n_kv fall outside and read 0
    const int64_t kext = n_kv > 0 ? (int64_t)(n_kv - 1) * k_nb1 + 2 * dblk_bytes<KT>() : 0;
    const int64_t vext = n_kv > 0 ? (int64_t)(n_kv - 1) * v_nb1 + 2 * dblk_bytes<VT>() : 0;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, kext);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase, vext);
    const int kvoff = lt * k_nb1 + lb * dblk_bytes<KT>();
    const int vvoff = lt * v_nb1 + lb * dblk_bytes<VT>();

    // ---- this lane's query row (MFMA column `col`) and its Q operand (hi + lo fp16) ----
    h8 qhi[2], qlo[2];
    float qsum[2];
    bool need_lo = false;
    RawBuf<blk_words<KT>()> RK[PD];
    RawBuf<blk_words<VT>()> RV[PD];
    {
        float x[2][8];
        // The K/V loads go out right behind Q, so the Q conversion below overlaps their latency
        // (memory results return in issue order).  They are issued for every prefetch step: a
        // step this wave does not have reads at an offset past the resource, which returns 0
        // without a memory access, so the load count is fixed and the Q conversion waits for Q
        // alone.
        constexpr int kPast = 0x40000000;
        auto issue_kv = [&]() {
#pragma unroll
            for (int p = 0; p < PD; p++) {
                blk_load<KT>(rk, kvoff, p < nsteps ? (w_begin + p * TS) * k_nb1 : kPast, RK[p]);
                blk_load<VT>(rv, vvoff, p < nsteps ? (w_begin + p * TS) * v_nb1 : kPast, RV[p]);
            }
        };
        auto load_q32 = [&]() {
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int j = 0; j < 8; j++) x[b][j] = as_f32(ldg_u32(qp + 4 * (32 * b + 8 * g + j)));
        };
        if (fast) {
            // nothing read from memory yet: f32 Q, then K/V
            load_q32();
            issue_kv();
        } else {
            if (U.q_f16) {
#pragma unroll
                for (int b = 0; b < 2; b++)
#pragma unroll
                    for (int j = 0; j < 8; j++) x[b][j] = ldg_half(qp + 2 * (32 * b + 8 * g + j));
            } else {
                load_q32();
            }
            issue_kv();
        }
        // keep every load above ahead of the Q conversion (the scheduler would otherwise sink
        // them below it, behind the wait for Q)
        __builtin_amdgcn_sched_barrier(0);

#pragma unroll
        for (int b = 0; b < 2; b++) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float xs = row_ok ? x[b][j] * (fast ? pre_scale_log2 : U.scale_log2) : 0.0f;
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
    // every wave holds the whole Q block, so the wave's own vote is the workgroup's (a workgroup
    // vote would read the launch's group size from memory)
    need_lo = __builtin_amdgcn_ballot_w64(need_lo) != 0;
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

    _Float16 *tK = sK[wv], *tV = sV[wv];
    float(*tS)[2][32] = sS[wv];

    for (int s0 = 0; s0 < nsteps; s0 += PD) {
#pragma unroll
        for (int p = 0; p < PD; p++) {
            const int step = s0 + p;
            if (step < nsteps) { // uniform
                const int t0 = w_begin + step * TS;
                // ---- unpack this step's blocks into the wave's tile, then refill the slot ----
                blk_stage<KT, false>(RK[p], tK + lrow * DEC_RS + 32 * lb);
                blk_stage<VT, true>(RV[p], tV + lrow * DEC_RS + 32 * lb);
                {
                    float d, m;
                    blk_scales<KT>(RK[p], d, m);
                    tS[0][lb][lrow] = d;
                    if constexpr (has_min(KT)) tS[1][lb][lrow] = m;
                    blk_scales<VT>(RV[p], d, m);
                    tS[2][lb][lrow] = d;
                    if constexpr (has_min(VT)) tS[3][lb][lrow] = m;
                }
                if (step + PD < nsteps) {
                    blk_load<KT>(rk, kvoff, (t0 + PD * TS) * k_nb1, RK[p]);
                    blk_load<VT>(rv, vvoff, (t0 + PD * TS) * v_nb1, RV[p]);
                }
                // the tile is wave-private: LDS keeps one wave's accesses in order
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

                // ---- scores: NT tiles of 16 tokens x 16 rows (S^T, lane = row col, tokens 4g+j) ----
                f4 sc[NT];
#pragma unroll
                for (int s = 0; s < NT; s++) {
                    f4 acc[2];
#pragma unroll
                    for (int b = 0; b < 2; b++) {
                        const f4 ci = b ? cinit1 : cinit0;
                        const h8 a0 = *(const h8 *)(tK + (16 * s + col) * DEC_RS + 32 * b + 8 * g);
                        f4 c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qhi[b], ci, 0, 0, 0);
                        if (need_lo) c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qlo[b], c0, 0, 0, 0);
                        acc[b] = c0;
                    }
                    const int sb = 16 * s + 4 * g; // scale rows of these tokens
                    if constexpr (is_quant(KT)) {
                        const f4 d0 = *(const f4 *)&tS[0][0][sb];
                        const f4 d1 = *(const f4 *)&tS[0][1][sb];
                        f4 v = d0 * acc[0] + d1 * acc[1];
                        if constexpr (has_min(KT)) {
                            const f4 m0 = *(const f4 *)&tS[1][0][sb];
                            const f4 m1 = *(const f4 *)&tS[1][1][sb];
                            v += m0 * qsum[0] + m1 * qsum[1];
                        }
                        sc[s] = v;
                    } else {
                        sc[s] = acc[0] + acc[1];
                    }
                }

                // ---- mask, range, softmax with a lazily raised reference maximum ----
                const bool full = t0 + TS <= w_end; // uniform
                float mx = -INFINITY;
#pragma unroll
                for (int s = 0; s < NT; s++) {
                    const int tb = t0 + 16 * s + 4 * g;
                    if constexpr (MASK) {
                        if (full) {
                            const u2 mw = ldg_u64(mrow + (int64_t)tb * 2);
                            const h2 a = as_h2(mw[0]), c2 = as_h2(mw[1]);
                            sc[s][0] += (float)a[0] * 1.4426950408889634f;
                            sc[s][1] += (float)a[1] * 1.4426950408889634f;
                            sc[s][2] += (float)c2[0] * 1.4426950408889634f;
                            sc[s][3] += (float)c2[1] * 1.4426950408889634f;
                        } else {
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                const int t = tb + j;
                                const float mv = ldg_half(mrow + (int64_t)min(t, n_kv - 1) * 2);
                                sc[s][j] = t < w_end ? sc[s][j] + mv * 1.4426950408889634f : -INFINITY;
                            }
                        }
                    } else if (!full) {
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            if (tb + j >= w_end) sc[s][j] = -INFINITY;
                    }
#pragma unroll
                    for (int j = 0; j < 4; j++) mx = fmaxf(mx, sc[s][j]);
                }
                // the cross-lane reduction and the raise only when some lane's maximum clears the
                // threshold (a row's maximum can only clear it through one of its lanes)
                if (__builtin_amdgcn_ballot_w64(mx > m_ref + DEC_RESCALE_LOG2)) { // uniform
                    mx = wave_max16x4(mx);
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
                }
                const float m_use = m_ref == -INFINITY ? 0.0f : m_ref;

                // ---- P^T operands (V block scale folded in) and O^T += V^T P^T ----
#pragma unroll
                for (int s = 0; s < NT; s++) {
                    f4 p;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        p[j] = fast_exp2(sc[s][j] - m_use);
                        l_run += p[j];
                    }
                    const int sb = 16 * s + 4 * g;
                    h4 pb[2];
#pragma unroll
                    for (int b = 0; b < 2; b++) {
                        f4 x = p;
                        if constexpr (is_quant(VT)) x = p * *(const f4 *)&tS[2][b][sb];
                        pb[b] = h4{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
                        if constexpr (has_min(VT)) {
                            const f4 t = p * *(const f4 *)&tS[3][b][sb];
                            corr[b] += t[0] + t[1] + t[2] + t[3];
                        }
                    }
                    // V^T operand rows: tokens 4g..4g+3 of this tile, dims 16i + col
                    const int vrow = 16 * s + 4 * g + (col >> 2);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const short4_t raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (__attribute__((address_space(3))) short4_t *)(tV + vrow * DEC_RS + 16 * i + 4 * (col & 3)));
                        const h4 a = __builtin_bit_cast(h4, raw);
                        oacc[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pb[i >> 1], oacc[i], 0, 0, 0);
                    }
                }
            }
        }
    }

    // ---------------- epilogue: merge the 4 waves (same rows, disjoint tokens) ----------------
    l_run = wave_sum16x4(l_run);
    if constexpr (has_min(VT)) {
        corr[0] = wave_sum16x4(corr[0]);
        corr[1] = wave_sum16x4(corr[1]);
#pragma unroll
        for (int i = 0; i < 4; i++) oacc[i] += corr[i >> 1];
    }
    __syncthreads(); // every wave is done with its tile: reuse them for the merge
    float *xo = (float *)&sK[0][0]; // [4][64 dims][16 rows]
    float *xm = &sS[0][0][0][0];    // [4][16] m, then [4][16] l
    static_assert(sizeof(sK) >= DEC_NW * 64 * 16 * sizeof(float), "merge buffer");
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
    // wave wv now owns dims 16*wv + 4g + j of row slot `col`
    if (fast) dst = args.p0.dst + (int64_t)fast_p * args.dst_ps;
    const int64_t grp = ((int64_t)bq * U.H_kv + kh) * U.n_rowgroups + rg;
    const int64_t slot0 = part_begin + grp * 16 * ns;
    if (ns == 1) {
        if (row_ok) {
            const float inv = L > 0.0f ? 1.0f / L : 0.0f;
            float *out = dst + (((int64_t)bq * U.n_q + iq) * U.H + hq) * HEAD;
            *(f4 *)&out[16 * wv + 4 * g] = o * inv;
        }
        return;
    }
    float *part0 = U.partials + slot0 * PART_STRIDE;
    const int o_off = ((split * 16 + col) * 64 + 16 * wv + 4 * g) * 4;
    const int ml_off = (dec_ml_offset(ns) + (col * dec_nsp(ns) + split) * 2) * 4;
    if constexpr (!BATCH) {
        if (row_ok) {
            *(f4 *)((char *)part0 + o_off) = o;
            if (wv == 0 && g == 0) *(float2 *)((char *)part0 + ml_off) = float2{M, L};
        }
        return;
    } else {
        // Partials are written and read with agent-coherent (sc1) buffer accesses, the form the
        // compiler gives agent-scope atomic loads and stores, but vectorised and all in flight.
        constexpr int SC1 = 16;
        const __amdgpu_buffer_rsrc_t rp = make_rsrc((gu8 *)part0, (int64_t)16 * ns * PART_STRIDE * 4);
        if (row_ok) {
            __builtin_amdgcn_raw_buffer_store_b128(as_u4(o), rp, o_off, 0, SC1);
            if (wv == 0 && g == 0) __builtin_amdgcn_raw_buffer_store_b64(u2{as_u32(M), as_u32(L)}, rp, ml_off, 0, SC1);
        }
        // once the partials have completed, the arrival count publishes them (a device-wide
        // fence would write back the whole L2)
        wait_memory();
        __syncthreads();
        if (tid == 0) {
            uint32_t *cnt = U.counters + (cnt_begin + grp) * CNT_STRIDE;
            const uint32_t prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = prev == (uint32_t)(ns - 1);
            if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last ? 1u : 0u;
        }
        __syncthreads();
        if (!s_last) return;
        dec_merge<true>(U, dst, part0, ns, kh, rg, bq);
    }
}

// Single calls: merge the split partials the decode kernel wrote; one workgroup per group.
static __global__ __launch_bounds__(256) void dec_combine_kernel(FaArgs args) {
    const FaUniform &U = args.u;
    const FaProblem &P = args.p0;
    const int64_t grp = blockIdx.x;
    const int rg = (int)(grp % U.n_rowgroups);
    const int kh = (int)((grp / U.n_rowgroups) % U.H_kv);
    const int bq = (int)(grp / ((int64_t)U.n_rowgroups * U.H_kv));
    dec_merge<false>(U, P.dst, U.partials + (P.part_begin + grp * 16 * P.n_splits) * PART_STRIDE, P.n_splits, kh,
                     rg, bq);
}

} // namespace cvattn
