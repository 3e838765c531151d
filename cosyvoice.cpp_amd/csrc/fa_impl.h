// fa_impl.h -- flash attention for gfx950 (the GGML_OP_FLASH_ATTN_EXT node of
// src/cosyvoice-kv-cache.cpp:383-384 and src/cosyvoice-graph.cpp:375-376): the row-tiled kernel
// for prefill, DiT and every problem with more than 64 query rows per kv head, plus what all
// attention kernels share (problem lookup, workgroup decomposition, split merges).
//
// Rows.  For one (batch b, kv head kh) the rows are the n_q * G query rows sharing kh
// (G = H / H_kv), ordered r = i * G + g (query i, q head kh*G + g).  A wave owns ROWS_SETS sets
// of 16 rows (the 16 columns of its MFMA tiles); each K or V operand read from LDS feeds one MFMA
// per set.  A workgroup is 4 waves (64 rows with one set) sharing 64-token K/V tiles that are
// staged once per step into LDS from registers loaded two steps ahead, so a step has one
// barrier.  With f16 K and V, step s runs the PV product of tile s-1 (its P^T operands kept in
// registers across the barrier), then QK and softmax of tile s, while tile s+1 is unpacked: K
// tiles are double-buffered and V tiles triple-buffered, so no buffer is written in a step that
// reads it.  The other type pairs run QK, softmax and PV of tile s in step s with two V buffers
// (their wider staging leaves no registers for P^T across the barrier).  With two key halves
// (KH = 2, for launches with fewer row groups than CUs) a
// workgroup is 8 waves: a step stages 128 tokens, waves w and w+4 compute the two 64-token
// halves for the same rows, and the halves are merged through LDS at the end.
//
// Per wave and 16-token tile (v_mfma_f32_16x16x32_f16, two 32-dim K halves):
//   S^T[t][r] = K[t][:] . Q[r][:]     A = K rows from the LDS tile, B = Q^T (registers)
// Quantized K is staged as fp16 "1024 + u" codes; the accumulator starts at -(1024 + off)*sum(Q)
// so it ends as sum(code*Q), and the block scale d (and min m) are applied per token afterwards.
// Q*scale is kept exactly in fp16 when it can be (f16 Q with a power-of-two scale: the scores
// are then turned into base 2 with one multiply); otherwise Q*scale*log2(e) is split into fp16
// hi + lo parts and two MFMAs give fp32-accurate scores.
// The C layout of S^T (lane l: row l%16, tokens 4*(l/16)+j) is the B layout of P^T for
//   O^T[dim][r] += V^T[dim][t] . P^T[t][r]
// when the 8 k-slots of lane group g are tokens {4g..4g+3} of one 16-token tile and
// {16+4g..16+4g+3} of the next; the A operand V^T comes from the token-major V tile through two
// ds_read_b64_tr_b16 per MFMA.  V codes are staged exactly (fp16 small integers); the V block
// scale is folded into P (one B operand per 32-dim block) and the V min into a per-row term.
// Softmax is base 2 with a lazily raised reference maximum (rescale only when a row maximum grows
// by more than 2^8).
#pragma once

#include "cvattn_device.h"
#include "cvattn_launch.h"
#include "kv_blocks.h"

#include <type_traits>

namespace cvattn {

constexpr int ROWS_NW = 4;          // waves per workgroup
// the wide form: 12 waves (192 rows) per workgroup, one workgroup per CU at 3 waves per SIMD, so
// each staged K/V tile serves 192 rows (unmasked fp16 launches with a row group for every CU)
constexpr int ROWS_NW_WIDE = 12;
constexpr int ROWS_SETS = 1;        // 16-row sets per wave (a set shares every K and V operand read);
                                    // one set: 64-row workgroups, 3 resident per CU (138 VGPRs), measured
                                    // faster than two sets (128-row workgroups, 2 per CU) for prefill and DiT
constexpr int ROWS_TS = 64;         // tokens per staged tile
static_assert(ROWS_TS == ROWS_TILE, "mask tile classes are per staged tile");
// halfs per LDS row of the token-major K and V tiles (64 dims + pad), and of the dim-major
// transposed-V tile.  The pad sets which LDS banks the operand reads of a wave hit together;
// measured on the DiT call (K / V row halfs): 72/72 43.8-44.7 us, 80/80 42.8-43.0, 80/88
// 42.6-43.3, 88/80 44.1, 96/96 50.8, 64/80 52.6.
constexpr int ROWS_RS = 80;
constexpr int ROWS_RS_VT = 72;
constexpr int ROWS_ROWS = 16 * ROWS_SETS * ROWS_NW;
constexpr float ROWS_RESCALE_LOG2 = 8.0f;
// the two K tile buffers double as the split-merge scratch (2 * ROWS * n_splits floats)
constexpr int ROWS_MERGE_MAX_SPLITS = (2 * ROWS_TS * ROWS_RS * 2 / 4) / (2 * ROWS_ROWS);

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

// Position of a workgroup unit inside its problem: unit = ((bq*n_splits + split)*H_kv + kh)*
// n_rowgroups + rg, counted from the problem's unit_begin.  Row groups are innermost, then kv
// heads, so that the units of one XCD (see xcd_unit) share the K/V rows of few heads in that
// XCD's L2.
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
    t = fdiv(ul, U.div_hkv);
    r.kh = (int)(ul - t * (uint32_t)U.H_kv);
    ul = t;
    t = fdiv(ul, P.div_splits);
    r.split = (int)(ul - t * (uint32_t)P.n_splits);
    r.bq = (int)t;
    return r;
}

// A prepared plan with a device-resident n_kv: the launch reads the current length (clamped to
// the capacity P.n_kv the plan was made for) and spreads it over the planned splits, each a
// multiple of split_unit tokens; splits past the end run empty and merge with weight 0.  The
// value is written before the launch (a kernel earlier on the stream, or a copy), so a plain
// load sees it.
template <bool BATCH>
__device__ __forceinline__ void resolve_n_kv(FaProblem &P) {
    if constexpr (BATCH) {
        if (P.n_kv_dev != nullptr) {
            // integer division runs on the VALU: the results go back to scalar registers, or every
            // bound derived from them (token range, step count, buffer extents) would occupy VGPRs
            const int n = min(max(*P.n_kv_dev, 0), P.n_kv);
            const int per = (n + P.n_splits - 1) / P.n_splits;
            const int u = P.split_unit;
            P.split_len = __builtin_amdgcn_readfirstlane(max(u, (per + u - 1) / u * u));
            P.n_kv = __builtin_amdgcn_readfirstlane(n);
        }
    }
}

// Last-arriving workgroup of a split row group merges all split partials of its rows
// (prepared batches: no separate combine launch).  The partials were written by other
// workgroups of the same launch and are read with agent-coherent (sc1) vector loads: (1) every
// split's (m, l) of every row into LDS, (2) one thread per row turns them into normalised split
// weights, (3) each thread sums 4-dim chunks of its rows over the splits, with the loads of 4
// splits x all its chunks in flight at once.
// `scratch` holds 2 * ROWS * n_splits floats (n_splits <= ROWS_MERGE_MAX_SPLITS).
template <int ROWS, int THREADS>
__device__ __forceinline__ void merge_splits(const FaUniform &U, const FaProblem &P, int bq, int kh, int rg,
                                             int64_t slot0, int tid, float *scratch) {
    constexpr int SC1 = 16;
    const int ns = P.n_splits;
    float *sm = scratch;             // [ROWS][ns] m, then normalised weights
    float *sl = scratch + ROWS * ns; // [ROWS][ns] l
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc((gu8 *)(U.partials + slot0 * PART_STRIDE), (int64_t)ROWS * ns * PART_STRIDE * 4);
    for (int idx = tid; idx < ROWS * ns; idx += THREADS) { // slot0 + r*ns + s == slot0 + idx
        const u2 ml = __builtin_amdgcn_raw_buffer_load_b64(rp, (idx * PART_STRIDE + 64) * 4, 0, SC1);
        sm[idx] = as_f32(ml[0]);
        sl[idx] = as_f32(ml[1]);
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
    constexpr int PER = ROWS * (HEAD / 4) / THREADS; // 4-dim chunks per thread
    static_assert(PER * THREADS == ROWS * (HEAD / 4), "merge tiling");
    f4 acc[PER];
#pragma unroll
    for (int e = 0; e < PER; e++) acc[e] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < ns; s0 += 4) {
        u4 ov[PER][4];
#pragma unroll
        for (int e = 0; e < PER; e++) {
            const int c = tid + e * THREADS, r = c >> 4, d0 = (c & 15) * 4;
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (s0 + j < ns)
                    ov[e][j] = __builtin_amdgcn_raw_buffer_load_b128(rp, ((r * ns + s0 + j) * PART_STRIDE + d0) * 4, 0, SC1);
        }
#pragma unroll
        for (int e = 0; e < PER; e++) {
            const int r = (tid + e * THREADS) >> 4;
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (s0 + j < ns) acc[e] += as_f4(ov[e][j]) * sm[r * ns + s0 + j];
        }
    }
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int c = tid + e * THREADS, r = c >> 4, d0 = (c & 15) * 4;
        const int row = rg * ROWS + r;
        if (row >= U.n_rows) continue;
        const int iq = row / U.G, hq = kh * U.G + row % U.G;
        *(f4 *)&P.dst[(((int64_t)bq * U.n_q + iq) * U.H + hq) * HEAD + d0] = acc[e];
    }
}

// KH = 2: two key halves.  The workgroup is 8 waves; waves w and w+4 own the same 16 rows and
// take the first and second 64 tokens of each 128-token staged step, then merge through LDS.  For
// launches with fewer row groups than CUs (prefill), where one wave per SIMD walks the whole key
// range, this halves the chain each wave runs.
template <int KT, int VT, int MASK, bool BATCH, int KH, int NW>
__global__ __launch_bounds__(64 * NW * KH)
// f16 K/V without mask: 3 waves per SIMD (168 VGPRs).  The masked instance does not fit 168 (it
// spilled 104-108 bytes per lane there) and runs faster unconstrained (DiT T=1500 with a 50-frame
// chunk mask: 73.3 -> 71.0 us).
// MASK: 0 none, 1 mask words read for every tile, 2 classified tiles (MCLS_*: the workgroup
// stages only tiles that are not all -inf for its row group, and reads mask words only for mixed
// ones; all-zero tiles run as unmasked).
__attribute__((amdgpu_waves_per_eu(KH == 1 && KT == T_F16 && VT == T_F16 && MASK != 1 ? 3 : 1)))
void fa_rows_kernel(FaArgs args) {
    constexpr int TS = ROWS_TS, NTILE = TS / 16, NKB = TS / 32, NR = ROWS_SETS;
    constexpr int TSS = TS * KH; // tokens per staged step
    constexpr int ROWS = 16 * NR * NW; // rows per workgroup (row group)
    static_assert(NW == ROWS_NW || (NW == ROWS_NW_WIDE && KH == 1 && MASK == 0 && !is_vt(VT)),
                  "the wide form is one key half without mask");
    constexpr int RSK = ROWS_RS, RSV = is_vt(VT) ? ROWS_RS_VT : ROWS_RS;
    static_assert(KH == 1 || (KH == 2 && !is_vt(VT)), "the transposed-V tile holds one 64-token step");
    constexpr int W = blk_words<KT>() > blk_words<VT>() ? blk_words<KT>() : blk_words<VT>();
    // SHIFT (f16 K and V): the PV product of tile s runs after the barrier that ends step s,
    // beside the QK product of tile s+1, while step s+1 stages tile s+2, so the V tiles are
    // triple-buffered.  The other type pairs run PV in the tile's own step (their P^T operands
    // held across the barrier cost more registers than the overlap gains) with two V buffers.
    constexpr bool SHIFT = KT == T_F16 && VT == T_F16;
    constexpr int NVB = SHIFT ? 3 : 2;
    __shared__ __attribute__((aligned(16))) _Float16 sK[2][TSS * RSK];
    __shared__ __attribute__((aligned(16))) _Float16 sV[NVB][TSS * RSV];
    // block scales {d, m} x block x token of quantized K (per K buffer) and V (per V buffer)
    __shared__ __attribute__((aligned(16))) float sSK[is_quant(KT) ? 2 : 1][2][2][is_quant(KT) ? TSS : 1];
    __shared__ __attribute__((aligned(16))) float sSV[is_quant(VT) ? NVB : 1][2][2][is_quant(VT) ? TSS : 1];

    const FaUniform &U = args.u;
    FaProblem P;
    const UnitPos pos = locate_unit<BATCH>(args, xcd_unit(blockIdx.x, gridDim.x), P);
    const int kh = pos.kh, rg = pos.rg, split = pos.split, bq = pos.bq;
    resolve_n_kv<BATCH>(P);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15; // MFMA column (query row) / A-operand row (token or dim)
    const int g = lane >> 4;   // lane group: k-slots 8g..8g+7, C rows 4g..4g+3
    const int rw = wv % NW;               // row wave: rows rw*16*NR.. of the row group
    const int hk = KH == 2 ? wv / NW : 0; // key half (uniform per wave)

    const int t_begin = split * P.split_len;
    const int t_end = min(P.n_kv, t_begin + P.split_len);
    const int nsteps_all = (max(0, t_end - t_begin) + TSS - 1) / TSS; // steps of the token range

    // Mask classes (MASK 2): this row group's key tiles (at most 64) become two scalar bit masks,
    // and the workgroup walks only the steps from its first to its last tile that is not all
    // -inf (the visible region of a causal, chunk or window mask is one such run; an all -inf
    // tile inside it is skipped by the waves).
    const bool use_cls = MASK == 2 && P.mcls != nullptr; // uniform
    uint64_t cls_zero = 0, cls_off = 0, cls_pre = 0;     // bit k: tile kt0+k all 0 / all -inf / prefix
    int t_first = t_begin;                               // first token of staged step 0, uniform
    int nsteps = nsteps_all, nfull = max(0, t_end - t_begin) / TSS; // staged steps / full ones, uniform
    const int kt0 = t_begin / TSS;                       // class column of the range's first tile
    if constexpr (MASK == 2) {
        static_assert(KH == 1, "mask classes are per 64-token step");
        if (use_cls) {
            const int c = lane < nsteps_all ? P.mcls[(int64_t)rg * P.mcls_ld + kt0 + lane] : MCLS_MIXED;
            cls_zero = __builtin_amdgcn_ballot_w64(c == MCLS_ZERO);
            cls_off = __builtin_amdgcn_ballot_w64(c == MCLS_OFF);
            cls_pre = __builtin_amdgcn_ballot_w64(c == MCLS_PREFIX);
            const uint64_t live = ~cls_off & (nsteps_all >= 64 ? ~0ull : ((1ull << nsteps_all) - 1));
            if (live == 0) {
                nsteps = nfull = 0;
            } else {
                const int first = (int)__builtin_ctzll(live), last = 63 - (int)__builtin_clzll(live);
                // the range's partial tile can only be the last step of the token range
                const bool part = nfull < nsteps_all && last == nsteps_all - 1;
                t_first = t_begin + first * TSS;
                nsteps = last - first + 1;
                nfull = nsteps - (part ? 1 : 0);
            }
        }
    }
    // the step counts are uniform: keep the loop control in scalar registers
    nsteps = __builtin_amdgcn_readfirstlane(nsteps);
    nfull = __builtin_amdgcn_readfirstlane(nfull);
    t_first = __builtin_amdgcn_readfirstlane(t_first);
    // first token of staged step i
    auto tok = [&](int i) -> int { return t_first + i * TSS; };

    // ---- staging role: waves 0..2KH-1 stage K blocks, the others V blocks; thread = (token, block) ----
    // Transposed V (non-flash-attention layout): thread = (dim, 16-byte run of tokens), VNCH runs
    // VDSTEP dims apart; the tile is kept dim-major in LDS, which is already the V^T operand.
    constexpr bool VTR = is_vt(VT);
    constexpr int VES = VT == T_VT_F32 ? 4 : 2;  // bytes per transposed-V element
    constexpr int VCH = 16 / VES;                 // tokens per 16-byte run
    constexpr int VCPD = TSS / VCH;               // runs per dim of a tile
    constexpr int VDSTEP = 128 * KH / VCPD;       // dims between one thread's runs
    constexpr int VNCH = HEAD / VDSTEP;           // runs per staging thread
    const bool stage_k = wv < 2 * KH; // uniform per wave
    // waves 0..4KH-1 stage the tiles; in the wide form the others only compute (their loads
    // get an empty range: no memory traffic, and the wait counts stay those of the stagers)
    const bool stager = NW == ROWS_NW || wv < 4 * KH;
    const int st_idx = tid & (128 * KH - 1);
    const int st_tok = st_idx >> 1, st_b = tid & 1;
    const int vt_tc = st_idx % VCPD, vt_d0 = st_idx / VCPD;
    gu8 *kbase = gptr(P.k) + (int64_t)kh * P.k_nb2 + (int64_t)(bq / P.rk3) * P.k_nb3;
    gu8 *vbase = gptr(P.v) + (int64_t)kh * P.v_nb2 + (int64_t)(bq / P.rv3) * P.v_nb3;
    // The tile loads are issued unconditionally, two steps ahead, also past the last step (so
    // the compiler can count them exactly and each wait covers only the tile it needs): the K and
    // V ranges end at the walk's last token, so loads past it read zeros without touching memory.
    const int t_lim = min(t_end, tok(nsteps));
    const int64_t kext = t_lim > 0 ? (int64_t)(t_lim - 1) * P.k_nb1 + 2 * dblk_bytes<KT>() : 0;
    // transposed f16: +2 bytes so the dword holding the last element is inside the range
    // (buffer loads check whole dwords; the extra element is zeroed with the tile's tail).  A
    // dim's tokens past n_kv are the next dim's; loads past the walk read them and go unused.
    const int64_t vext = P.n_kv <= 0 ? 0
                         : VTR    ? (int64_t)(HEAD - 1) * P.v_nb1 + (int64_t)P.n_kv * VES + (VES == 2 ? 2 : 0)
                         : t_lim > 0 ? (int64_t)(t_lim - 1) * P.v_nb1 + 2 * dblk_bytes<VT>()
                                     : 0;
    const __amdgpu_buffer_rsrc_t rsrc = stage_k ? make_rsrc(kbase, kext) : make_rsrc(vbase, stager ? vext : 0);
    const int nb1 = stage_k ? (int)P.k_nb1 : VTR ? VES : (int)P.v_nb1; // bytes per token
    const int voff = stage_k ? st_tok * nb1 + st_b * dblk_bytes<KT>()
                     : VTR   ? vt_d0 * (int)P.v_nb1 + 16 * vt_tc
                             : st_tok * nb1 + st_b * dblk_bytes<VT>();

    // Register buffers of staged tiles: tile t is loaded into R[t % NRB] NRB steps before the step
    // that unpacks it into LDS (one step before the step that computes it).  The two-half f16
    // form (prefill: one workgroup per CU, two waves per SIMD, so little else hides a load's
    // latency) keeps three, 16 words each; the others keep two (a third cost the one-half
    // forms 15-32 VGPRs: spills at the f16 cap, and 3 -> 2 waves per SIMD for q8_0).
    constexpr int NRB = KT == T_F16 && VT == T_F16 && KH == 2 ? 3 : 2;
    RawBuf<W> R[NRB];
    auto load_tile = [&](int t0, RawBuf<W> &r) {
        if (stage_k) {
            blk_load<KT>(rsrc, voff, t0 * nb1, r);
        } else if constexpr (VTR) {
            if (P.v_align2) { // uniform: fp16 runs at 2-byte alignment, loaded element by element
#pragma unroll
                for (int i = 0; i < VNCH; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int o = voff + i * VDSTEP * (int)P.v_nb1 + 4 * j;
                        r.w[4 * i + j] = bld_u16(rsrc, o, t0 * VES) | (bld_u16(rsrc, o + 2, t0 * VES) << 16);
                    }
            } else {
#pragma unroll
                for (int i = 0; i < VNCH; i++) {
                    const u4 a = bld_u128(rsrc, voff + i * VDSTEP * (int)P.v_nb1, t0 * VES);
                    r.w[4 * i + 0] = a[0];
                    r.w[4 * i + 1] = a[1];
                    r.w[4 * i + 2] = a[2];
                    r.w[4 * i + 3] = a[3];
                }
            }
        } else {
            blk_load<VT>(rsrc, voff, t0 * nb1, r);
        }
    };
    // One-half workgroups (several per CU) issue their first tiles before Q; the two-half form
    // (prefill: one workgroup per CU) issues them after Q and the first mask words, below, so that
    // its wait for Q does not also cover them (the wait counter completes loads in issue order):
    // the 256-row prefill chunks 0.3-0.4 us faster each, the fp32-view DiT call ~0.8 us slower
    // in the other order
    if constexpr (KH == 1) {
#pragma unroll
        for (int j = 0; j < NRB; j++) load_tile(tok(j), R[j]);
    }

    // ---- this lane's query rows (one per 16-row set) and their Q operands ----
    int row[NR], iq[NR], hq[NR];
    bool row_ok[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        row[r] = rg * ROWS + rw * (16 * NR) + 16 * r + col;
        row_ok[r] = row[r] < U.n_rows;
        iq[r] = row_ok[r] ? row[r] / U.G : 0;
        hq[r] = kh * U.G + (row_ok[r] ? row[r] % U.G : 0);
    }
    gu8 *mrow[NR];
#pragma unroll
    for (int r = 0; r < NR; r++)
        mrow[r] = MASK ? gptr(P.mask) + (int64_t)iq[r] * P.m_nb1 + (int64_t)(hq[r] % P.m_ne2) * P.m_nb2 +
                             (int64_t)(bq % P.m_ne3) * P.m_nb3
                       : nullptr;
    // MASK 1: mask words of this wave's next full tile, loaded one step ahead; below, the first
    // one's (a wave whose first tile is partial never reads them)
    u2 mpre[NR][NTILE];
    h8 qhi[NR][2], qlo[NR][2];
    float qsum[NR][2];
    constexpr int BND_HELD = 4; // MASK 2: prefix tiles whose per-row lengths stay in registers
    uint32_t bnd_pk[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) bnd_pk[r] = 0;
    float smul; // multiplies the staged K scales / raw scores into base-2 logits
    bool need_lo;
    {
        float x[NR][2][8];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            gu8 *qp = gptr(P.q) + (int64_t)iq[r] * P.q_nb1 + (int64_t)hq[r] * P.q_nb2 + (int64_t)bq * P.q_nb3;
            if (U.q_f16) { // uniform
#pragma unroll
                for (int b = 0; b < 2; b++)
#pragma unroll
                    for (int j = 0; j < 8; j++) x[r][b][j] = ldg_half(qp + 2 * (32 * b + 8 * g + j));
            } else {
#pragma unroll
                for (int b = 0; b < 2; b++)
#pragma unroll
                    for (int j = 0; j < 8; j++) x[r][b][j] = as_f32(ldg_u32(qp + 4 * (32 * b + 8 * g + j)));
            }
        }
        // MASK 2: the prefix lengths of the range's first BND_HELD prefix tiles, a byte each, read
        // beside Q (the loop then reads no memory for them)
        if constexpr (MASK == 2) {
            uint64_t pre = cls_pre; // uniform
            const int q0 = rg * ROWS / U.G;
#pragma unroll
            for (int i = 0; i < BND_HELD; i++) {
                if (pre == 0) break; // uniform
                const int k = (int)__builtin_ctzll(pre);
                pre &= pre - 1;
                gu8 *b = gptr(mcls_bounds(P, U.mcls_blocks, (int64_t)rg * P.mcls_ld + kt0 + k));
#pragma unroll
                for (int r = 0; r < NR; r++)
                    if (row_ok[r]) bnd_pk[r] |= (uint32_t)b[iq[r] - q0] << (8 * i);
            }
        }
        if constexpr (MASK == 1) {
            const int t0 = tok(0) + hk * TS;
            if (t0 + TS <= t_end) { // uniform
#pragma unroll
                for (int r = 0; r < NR; r++)
#pragma unroll
                    for (int tt = 0; tt < NTILE; tt++) mpre[r][tt] = ldg_u64(mrow[r] + (int64_t)(t0 + 16 * tt + 4 * g) * 2);
            }
        }
        if constexpr (KH == 2) {
#pragma unroll
            for (int j = 0; j < NRB; j++) load_tile(tok(j), R[j]);
        }
        // Q*scale exact in fp16 (up to fp16 subnormal rounding, below 2^-24) for every row?
        bool inexact = false;
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float xs = row_ok[r] ? x[r][b][j] * U.scale : 0.0f;
                    inexact |= fabsf((float)(_Float16)xs - xs) > 0x1p-25f;
                }
        if constexpr (MASK == 2) {
            // wait for the lengths here, with Q, not at their first use inside the loop (where the
            // wait would also cover the tile loads issued since)
#pragma unroll
            for (int r = 0; r < NR; r++) asm volatile("" ::"v"(bnd_pk[r]));
        }
        need_lo = __syncthreads_or(inexact) != 0;
        const float qmul = need_lo ? U.scale_log2 : U.scale;
        smul = need_lo ? 1.0f : 1.4426950408889634f;
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
            for (int b = 0; b < 2; b++) {
                float sm = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float xs = row_ok[r] ? x[r][b][j] * qmul : 0.0f;
                    const _Float16 hx = (_Float16)xs;
                    const _Float16 lx = (_Float16)(xs - (float)hx);
                    qhi[r][b][j] = hx;
                    qlo[r][b][j] = lx;
                    sm += (float)hx + (need_lo ? (float)lx : 0.0f);
                }
                qsum[r][b] = wave_sum16x4(sm);
            }
    }
    constexpr float kbias = stage_bias<KT>();

    // unpack a staged tile's blocks (tokens t0..t0+TS) into LDS buffer `buf`
    // (step: the step of the tile: K buffer step&1, V buffer step%NVB)
    auto write_tile = [&](const RawBuf<W> &r, int step, int t0) {
        if (!stager) return; // uniform
        float d, m;
        const int buf = step & 1, vbuf = step % NVB;
        if (stage_k) {
            blk_stage<KT, false>(r, sK[buf] + st_tok * RSK + 32 * st_b);
            blk_scales<KT>(r, d, m);
            if constexpr (is_quant(KT)) {
                sSK[buf][0][st_b][st_tok] = d * smul;
                if constexpr (has_min(KT)) sSK[buf][1][st_b][st_tok] = m * smul;
            }
        } else if constexpr (VTR) {
            // dim-major rows of fp16; tokens from n_kv on are zeroed (the cache row continues
            // past them with whatever the cache holds, and they meet zero weights)
            const int nvalid = P.n_kv - t0 - VCH * vt_tc; // valid tokens of each run
#pragma unroll
            for (int i = 0; i < VNCH; i++) {
                _Float16 *dst = sV[vbuf] + (vt_d0 + VDSTEP * i) * RSV + VCH * vt_tc;
                if constexpr (VT == T_VT_F16) {
                    u4 w = {r.w[4 * i], r.w[4 * i + 1], r.w[4 * i + 2], r.w[4 * i + 3]};
                    if (t0 + TSS > P.n_kv) { // uniform: the cache's last tile
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            w[j] &= (2 * j < nvalid ? 0xffffu : 0u) | (2 * j + 1 < nvalid ? 0xffff0000u : 0u);
                    }
                    *(u4 *)dst = w;
                } else {
                    h4 h;
#pragma unroll
                    for (int j = 0; j < 4; j++) h[j] = j < nvalid ? (_Float16)as_f32(r.w[4 * i + j]) : (_Float16)0.0f;
                    *(h4 *)dst = h;
                }
            }
        } else {
            blk_stage<VT, true>(r, sV[vbuf] + st_tok * RSV + 32 * st_b);
            blk_scales<VT>(r, d, m);
            if constexpr (is_quant(VT)) {
                sSV[vbuf][0][st_b][st_tok] = d;
                if constexpr (has_min(VT)) sSV[vbuf][1][st_b][st_tok] = m;
            }
        }
    };

    float m_ref[NR], l_run[NR], corr[NR][2];
    f4 oacc[NR][4];
    // unquantized V: the row sums come out of the PV MFMAs as a 65th output dim, from an A operand
    // whose row 0 is ones (lane (col, g) holds A[col][8g..8g+7]): C[0][row] = sum_t P[t][row]
    f4 lacc[NR];
    h8 ones_a;
#pragma unroll
    for (int j = 0; j < 8; j++) ones_a[j] = col == 0 ? (_Float16)1.0f : (_Float16)0.0f;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        m_ref[r] = -INFINITY; // reference maximum (base 2) of this lane's row
        l_run[r] = 0.0f;
        corr[r][0] = corr[r][1] = 0.0f;
        lacc[r] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 4; i++) oacc[r][i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    // P^T operands of the last tile, kept until its PV product (after the step's barrier)
    h8 pb[NR][NKB][2];

    // QK and softmax of one staged tile for both row sets (K buffer kb, V scales of V buffer vb,
    // tokens t0..t0+TS), leaving its P^T operands in pb; `full_c` (std::true_type) says every
    // token of the tile is in range, so no bounds code is emitted (t0: this wave's 64 tokens, key
    // half hk of the staged step).  False when the mask removes the whole tile for this wave.
    auto qk_soft = [&](int kb, int vb, int t0, int tn, auto full_c) -> bool {
        const _Float16 *cK = sK[kb] + hk * TS * RSK;
        auto cS = [&](int x, int b) { return x < 2 ? &sSK[kb][x][b][hk * TS] : &sSV[vb][x - 2][b][hk * TS]; };
        constexpr bool full = decltype(full_c)::value;
        // a skipped tile leaves no P^T operands: pb is cleared so that the operands of the
        // previous tile (already consumed) need not stay live beside the ones being computed
        auto skip = [&]() -> bool {
#pragma unroll
            for (int r = 0; r < NR; r++)
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) pb[r][kb][0] = pb[r][kb][1] = h8{};
            return false;
        };
        // masks: a tile whose mask is -inf for every row of the wave (the masked-out triangle of a
        // causal prefill) contributes nothing; the wave skips it
        u2 mwv[NR][NTILE];
        bool mixed = MASK != 0;  // the tile adds mask words (uniform)
        bool prefix = false;     // MASK 2: the tile keeps the first bnd[r] keys of each row (uniform)
        int bnd[NR];
        int k = 0; // MASK 2: the tile's class bit (uniform)
        if constexpr (MASK == 2) {
            // an all-zero tile runs as unmasked, a prefix-shaped one masks each row past its
            // prefix length, an all -inf one inside the walked range (a hole; the range itself
            // starts and ends at visible tiles) runs as a prefix tile of length 0, and a mixed one
            // reads its mask words after the QK products (so they do not add to the K operands'
            // live registers).  Skipping holes instead would keep a second set of P^T operands
            // live across the loop.
            k = (t0 - t_begin) / TS;
            prefix = use_cls && (((cls_pre | cls_off) >> k) & 1);
            mixed = !((cls_zero >> k) & 1) && !prefix;
        } else if constexpr (MASK == 1) {
            if constexpr (full) {
                bool live = false;
                // this tile's words were loaded one step ahead (the wave's first full tile's
                // before the pipeline); the words of its tile of the next staged step are loaded
                // now.  Past the last full tile the current one is read again: the loads are then
                // unconditional, and the waits for them and for the staged tiles count exactly.
#pragma unroll
                for (int r = 0; r < NR; r++)
#pragma unroll
                    for (int tt = 0; tt < NTILE; tt++) mwv[r][tt] = mpre[r][tt];
                const int tp = tn >= 0 && tn + TS <= t_end ? tn : t0;
#pragma unroll
                for (int r = 0; r < NR; r++)
#pragma unroll
                    for (int tt = 0; tt < NTILE; tt++) mpre[r][tt] = ldg_u64(mrow[r] + (int64_t)(tp + 16 * tt + 4 * g) * 2);
#pragma unroll
                for (int r = 0; r < NR; r++)
#pragma unroll
                    for (int tt = 0; tt < NTILE; tt++) {
                        // fp16 -inf is 0xfc00; any other half of the four keeps the tile
                        live |= row_ok[r] && ((mwv[r][tt][0] & 0xffffu) != 0xfc00u || (mwv[r][tt][0] >> 16) != 0xfc00u ||
                                              (mwv[r][tt][1] & 0xffffu) != 0xfc00u || (mwv[r][tt][1] >> 16) != 0xfc00u);
                    }
                if (__builtin_amdgcn_ballot_w64(live) == 0) return skip(); // uniform
            }
        }
        f4 s[NR][NTILE];
        // every K operand of the tile is read before the first MFMA (one LDS wait, not four)
        h8 ka[NTILE][2];
#pragma unroll
        for (int tt = 0; tt < NTILE; tt++) {
            ka[tt][0] = *(const h8 *)&cK[(16 * tt + col) * RSK + 8 * g];
            ka[tt][1] = *(const h8 *)&cK[(16 * tt + col) * RSK + 32 + 8 * g];
        }
        // the lo MFMAs are a uniform choice per launch; each choice is one straight-line block
        auto qk = [&](auto lo_c) {
            constexpr bool LO = decltype(lo_c)::value;
#pragma unroll
            for (int tt = 0; tt < NTILE; tt++) {
                const h8 a0 = ka[tt][0];
                const h8 a1 = ka[tt][1];
#pragma unroll
                for (int r = 0; r < NR; r++) {
                    const f4 ci0 = {-kbias * qsum[r][0], -kbias * qsum[r][0], -kbias * qsum[r][0], -kbias * qsum[r][0]};
                    if constexpr (!is_quant(KT)) {
                        // no block scales: one accumulator chain over both halves (its init is 0)
                        f4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qhi[r][0], f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qhi[r][1], acc, 0, 0, 0);
                        if constexpr (LO) {
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qlo[r][0], acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qlo[r][1], acc, 0, 0, 0);
                        }
                        s[r][tt] = acc;
                    } else {
                        const f4 ci1 = {-kbias * qsum[r][1], -kbias * qsum[r][1], -kbias * qsum[r][1], -kbias * qsum[r][1]};
                        f4 acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qhi[r][0], ci0, 0, 0, 0);
                        f4 acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qhi[r][1], ci1, 0, 0, 0);
                        if constexpr (LO) {
                            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qlo[r][0], acc0, 0, 0, 0);
                            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qlo[r][1], acc1, 0, 0, 0);
                        }
                        const f4 d0 = *(const f4 *)&cS(0, 0)[16 * tt + 4 * g];
                        const f4 d1 = *(const f4 *)&cS(0, 1)[16 * tt + 4 * g];
                        f4 v = d0 * acc0 + d1 * acc1;
                        if constexpr (has_min(KT)) {
                            const f4 m0 = *(const f4 *)&cS(1, 0)[16 * tt + 4 * g];
                            const f4 m1 = *(const f4 *)&cS(1, 1)[16 * tt + 4 * g];
                            v += m0 * qsum[r][0] + m1 * qsum[r][1];
                        }
                        s[r][tt] = v;
                    }
                }
            }
        };
        if (need_lo) qk(std::true_type{});
        else qk(std::false_type{});
        if constexpr (MASK == 2) {
            if (prefix) { // uniform
                // the range's first BND_HELD prefix tiles have their lengths in registers; later
                // ones (and only they) read them here
                const int idx = __builtin_popcountll(cls_pre & ((1ull << k) - 1)); // uniform
                if ((cls_off >> k) & 1) {
#pragma unroll
                    for (int r = 0; r < NR; r++) bnd[r] = 0;
                } else if (idx < BND_HELD) {
#pragma unroll
                    for (int r = 0; r < NR; r++) bnd[r] = (bnd_pk[r] >> (8 * idx)) & 0xff;
                } else {
                    __builtin_amdgcn_sched_barrier(0);
                    const int q0 = rg * ROWS / U.G;
                    gu8 *b = gptr(mcls_bounds(P, U.mcls_blocks, (int64_t)rg * P.mcls_ld + kt0 + k));
#pragma unroll
                    for (int r = 0; r < NR; r++) {
                        bnd[r] = row_ok[r] ? b[iq[r] - q0] : 0;
                        // complete the load inside this branch: a load still pending where the
                        // branches meet would make the other paths wait for every load in flight
                        asm volatile("" ::"v"(bnd[r]));
                    }
                }
            }
            if constexpr (full) {
                if (mixed) { // uniform
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int r = 0; r < NR; r++)
#pragma unroll
                        for (int tt = 0; tt < NTILE; tt++) mwv[r][tt] = ldg_u64(mrow[r] + (int64_t)(t0 + 16 * tt + 4 * g) * 2);
                    // complete the loads inside this branch (as for the prefix lengths above)
#pragma unroll
                    for (int r = 0; r < NR; r++)
#pragma unroll
                        for (int tt = 0; tt < NTILE; tt++) asm volatile("" ::"v"(mwv[r][tt]));
                }
            }
        }
        // scores so far are base-2 logits divided by sm2 (quantized K has smul folded into its
        // scales); the mask path turns them into base-2 logits here, the others in the exponent
        float sm2 = is_quant(KT) || MASK == 1 ? 1.0f : smul;
        const float mmul = is_quant(KT) ? 1.0f : smul;
        // MASK 2 keeps the scores in the unmasked scale and adds mask * log2(e) / sm2
        const float madd = 1.4426950408889634f / mmul;
#pragma unroll
        for (int r = 0; r < NR; r++) {
            // ---- mask, bounds, softmax with a lazily raised reference maximum ----
            float mx = -INFINITY;
            // prefix tiles: key 16tt + 4g + j of the tile is visible below the row's prefix length
            // (and the range's end, in a partial tile); the lane's offset 4g moves to the bound so
            // the comparisons are against constants
            int plim = 0;
            if constexpr (MASK == 2) {
                if (prefix) plim = (full ? bnd[r] : min(bnd[r], t_end - t0)) - 4 * g;
            }
#pragma unroll
            for (int tt = 0; tt < NTILE; tt++) {
                const int tb = t0 + 16 * tt + 4 * g;
                if constexpr (MASK == 2) {
                    if (prefix) { // uniform
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            if (16 * tt + j >= plim) s[r][tt][j] = -INFINITY;
                    } else if constexpr (full) {
                        if (mixed) { // uniform
                            const h2 a = as_h2(mwv[r][tt][0]), c2 = as_h2(mwv[r][tt][1]);
                            s[r][tt][0] = __builtin_fmaf((float)a[0], madd, s[r][tt][0]);
                            s[r][tt][1] = __builtin_fmaf((float)a[1], madd, s[r][tt][1]);
                            s[r][tt][2] = __builtin_fmaf((float)c2[0], madd, s[r][tt][2]);
                            s[r][tt][3] = __builtin_fmaf((float)c2[1], madd, s[r][tt][3]);
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int t = tb + j;
                            const float mv = ldg_half(mrow[r] + (int64_t)min(t, P.n_kv - 1) * 2);
                            s[r][tt][j] = t < t_end ? __builtin_fmaf(mv, madd, s[r][tt][j]) : -INFINITY;
                        }
                    }
                } else if constexpr (MASK == 1) {
                    if constexpr (full) {
                        const u2 mw = mwv[r][tt];
                        const h2 a = as_h2(mw[0]), c2 = as_h2(mw[1]);
                        s[r][tt][0] = s[r][tt][0] * mmul + (float)a[0] * 1.4426950408889634f;
                        s[r][tt][1] = s[r][tt][1] * mmul + (float)a[1] * 1.4426950408889634f;
                        s[r][tt][2] = s[r][tt][2] * mmul + (float)c2[0] * 1.4426950408889634f;
                        s[r][tt][3] = s[r][tt][3] * mmul + (float)c2[1] * 1.4426950408889634f;
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int t = tb + j;
                            const float mv = ldg_half(mrow[r] + (int64_t)min(t, P.n_kv - 1) * 2);
                            s[r][tt][j] = t < t_end ? s[r][tt][j] * mmul + mv * 1.4426950408889634f : -INFINITY;
                        }
                    }
                } else if constexpr (!full) {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if (tb + j >= t_end) s[r][tt][j] = -INFINITY;
                }
#pragma unroll
                for (int j = 0; j < 4; j++) mx = fmaxf(mx, s[r][tt][j]);
            }
            // A row's maximum can only clear the threshold if one of its lanes' maxima does: the
            // cross-lane reduction and the raise run only when some lane of the wave needs it
            // (the first tiles, then rarely), and give the same reference as running every tile
            if (__builtin_amdgcn_ballot_w64(mx * sm2 > m_ref[r] + ROWS_RESCALE_LOG2)) { // uniform
                mx = wave_max16x4(mx) * sm2;
                const bool raise = mx > m_ref[r] + ROWS_RESCALE_LOG2;
                const float m_new = raise ? mx : m_ref[r];
                if (__builtin_amdgcn_ballot_w64(raise && m_ref[r] != -INFINITY)) { // uniform
                    const float alpha = fast_exp2(m_ref[r] - m_new);
                    l_run[r] *= alpha;
                    corr[r][0] *= alpha;
                    corr[r][1] *= alpha;
#pragma unroll
                    for (int i = 0; i < 4; i++) oacc[r][i] *= alpha;
                    lacc[r] *= alpha;
                }
                m_ref[r] = m_new;
            }
            const float m_use = m_ref[r] == -INFINITY ? 0.0f : m_ref[r];
#pragma unroll
            for (int tt = 0; tt < NTILE; tt++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float p = fast_exp2(__builtin_fmaf(s[r][tt][j], sm2, -m_use));
                    s[r][tt][j] = p;
                    // with quantized V the row sum is taken here; otherwise from the fp16 weights
                    // the PV product uses (an extra MFMA against a ones row, below)
                    if constexpr (is_quant(VT)) l_run[r] += p;
                }
            // P^T operands: 32 tokens (tiles 2kb and 2kb+1) per MFMA, V block scale folded in
#pragma unroll
            for (int kb = 0; kb < NKB; kb++) {
                const f4 plo = s[r][2 * kb], phi = s[r][2 * kb + 1];
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    f4 xlo = plo, xhi = phi;
                    if constexpr (is_quant(VT)) {
                        xlo = plo * *(const f4 *)&cS(2, b)[32 * kb + 4 * g];
                        xhi = phi * *(const f4 *)&cS(2, b)[32 * kb + 16 + 4 * g];
                    }
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        pb[r][kb][b][j] = (_Float16)xlo[j];
                        pb[r][kb][b][4 + j] = (_Float16)xhi[j];
                    }
                    if constexpr (has_min(VT)) {
                        const f4 mlo = *(const f4 *)&cS(3, b)[32 * kb + 4 * g];
                        const f4 mhi = *(const f4 *)&cS(3, b)[32 * kb + 16 + 4 * g];
                        const f4 t = plo * mlo + phi * mhi;
                        corr[r][b] += t[0] + t[1] + t[2] + t[3];
                    }
                    if constexpr (!is_quant(VT)) {
                        pb[r][kb][1] = pb[r][kb][0]; // one B operand serves both blocks
                        break;
                    }
                }
            }
        }

        return true;
    };

    // ---- O^T += V^T P^T for the tile whose P^T operands are in pb (V buffer vb): each V^T
    //      operand (two ds_read_b64_tr_b16) serves every row set ----
    auto pv = [&](int vb) {
        const _Float16 *cV = sV[vb] + hk * TS * RSV;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const int vrow = 32 * kb + 4 * g + (col >> 2);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                h4 lo, hi;
                if constexpr (VTR) {
                    // dim-major tile: dim 16i+col, tokens 4g..4g+3 and 16+4g..16+4g+3 of the 32
                    const _Float16 *va = cV + (16 * i + col) * RSV + 32 * kb + 4 * g;
                    lo = *(const h4 *)va;
                    hi = *(const h4 *)(va + 16);
                } else {
                    const _Float16 *va = cV + vrow * RSV + 16 * i + 4 * (col & 3);
                    lo = __builtin_bit_cast(
                        h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t *)va));
                    hi = __builtin_bit_cast(
                        h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                (__attribute__((address_space(3))) short4_t *)(va + 16 * RSV)));
                }
                const h8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
                for (int r = 0; r < NR; r++)
                    oacc[r][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb[r][kb][i >> 1], oacc[r][i], 0, 0, 0);
            }
            if constexpr (!is_quant(VT)) {
#pragma unroll
                for (int r = 0; r < NR; r++)
                    lacc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones_a, pb[r][kb][0], lacc[r], 0, 0, 0);
            }
        }
    };

    // ---- pipeline: step s runs the PV product of tile s-1 (V buffer (s-1)%3, its operands kept
    //      in pb across the barrier), then QK and softmax of tile s (K buffer s&1), while tile
    //      s+1 is unpacked into K buffer (s+1)&1 and V buffer (s+1)%3 from registers loaded two
    //      steps earlier; no buffer is written in the step that reads it ----
    if (nsteps > 0) write_tile(R[0], 0, tok(0));
    load_tile(tok(NRB), R[0]);
    __syncthreads();
    // full steps run in the loop; only the last step can be partial, and it runs after the loop
    // from the buffers the loop staged it into
    const int t_half = hk * TS;                      // this wave's tokens within a step
    bool pend = false; // SHIFT: pb holds a tile whose PV product has not run (uniform per wave)
    auto step_full = [&](int s_) {
        const int t0 = tok(s_) + t_half, tn = s_ + 1 < nsteps ? tok(s_ + 1) + t_half : -1;
        if constexpr (SHIFT) {
            if (pend) pv((s_ + NVB - 1) % NVB); // tile s_-1
            pend = qk_soft(s_ & 1, s_ % NVB, t0, tn, std::true_type{});
        } else {
            if (qk_soft(s_ & 1, s_ % NVB, t0, tn, std::true_type{})) pv(s_ % NVB);
        }
    };
    // Every step writes the next tile and issues the loads of the one after (past the walk they
    // stage zeros into buffers nothing reads), and the loop has no early exit: the tile loads
    // are then counted exactly on every path, so each write waits only for its own tile.
    int s0 = 0;
    if constexpr (NRB == 2) {
        for (; s0 + 1 < nfull; s0 += 2) {
            // even step: stage step s0+1 from R[1]
            step_full(s0);
            write_tile(R[1], s0 + 1, tok(s0 + 1));
            load_tile(tok(s0 + 3), R[1]);
            __syncthreads();
            // odd step: stage step s0+2 from R[0]
            step_full(s0 + 1);
            write_tile(R[0], s0 + 2, tok(s0 + 2));
            load_tile(tok(s0 + 4), R[0]);
            __syncthreads();
        }
    }
    for (; NRB > 2 && s0 + NRB <= nfull; s0 += NRB) { // NRB > 2
        // NRB steps with compile-time buffer indexes: step s0+j stages tile s0+j+1 from its
        // buffer, which then takes the loads of tile s0+j+1+NRB
#pragma unroll
        for (int j = 0; j < NRB; j++) {
            step_full(s0 + j);
            write_tile(R[(j + 1) % NRB], s0 + j + 1, tok(s0 + j + 1));
            load_tile(tok(s0 + j + 1 + NRB), R[(j + 1) % NRB]);
            __syncthreads();
        }
    }
    // the last nfull % NRB full steps (s0 is a multiple of NRB, so the buffer indexes continue)
    if constexpr (NRB == 2) {
        if (s0 < nfull) { // an odd count of full steps: the last one
            step_full(s0);
            write_tile(R[1], s0 + 1, tok(s0 + 1));
            __syncthreads();
        }
    } else {
#pragma unroll
        for (int j = 0; j + 1 < NRB; j++) {
            if (s0 + j < nfull) { // uniform
                step_full(s0 + j);
                write_tile(R[(j + 1) % NRB], s0 + j + 1, tok(s0 + j + 1));
                __syncthreads();
            }
        }
    }
    if (nfull < nsteps) {
        // the partial last step: with two key halves, a half's 64 tokens may be full, partial or
        // past the end (uniform per wave)
        const int t0w = tok(nfull) + t_half;
        if (pend) pv((nfull + NVB - 1) % NVB);
        const int kb = nfull & 1, vb = nfull % NVB;
        if constexpr (KH == 1) {
            pend = qk_soft(kb, vb, t0w, -1, std::false_type{});
        } else {
            if (t0w + TS <= t_end) pend = qk_soft(kb, vb, t0w, -1, std::true_type{});
            else if (t0w < t_end) pend = qk_soft(kb, vb, t0w, -1, std::false_type{});
            else pend = false;
        }
        if constexpr (!SHIFT) {
            if (pend) pv(vb);
            pend = false;
        }
    }
    if (pend) pv((nsteps - 1) % NVB);

    // unquantized V: this lane's share of the row sum (the row's lane group 0 holds it all)
    if constexpr (!is_quant(VT)) {
#pragma unroll
        for (int r = 0; r < NR; r++) l_run[r] = g == 0 ? lacc[r][0] : 0.0f;
    }

    // two key halves: half 1 hands (m, l, corr, O) of each lane to the same lane of half 0, which
    // merges them (O and l scale by 2^(m - max), as in a split merge); half 0 alone stores
    const bool writer = KH == 1 || hk == 0; // uniform per wave
    if constexpr (KH == 2) {
        constexpr int XV = 4 + 16;                // values per lane and row set
        float *xch = (float *)&sK[0][0];          // 4 row waves x NR x XV x 64 lanes
        __syncthreads();                          // every wave is done with the K/V tiles
#pragma unroll
        for (int r = 0; r < NR; r++) {
            float *x = xch + ((rw * NR + r) * XV) * 64 + lane;
            if (hk == 1) {
                x[0] = m_ref[r];
                x[64] = l_run[r];
                x[128] = corr[r][0];
                x[192] = corr[r][1];
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) x[(4 + 4 * i + j) * 64] = oacc[r][i][j];
            }
        }
        __syncthreads();
        if (hk == 0) {
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const float *x = xch + ((rw * NR + r) * XV) * 64 + lane;
                const float m1 = x[0];
                const float M = fmaxf(m_ref[r], m1);
                const float w0 = M == -INFINITY ? 0.0f : fast_exp2(m_ref[r] - M);
                const float w1 = M == -INFINITY ? 0.0f : fast_exp2(m1 - M);
                l_run[r] = l_run[r] * w0 + x[64] * w1;
                corr[r][0] = corr[r][0] * w0 + x[128] * w1;
                corr[r][1] = corr[r][1] * w0 + x[192] * w1;
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) oacc[r][i][j] = oacc[r][i][j] * w0 + x[(4 + 4 * i + j) * 64] * w1;
                m_ref[r] = M;
            }
        }
    }

    // ---------------- epilogue ----------------
    // partial slot of (row r of this row group, split s) = slot0 + r * n_splits + s
    const int64_t slot0 = P.part_begin + (((int64_t)bq * U.H_kv + kh) * U.n_rowgroups + rg) * ROWS * P.n_splits;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        l_run[r] = wave_sum16x4(l_run[r]);
        if constexpr (has_min(VT)) {
            corr[r][0] = wave_sum16x4(corr[r][0]);
            corr[r][1] = wave_sum16x4(corr[r][1]);
#pragma unroll
            for (int i = 0; i < 4; i++) oacc[r][i] += corr[r][i >> 1];
        }
        if (writer && row_ok[r]) {
            if (P.n_splits == 1) {
                // a row with every key masked: 0 (flash attention) or NaN (soft_max path)
                const float inv = l_run[r] > 0.0f ? 1.0f / l_run[r] : U.empty_row;
                float *o = P.dst + (((int64_t)bq * U.n_q + iq[r]) * U.H + hq[r]) * HEAD;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    // the output is read by the next operation, not by this launch: non-temporal
                    // stores (a 32 MB store probe: 7.4 -> 6.1 us)
                    __builtin_nontemporal_store(oacc[r][i] * inv, (f4 *)&o[16 * i + 4 * g]);
                }
            } else {
                const int64_t slot = slot0 + (int64_t)(row[r] - rg * ROWS) * P.n_splits + split;
                float *o = U.partials + slot * PART_STRIDE;
                if constexpr (BATCH) {
                    // agent-coherent (sc1) vector stores, the form of agent-scope atomic stores
                    const __amdgpu_buffer_rsrc_t rp = make_rsrc((gu8 *)o, PART_STRIDE * 4);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        __builtin_amdgcn_raw_buffer_store_b128(as_u4(oacc[r][i]), rp, (16 * i + 4 * g) * 4, 0, 16);
                    if (g == 0) __builtin_amdgcn_raw_buffer_store_b64(u2{as_u32(m_ref[r]), as_u32(l_run[r])}, rp, 64 * 4, 0, 16);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++) *(f4 *)&o[16 * i + 4 * g] = oacc[r][i];
                    if (g == 0) {
                        o[64] = m_ref[r];
                        o[65] = l_run[r];
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
                uint32_t *cnt = U.counters + (P.cnt_begin + ((int64_t)bq * U.H_kv + kh) * U.n_rowgroups + rg) * CNT_STRIDE;
                const uint32_t prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const bool last = prev == (uint32_t)(P.n_splits - 1);
                // the last arrival leaves the counter zeroed for the next launch
                if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_last = last ? 1u : 0u;
            }
            __syncthreads();
            if (s_last) merge_splits<ROWS, 64 * NW * KH>(U, P, bq, kh, rg, slot0, tid, (float *)&sK[0][0]);
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
    P.dst[(((int64_t)bq * U.n_q + iq) * U.H + hq) * HEAD + d] = L > 0.0f ? acc / L : U.empty_row;
}

using FaLaunchFn = hipError_t (*)(const FaArgs &, hipStream_t);

template <int KT, int VT, int MASK, bool BATCH, int KH = 1, int NW = ROWS_NW>
hipError_t launch_rows(const FaArgs &a, hipStream_t st) {
    if (a.u.total_units <= 0) return hipSuccess;
    hipLaunchKernelGGL((fa_rows_kernel<KT, VT, MASK, BATCH, KH, NW>), dim3((unsigned)a.u.total_units),
                       dim3(64 * NW * KH), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // single calls merge split partials with a second launch; prepared batches merge in-kernel
    if (!BATCH && a.p0.n_splits > 1 && a.u.total_rows > 0) {
        hipLaunchKernelGGL((fa_combine_kernel<16 * ROWS_SETS * NW, BATCH>), dim3((unsigned)a.u.total_rows), dim3(64), 0, st, a);
        e = hipGetLastError();
    }
    return e;
}

// Launch table [k type index][v type index]; index order f32 f16 q8_0 q4_0 q4_1 q5_0 q5_1.
#define CVATTN_V_ROW(KT, MASK, BATCH, KH)                                                            \
    {launch_rows<KT, T_F32, MASK, BATCH, KH>, launch_rows<KT, T_F16, MASK, BATCH, KH>,             \
     launch_rows<KT, T_Q8_0, MASK, BATCH, KH>, launch_rows<KT, T_Q4_0, MASK, BATCH, KH>,           \
     launch_rows<KT, T_Q4_1, MASK, BATCH, KH>, launch_rows<KT, T_Q5_0, MASK, BATCH, KH>,           \
     launch_rows<KT, T_Q5_1, MASK, BATCH, KH>}
#define CVATTN_TABLE(MASK, BATCH, KH)                                                                 \
    {CVATTN_V_ROW(T_F32, MASK, BATCH, KH), CVATTN_V_ROW(T_F16, MASK, BATCH, KH),                   \
     CVATTN_V_ROW(T_Q8_0, MASK, BATCH, KH), CVATTN_V_ROW(T_Q4_0, MASK, BATCH, KH),                 \
     CVATTN_V_ROW(T_Q4_1, MASK, BATCH, KH), CVATTN_V_ROW(T_Q5_0, MASK, BATCH, KH),                 \
     CVATTN_V_ROW(T_Q5_1, MASK, BATCH, KH)}

} // namespace cvattn
