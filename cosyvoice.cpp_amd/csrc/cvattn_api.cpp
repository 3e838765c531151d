// cvattn_api.cpp -- the C ABI of include/cvattn.h: argument validation (the shape rules of
// ggml_flash_attn_ext / ggml_set_rows as cosyvoice.cpp uses them), workspace planning and
// dispatch to the gfx950 kernels.  No device allocation, no host<->device synchronisation.
#include "../../include/cvattn.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

#include "cvattn_common.h"
#include "cvattn_launch.h"

using namespace cvattn;

namespace {

constexpr int kRowsPerCu = 3;   // resident row-tiled workgroups per CU (register bound)
constexpr int kDecodePerCu = 3; // resident decode workgroups per CU (41 KB of LDS each)

// Compute units of the current device (256 on MI355X).  The attribute is a fixed property of the
// device, so it is read once per device; concurrent first calls store the same value.
int cu_count() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}
constexpr size_t kAlign = 256;

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

bool is_kv_type(int t) {
    return t == T_F32 || t == T_F16 || t == T_Q8_0 || t == T_Q4_0 || t == T_Q4_1 || t == T_Q5_0 || t == T_Q5_1;
}

// A head row of the K/V view must be contiguous: nb0 equals the element/block size.
bool kv_ok(const cvattn_tensor *t) {
    if (!t || !t->data || !is_kv_type(t->type)) return false;
    if (t->ne[0] != HEAD) return false;
    if (t->nb[0] != (size_t)type_bytes(t->type)) return false;
    for (int i = 1; i < 4; i++)
        if (t->ne[i] <= 0 && !(i == 1 && t->ne[1] == 0)) return false;
    return true;
}

struct FaShape {
    int n_q, H, H_kv, G, B, n_kv;
    int n_rows, n_rowgroups;
    FaKernelShape ks;
};

// Transposed V of the non-flash-attention path: [n_kv, Dv, H_kv, B] of f32/f16 with the tokens
// contiguous (src/cosyvoice-kv-cache.cpp:338-345: the view over the [max_seq, H_kv*Dv] cache).
bool vt_ok(const cvattn_tensor *t) {
    if (!t || !t->data || (t->type != T_F32 && t->type != T_F16)) return false;
    if (t->ne[1] != HEAD || t->nb[0] != (size_t)type_bytes(t->type)) return false;
    // element alignment (f32 rows are then 4-byte aligned; f16 rows may be 2-byte aligned)
    if (((uintptr_t)t->data | (uintptr_t)t->nb[1] | (uintptr_t)t->nb[2] | (uintptr_t)t->nb[3]) % t->nb[0]) return false;
    for (int i = 2; i < 4; i++)
        if (t->ne[i] <= 0) return false;
    if (t->ne[0] < 0) return false;
    // the kernel addresses one head's [n_kv, Dv] with 32-bit byte offsets
    return (int64_t)(HEAD - 1) * (int64_t)t->nb[1] + t->ne[0] * (int64_t)t->nb[0] < ((int64_t)1 << 31);
}

// vt: v is the transposed view of the non-flash-attention path (always the row-tiled kernel).
int check_fa(const cvattn_tensor *q, const cvattn_tensor *k, const cvattn_tensor *v,
             const cvattn_tensor *mask, FaShape *sh, bool vt = false) {
    if (!q || !k || !v) return CVATTN_ERR_BAD_ARGS;
    if (!q->data) return CVATTN_ERR_BAD_ARGS;
    if (q->type != T_F32 && q->type != T_F16) return CVATTN_ERR_UNSUPPORTED;
    if (q->ne[0] != HEAD || k->ne[0] != HEAD || (vt ? v->ne[1] : v->ne[0]) != HEAD) return CVATTN_ERR_UNSUPPORTED;
    if (q->nb[0] != (size_t)type_bytes(q->type)) return CVATTN_ERR_UNSUPPORTED;
    if (!kv_ok(k)) return is_kv_type(k->type) ? CVATTN_ERR_BAD_ARGS : CVATTN_ERR_UNSUPPORTED;
    if (vt) {
        // the non-flash-attention V cache must be f32/f16 (src/cosyvoice-loader.cpp:639-641)
        if (v->type != T_F32 && v->type != T_F16) return CVATTN_ERR_UNSUPPORTED;
        if (!vt_ok(v)) return CVATTN_ERR_BAD_ARGS;
    } else if (!kv_ok(v)) {
        return is_kv_type(v->type) ? CVATTN_ERR_BAD_ARGS : CVATTN_ERR_UNSUPPORTED;
    }
    for (int i = 1; i < 4; i++)
        if (q->ne[i] <= 0) return CVATTN_ERR_BAD_ARGS;
    if (k->ne[1] != (vt ? v->ne[0] : v->ne[1])) return CVATTN_ERR_BAD_ARGS;
    if (k->ne[2] != v->ne[2]) return CVATTN_ERR_UNSUPPORTED;
    if (q->ne[2] % k->ne[2]) return CVATTN_ERR_BAD_ARGS;
    if (q->ne[3] % k->ne[3] || q->ne[3] % v->ne[3]) return CVATTN_ERR_BAD_ARGS;
    if (mask && mask->data) {
        if (mask->type != T_F16 || mask->nb[0] != 2) return CVATTN_ERR_UNSUPPORTED;
        if (mask->ne[0] < k->ne[1] || mask->ne[1] < q->ne[1]) return CVATTN_ERR_BAD_ARGS;
        if (mask->ne[2] <= 0 || mask->ne[3] <= 0) return CVATTN_ERR_BAD_ARGS;
        if (q->ne[2] % mask->ne[2] || q->ne[3] % mask->ne[3]) return CVATTN_ERR_BAD_ARGS;
    }
    const int64_t lim = (int64_t)1 << 30;
    if (q->ne[1] >= lim || q->ne[2] >= lim || q->ne[3] >= lim || k->ne[1] >= lim) return CVATTN_ERR_UNSUPPORTED;
    sh->n_q = (int)q->ne[1];
    sh->H = (int)q->ne[2];
    sh->H_kv = (int)k->ne[2];
    sh->G = sh->H / sh->H_kv;
    sh->B = (int)q->ne[3];
    sh->n_kv = (int)k->ne[1];
    sh->n_rows = sh->n_q * sh->G;
    // Both kernels address the K/V rows of one head with 32-bit buffer offsets (token * nb1): a
    // view whose head spans 2^31 bytes or more is not served (the transposed V checks its own
    // extent in vt_ok)
    const int64_t lim31 = ((int64_t)1 << 31) - 1;
    if ((int64_t)k->ne[1] * (int64_t)k->nb[1] >= lim31) return CVATTN_ERR_UNSUPPORTED;
    if (!vt && (int64_t)v->ne[1] * (int64_t)v->nb[1] >= lim31) return CVATTN_ERR_UNSUPPORTED;
    sh->ks = fa_shape(sh->n_rows, !vt);
    sh->n_rowgroups = (sh->n_rows + sh->ks.rows_per_group - 1) / sh->ks.rows_per_group;
    return CVATTN_OK;
}

int check_dst(const cvattn_tensor *dst, const FaShape &sh) {
    if (!dst || !dst->data) return CVATTN_ERR_BAD_ARGS;
    if (dst->type != T_F32) return CVATTN_ERR_UNSUPPORTED;
    const int64_t want[4] = {HEAD, sh.H, sh.n_q, sh.B};
    size_t stride = 4;
    for (int i = 0; i < 4; i++) {
        if (dst->ne[i] != want[i]) return CVATTN_ERR_BAD_ARGS;
        if (dst->nb[i] != stride) return CVATTN_ERR_BAD_ARGS;
        stride *= (size_t)want[i];
    }
    return CVATTN_OK;
}

// Token splits.  Decode-shaped problems (waves split the tokens) size each wave's token run so
// the whole launch has about kTargetWaves waves in flight (an eighth of that when each kv head
// has several row groups, which already multiply the workgroups reading a head: the 50-row DiT
// chunk over 1050 tokens then runs unsplit, 10.2 us against 11.2 us with 3 splits at a half and
// 10.75 us with 2 at a quarter); row-tiled problems
// split only when their row groups alone cannot fill the chip.  `work` is the launch-wide sum
// of B*H_kv*n_rowgroups*n_kv (decode) or of B*H_kv*n_rowgroups (row-tiled).
constexpr int64_t kTargetWaves = 4096;
// row-tiled kernel cost terms (MI355X, measured): one 64-token tile of a workgroup, and the fixed
// cost of a split (partial stores, arrival counter, last-arrival merge)
constexpr double kTileUs = 0.85, kMergeUs = 3.4;
// two_rounds: the decode kernel may merge up to two rounds of splits (long sequences); the
// callers turn it off when the extra splits would not all be resident at once.
void plan_splits(const FaShape &sh, int n_kv, int64_t work, int *n_splits, int *split_len, bool two_rounds = true) {
    // row-tiled with two key halves: 128-token steps
    const int tstep = sh.ks.wsplit ? sh.ks.tstep : sh.ks.tstep * sh.ks.kh;
    int len;
    if (sh.ks.wsplit) {
        // tokens per wave: a multiple of the wave step
        const int64_t tw = sh.n_rowgroups > 1 ? kTargetWaves / 8 : kTargetWaves;
        int64_t wlen = (std::max<int64_t>(1, work) + tw - 1) / tw;
        wlen = std::min<int64_t>(1024, std::max<int64_t>(tstep, (wlen + tstep - 1) / tstep * tstep));
        len = (int)wlen * sh.ks.nw;
    } else {
        // Split only when the row groups leave most resident workgroup slots idle AND the
        // shorter key run pays for the partials: every split writes (and the merge reads back) a
        // full fp32 partial of each of its rows through agent-coherent stores and loads, which
        // measured ~0.9 TB/s plus ~3.4 us, against ~0.85 us per 64-token tile of a workgroup
        // (1024-token prefill: 16.7 us unsplit vs 21.8 / 24.4 us with 2 / 3 splits).
        const int min_split = 256;
        const int64_t base = std::max<int64_t>(1, work);
        // two halves (90 KB LDS) and the wide form (12 waves): 1 per CU
        const int64_t slots = (sh.ks.kh == 2 || sh.ks.rows_per_group > 64 ? 1 : kRowsPerCu) * cu_count();
        int want = 1;
        if (2 * base < slots) {
            want = (int)((slots + base - 1) / base);
            want = std::min(want, std::max(1, (n_kv + min_split - 1) / min_split));
            want = std::min(want, sh.ks.max_splits);
            if (want > 1) {
                const double tiles = (double)((n_kv + tstep - 1) / tstep); // steps of tstep tokens
                const double step_us = kTileUs * tstep / sh.ks.tstep / sh.ks.kh; // halves run side by side
                const double part_us = (double)want * (double)base * sh.ks.rows_per_group * PART_STRIDE * 4 / 0.9e6;
                const double t_one = tiles * step_us;
                const double t_split = std::ceil(tiles / want) * step_us + kMergeUs + part_us;
                if (t_split >= t_one) want = 1;
            }
        }
        len = (n_kv + want - 1) / want;
        len = std::max(tstep, (len + tstep - 1) / tstep * tstep);
    }
    const int unit = sh.ks.wsplit ? tstep * sh.ks.nw : tstep;
    // never more splits than the in-kernel merge takes; the decode kernel's second merge round
    // is used only for sequences that one round's splits would leave long per workgroup
    int max_splits = sh.ks.max_splits;
    if (sh.ks.wsplit &&
        (!two_rounds || (n_kv + sh.ks.round_splits - 1) / sh.ks.round_splits <= sh.ks.long_split))
        max_splits = sh.ks.round_splits;
    const int min_len = (n_kv + max_splits - 1) / max_splits;
    if (len < min_len) len = (min_len + unit - 1) / unit * unit;
    *split_len = len;
    *n_splits = n_kv > 0 ? (n_kv + len - 1) / len : 1;
}

int64_t split_work(const FaShape &sh) {
    const int64_t groups = (int64_t)sh.B * sh.H_kv * sh.n_rowgroups;
    return sh.ks.wsplit ? groups * sh.n_kv : groups;
}

void fill_problem(FaProblem &p, const cvattn_tensor *q, const cvattn_tensor *k, const cvattn_tensor *v,
                  const cvattn_tensor *mask, const cvattn_tensor *dst, const FaShape &sh) {
    std::memset(&p, 0, sizeof(p));
    p.q = q->data;
    p.k = k->data;
    p.v = v->data;
    p.dst = (float *)dst->data;
    p.q_nb1 = (int64_t)q->nb[1];
    p.q_nb2 = (int64_t)q->nb[2];
    p.q_nb3 = (int64_t)q->nb[3];
    p.k_nb1 = (int64_t)k->nb[1];
    p.k_nb2 = (int64_t)k->nb[2];
    p.k_nb3 = (int64_t)k->nb[3];
    p.v_nb1 = (int64_t)v->nb[1];
    p.v_nb2 = (int64_t)v->nb[2];
    p.v_nb3 = (int64_t)v->nb[3];
    if (mask && mask->data) {
        p.mask = mask->data;
        p.m_nb1 = (int64_t)mask->nb[1];
        p.m_nb2 = (int64_t)mask->nb[2];
        p.m_nb3 = (int64_t)mask->nb[3];
        p.m_ne2 = (int32_t)mask->ne[2];
        p.m_ne3 = (int32_t)mask->ne[3];
    } else {
        p.m_ne2 = 1;
        p.m_ne3 = 1;
    }
    p.n_kv = sh.n_kv;
    p.rk3 = (int32_t)(sh.B / k->ne[3]);
    p.rv3 = (int32_t)(sh.B / v->ne[3]);
    // 16-byte loads need 4-byte aligned rows (a transposed f16 V over an odd max_seq has 2)
    p.v_align2 = (((uintptr_t)v->data | (uintptr_t)v->nb[1] | (uintptr_t)v->nb[2] | (uintptr_t)v->nb[3]) & 3) != 0;
}

void fill_uniform(FaUniform &u, const FaShape &sh, int q_type, float scale) {
    std::memset(&u, 0, sizeof(u));
    u.n_q = sh.n_q;
    u.H = sh.H;
    u.H_kv = sh.H_kv;
    u.G = sh.G;
    u.B = sh.B;
    u.n_rows = sh.n_rows;
    u.n_rowgroups = sh.n_rowgroups;
    u.q_f16 = q_type == T_F16 ? 1 : 0;
    u.scale = scale;
    u.scale_log2 = scale * 1.4426950408889634f;
    u.div_hkv = make_fastdiv((uint32_t)sh.H_kv);
    u.div_rowgroups = make_fastdiv((uint32_t)sh.n_rowgroups);
    u.div_upp = make_fastdiv(1);
}

// The preloaded addressing of a decode launch (DecPre) when its problems allow it: one sequence,
// one query token and so one row group per kv head, no mask, a static n_kv, f32 Q with contiguous
// heads, kv heads dense in the cache rows, row bytes and split lengths below 2^16, and problem
// i's K, V and Q at i times a fixed int32 byte stride from problem 0's, all with the same n_kv and
// split plan.  Leaves a.pre zeroed (the kernel then locates its problem in memory) otherwise.
void fill_dec_pre(FaArgs &a, const FaShape &sh, const FaProblem *probs, int n, int q_type, bool has_mask) {
    std::memset(&a.pre, 0, sizeof(a.pre));
    if (!sh.ks.wsplit || has_mask || n < 1 || sh.B != 1 || sh.n_q != 1 || sh.n_rowgroups != 1) return;
    if (q_type != T_F32 || sh.H_kv > 255 || sh.G > 255) return;
    const FaProblem &p0 = probs[0];
    if (p0.n_kv_dev || p0.q_nb2 != HEAD * 4) return;
    for (const int64_t nb1_nb2 : {p0.k_nb1, p0.v_nb1})
        if (nb1_nb2 <= 0 || nb1_nb2 >= 65536 || nb1_nb2 % sh.H_kv) return;
    if (p0.k_nb2 * sh.H_kv != p0.k_nb1 || p0.v_nb2 * sh.H_kv != p0.v_nb1) return;
    if (p0.split_len <= 0 || p0.split_len >= 65536 || p0.n_splits >= 256 || p0.n_kv >= (1 << 24)) return;
    const int64_t k_ps = n > 1 ? (const uint8_t *)probs[1].k - (const uint8_t *)p0.k : 0;
    const int64_t v_ps = n > 1 ? (const uint8_t *)probs[1].v - (const uint8_t *)p0.v : 0;
    const int64_t q_ps = n > 1 ? (const uint8_t *)probs[1].q - (const uint8_t *)p0.q : 0;
    for (const int64_t ps : {k_ps, v_ps, q_ps})
        if (ps < INT32_MIN || ps > INT32_MAX) return;
    // outputs at a uniform float stride, and the partial slots and counters the planner laid out
    // problem after problem (H_kv groups each)
    const int64_t dst_ps = n > 1 ? probs[1].dst - p0.dst : 0;
    for (int i = 0; i < n; i++) {
        const FaProblem &pi = probs[i];
        if ((const uint8_t *)pi.k - (const uint8_t *)p0.k != i * k_ps ||
            (const uint8_t *)pi.v - (const uint8_t *)p0.v != i * v_ps ||
            (const uint8_t *)pi.q - (const uint8_t *)p0.q != i * q_ps)
            return;
        if (pi.dst - p0.dst != i * dst_ps) return;
        const int64_t groups = (int64_t)sh.H_kv;
        if (pi.part_begin != (p0.n_splits > 1 ? i * groups * 16 * p0.n_splits : 0) ||
            (p0.n_splits > 1 && pi.cnt_begin != i * groups))
            return;
        if (pi.n_kv != p0.n_kv || pi.n_splits != p0.n_splits || pi.split_len != p0.split_len || pi.n_kv_dev ||
            pi.k_nb1 != p0.k_nb1 || pi.v_nb1 != p0.v_nb1 || pi.k_nb2 != p0.k_nb2 || pi.v_nb2 != p0.v_nb2 ||
            pi.q_nb2 != p0.q_nb2)
            return;
    }
    DecPre &d = a.pre;
    d.k = (const uint8_t *)p0.k;
    d.v = (const uint8_t *)p0.v;
    d.q = (const uint8_t *)p0.q;
    d.k_ps = (int32_t)k_ps;
    d.v_ps = (int32_t)v_ps;
    d.q_ps = (int32_t)q_ps;
    d.kv = (uint32_t)p0.n_kv | ((uint32_t)p0.n_splits << 24);
    d.lens = (uint32_t)p0.split_len | ((uint32_t)p0.k_nb1 << 16);
    d.shape = (uint32_t)p0.v_nb1 | ((uint32_t)sh.H_kv << 16) | ((uint32_t)sh.G << 24);
    d.units = (uint32_t)a.u.total_units;
    d.scale_log2 = a.u.scale_log2;
    a.dst_ps = dst_ps;
}

// Workgroup units of a launch are decomposed with 32-bit arithmetic.
constexpr int64_t kMaxUnits = ((int64_t)1 << 31) - 1;

int64_t slots_per_split(const FaShape &sh) {
    return (int64_t)sh.B * sh.H_kv * sh.n_rowgroups * sh.ks.rows_per_group;
}

// Plan for a single problem: splits, fp16 copies of fp32 K/V, and the workspace size
// ([split partials | K copy | V copy], each part 256-byte aligned).
struct SinglePlan {
    FaShape sh;
    int n_splits, split_len;
    bool cvt_k, cvt_v;
    size_t k_off, v_off;
    int64_t v_row; // halfs per row of the V copy
    size_t mcls_off;  // mask tile classes (row-tiled kernel): n_rowgroups x mcls_ld bytes
    int mcls_ld;      // key tiles per row group, 0: not classified
    size_t ws_bytes;
};

// Key tiles whose mask class the row-tiled kernel reads (0: the mask is not classified).  Masks
// shared by every head and sequence (ne2 = ne3 = 1: the causal LLM mask, the DiT chunk mask) over
// 2..MCLS_MAX_TILES key tiles, in launches of one key half per workgroup (more row groups than
// CUs, e.g. the T=1500 DiT call).  A pass over the mask before the attention launch then lets a
// workgroup stage only the key tiles that are not all -inf for its row group, and skip the mask
// words of tiles that are all 0.  Launches with two key halves (fewer row groups than CUs) are not
// classified: their critical path is the longest row group, which the classes do not shorten,
// and the extra pass measured slower there (1024-token causal prefill 18.1 -> 21.7 us).
int mcls_tiles(const FaShape &sh, const cvattn_tensor *mask, int ktype, int vtype) {
    if (!mask || !mask->data || sh.ks.wsplit || sh.ks.kh != 1 || !rows_cls_ok(ktype, vtype)) return 0;
    if (mask->ne[2] != 1 || mask->ne[3] != 1) return 0;
    const int nkt = (sh.n_kv + ROWS_TILE - 1) / ROWS_TILE;
    return nkt >= 2 && nkt <= MCLS_MAX_TILES ? nkt : 0;
}

// fp32 K/V read by at least this many row groups are copied once to fp16 in the workspace
// before the row-tiled kernel runs: the kernel stages fp32 tiles by converting them to fp16
// anyway (the copy rounds the same way, so the staged tiles are the same), and staging fp32 holds
// twice the registers, which keeps fewer workgroups resident (DiT T=1500, 16 heads, batch 2:
// 84-90 us from fp32 views, 43 us from fp16 K/V).  The copy costs one pass over K/V, paid back
// when several row groups re-read every tile.
constexpr int kCvtMinRowGroups = 4;

int64_t view_rows(const cvattn_tensor *t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

// The wide row-tiled form: one 192-row workgroup per CU, whose 12 waves share each staged K/V
// tile (a third of the staging per row of the 64-row form).  Taken for unmasked one-half launches
// of fp16 K/V with no split whose 192-row groups still give every CU one: the DiT call (T=1500,
// 2 x 16 heads: 256 groups) 37.7-38.0 -> 33.3-34.8 us.
static void make_wide(FaShape &sh) {
    fa_shape_wide(sh.ks);
    sh.n_rowgroups = (sh.n_rows + sh.ks.rows_per_group - 1) / sh.ks.rows_per_group;
}
static int64_t wide_groups(FaShape sh) {
    make_wide(sh);
    return (int64_t)sh.B * sh.H_kv * sh.n_rowgroups;
}

// Two key halves per row-tiled workgroup when the row groups alone would leave CUs idle (one
// 8-wave workgroup per CU then runs each row set's key range in two halves); not for the
// transposed-V form, whose dim-major tile holds one 64-token step.
void choose_kh(FaShape &sh, int64_t groups, bool vt) {
    sh.ks.kh = !sh.ks.wsplit && !vt && groups <= cu_count() ? 2 : 1;
}

int plan_single(const cvattn_tensor *q, const cvattn_tensor *k, const cvattn_tensor *v,
                const cvattn_tensor *mask, SinglePlan *pl, bool vt = false) {
    int rc = check_fa(q, k, v, mask, &pl->sh, vt);
    if (rc) return rc;
    choose_kh(pl->sh, split_work(pl->sh), vt);
    const FaShape &sh = pl->sh;
    plan_splits(sh, sh.n_kv, split_work(sh), &pl->n_splits, &pl->split_len);
    if (sh.ks.wsplit && (int64_t)sh.B * sh.H_kv * sh.n_rowgroups * pl->n_splits > kDecodePerCu * cu_count())
        plan_splits(sh, sh.n_kv, split_work(sh), &pl->n_splits, &pl->split_len, false);
    size_t bytes = pl->n_splits > 1 ? (size_t)slots_per_split(sh) * pl->n_splits * PART_STRIDE * sizeof(float) : 0;
    const bool many = !sh.ks.wsplit && sh.n_rowgroups >= kCvtMinRowGroups;
    // the transposed V's rows are its tokens: padded to 8 halfs, so they stay 16-byte aligned
    const int64_t v_row = vt ? (v->ne[0] + 7) / 8 * 8 : HEAD;
    // (an empty view -- n_kv 0 -- has nothing to copy)
    pl->cvt_k = many && k->type == T_F32 && view_rows(k) > 0 && view_rows(k) * (HEAD / 8) <= kCvtMaxChunks;
    pl->cvt_v = many && v->type == T_F32 && view_rows(v) > 0 && view_rows(v) * (v_row / 8) <= kCvtMaxChunks;
    pl->k_off = pl->v_off = 0;
    pl->v_row = 0;
    if (pl->cvt_k) {
        pl->k_off = bytes = align_up(bytes, kAlign);
        bytes += (size_t)view_rows(k) * HEAD * sizeof(_Float16);
    }
    if (pl->cvt_v) {
        pl->v_row = v_row;
        pl->v_off = bytes = align_up(bytes, kAlign);
        bytes += (size_t)view_rows(v) * (size_t)pl->v_row * sizeof(_Float16);
    }
    // (the kernel sees the fp16 copies' type; the transposed-V form is not classified)
    if (!vt && !sh.ks.wsplit && sh.ks.kh == 1 && pl->n_splits == 1 && !(mask && mask->data) &&
        rows_wide_ok(pl->cvt_k ? T_F16 : k->type, pl->cvt_v ? T_F16 : v->type) && wide_groups(sh) >= cu_count())
        make_wide(pl->sh);
    pl->mcls_ld = vt ? 0 : mcls_tiles(sh, mask, pl->cvt_k ? T_F16 : k->type, pl->cvt_v ? T_F16 : v->type);
    pl->mcls_off = 0;
    if (pl->mcls_ld) {
        // the classes, then the prefix lengths (64 per block)
        pl->mcls_off = bytes = align_up(bytes, kAlign);
        bytes += (size_t)mcls_table_bytes((int64_t)sh.n_rowgroups * pl->mcls_ld);
    }
    pl->ws_bytes = bytes;
    return CVATTN_OK;
}

// Describe the copy of an fp32 view into the workspace as dense fp16 rows of `row` halfs (`c`,
// for cvt_f16_launch) and the copy as a view of the same shape (`out`).
void copy_to_f16(const cvattn_tensor *t, uint8_t *dst, int64_t row, CvtF16Args &c, cvattn_tensor *out) {
    c.src = (const uint8_t *)t->data;
    c.dst = (_Float16 *)dst;
    c.ne0 = t->ne[0];
    c.ne1 = t->ne[1];
    c.ne2 = t->ne[2];
    c.nb1 = (int64_t)t->nb[1];
    c.nb2 = (int64_t)t->nb[2];
    c.nb3 = (int64_t)t->nb[3];
    c.dst_row = row;
    c.chunks = row / 8;
    c.total = view_rows(t) * c.chunks;
    *out = *t;
    out->type = T_F16;
    out->data = dst;
    out->nb[0] = sizeof(_Float16);
    out->nb[1] = (size_t)row * sizeof(_Float16);
    out->nb[2] = out->nb[1] * (size_t)t->ne[1];
    out->nb[3] = out->nb[2] * (size_t)t->ne[2];
}

// Host-side launch plan for batches (stored in cvattn_fa_plan::opaque).
struct BatchPlan {
    uint32_t magic;
    int32_t ktype, vtype, has_mask;
    FaKernelShape ks;
    FaArgs args;
};
static_assert(sizeof(BatchPlan) <= sizeof(cvattn_fa_plan), "plan too large");
constexpr uint32_t kPlanMagic = 0x43564150u;

int hip_status(hipError_t e) { return e == hipSuccess ? CVATTN_OK : CVATTN_ERR_HIP; }

} // namespace

// Workspace of cvattn_flash_attn_ext_noalloc: one array per GPU the library runs on, held until
// the process ends.  Host code never passes `scratch` itself to a kernel or a copy (on the host it
// is only a stand-in for the device symbol): the device address comes from hipGetSymbolAddress,
// once per device with that device current, and is kept per device below.
constexpr size_t kNoallocScratchBytes = (size_t)CVATTN_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
static std::atomic<void *> g_scratch_ptr[kMaxDevices];

// Device address of this device's `scratch`, looked up on the first call on the device (concurrent
// first calls look up the same address).  nullptr on failure.
static void *noalloc_scratch() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    void *ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (ptr) return ptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    return ptr;
}

extern "C" {

CVATTN_API int cvattn_supports_flash_attn_ext(const cvattn_tensor *q, const cvattn_tensor *k,
                                              const cvattn_tensor *v, const cvattn_tensor *mask) {
    FaShape sh;
    return check_fa(q, k, v, mask, &sh) == CVATTN_OK ? 1 : 0;
}

CVATTN_API size_t cvattn_flash_attn_ext_workspace(const cvattn_tensor *q, const cvattn_tensor *k,
                                                  const cvattn_tensor *v, const cvattn_tensor *mask) {
    SinglePlan pl;
    if (plan_single(q, k, v, mask, &pl)) return 0;
    return pl.ws_bytes;
}

static int run_single(const cvattn_tensor *q, const cvattn_tensor *k, const cvattn_tensor *v,
                      const cvattn_tensor *mask, const cvattn_tensor *dst, float scale, void *ws, size_t ws_bytes,
                      cvattn_stream_t stream, bool vt);

CVATTN_API int cvattn_flash_attn_ext(const cvattn_tensor *q, const cvattn_tensor *k,
                                     const cvattn_tensor *v, const cvattn_tensor *mask,
                                     const cvattn_tensor *dst, float scale, float max_bias,
                                     float logit_softcap, int prec, void *ws, size_t ws_bytes,
                                     cvattn_stream_t stream) {
    if (max_bias != 0.0f || logit_softcap != 0.0f) return CVATTN_ERR_UNSUPPORTED;
    if (prec != CVATTN_PREC_DEFAULT && prec != CVATTN_PREC_F32) return CVATTN_ERR_BAD_ARGS;
    if (!std::isfinite(scale)) return CVATTN_ERR_BAD_ARGS;
    return run_single(q, k, v, mask, dst, scale, ws, ws_bytes, stream, false);
}

// One problem, one launch (plus the split merge).  vt: the non-flash-attention form (transposed
// V, soft_max's NaN for a row with every key masked).
static int run_single(const cvattn_tensor *q, const cvattn_tensor *k, const cvattn_tensor *v,
                      const cvattn_tensor *mask, const cvattn_tensor *dst, float scale, void *ws, size_t ws_bytes,
                      cvattn_stream_t stream, bool vt) {
    SinglePlan pl;
    int rc = plan_single(q, k, v, mask, &pl, vt);
    if (rc) return rc;
    rc = check_dst(dst, pl.sh);
    if (rc) return rc;
    if (ws_bytes < pl.ws_bytes || (pl.ws_bytes && !ws)) return CVATTN_ERR_WORKSPACE_TOO_SMALL;
    if (pl.ws_bytes && ((uintptr_t)ws & (kAlign - 1))) return CVATTN_ERR_BAD_ARGS; // tables use aligned vector stores
    cvattn_tensor k16, v16;
    CvtF16Args cvt[2];
    int n_cvt = 0;
    if (pl.cvt_k) {
        copy_to_f16(k, (uint8_t *)ws + pl.k_off, HEAD, cvt[n_cvt++], &k16);
        k = &k16;
    }
    if (pl.cvt_v) {
        copy_to_f16(v, (uint8_t *)ws + pl.v_off, pl.v_row, cvt[n_cvt++], &v16);
        v = &v16;
    }
    if (n_cvt && cvt_f16_launch(cvt, n_cvt, (hipStream_t)stream) != hipSuccess) return CVATTN_ERR_HIP;
    FaArgs a;
    std::memset(&a, 0, sizeof(a));
    fill_uniform(a.u, pl.sh, q->type, scale);
    if (vt) a.u.empty_row = std::numeric_limits<float>::quiet_NaN();
    fill_problem(a.p0, q, k, v, mask, dst, pl.sh);
    a.p0.n_splits = pl.n_splits;
    a.p0.div_splits = make_fastdiv((uint32_t)pl.n_splits);
    a.p0.split_len = pl.split_len;
    a.u.n_problems = 1;
    a.u.total_units = (int64_t)pl.sh.B * pl.sh.H_kv * pl.sh.n_rowgroups * pl.n_splits;
    if (a.u.total_units > kMaxUnits) return CVATTN_ERR_UNSUPPORTED;
    a.u.total_rows = (int64_t)pl.sh.B * pl.sh.H * pl.sh.n_q;
    a.u.partials = (float *)ws;
    const bool has_mask = mask && mask->data;
    if (!vt) fill_dec_pre(a, pl.sh, &a.p0, 1, q->type, has_mask);
    if (pl.mcls_ld) {
        a.p0.mcls = (uint8_t *)ws + pl.mcls_off;
        a.p0.mcls_ld = pl.mcls_ld;
        a.p0.mcls_begin = 0;
        a.u.mcls_blocks = (int64_t)pl.sh.n_rowgroups * pl.mcls_ld;
        if (mask_classify_launch(a, false, (hipStream_t)stream) != hipSuccess) return CVATTN_ERR_HIP;
    }
    if (vt)
        return hip_status(fa_launch_vt(k->type, v->type == T_F32 ? T_VT_F32 : T_VT_F16, has_mask, a,
                                       (hipStream_t)stream));
    return hip_status(fa_launch(pl.sh.ks, k->type, v->type, has_mask, false, a, (hipStream_t)stream));
}

// ---- the no-allocation variant ------------------------------------------------------------------

CVATTN_API int cvattn_flash_attn_ext_noalloc(const cvattn_tensor *q, const cvattn_tensor *k,
                                             const cvattn_tensor *v, const cvattn_tensor *mask,
                                             const cvattn_tensor *dst, float scale, float max_bias,
                                             float logit_softcap, int prec, cvattn_stream_t stream) {
    if (max_bias != 0.0f || logit_softcap != 0.0f) return CVATTN_ERR_UNSUPPORTED;
    if (prec != CVATTN_PREC_DEFAULT && prec != CVATTN_PREC_F32) return CVATTN_ERR_BAD_ARGS;
    if (!std::isfinite(scale)) return CVATTN_ERR_BAD_ARGS;
    SinglePlan pl;
    int rc = plan_single(q, k, v, mask, &pl);
    if (rc) return rc;
    if (pl.ws_bytes > kNoallocScratchBytes) return CVATTN_ERR_WORKSPACE_TOO_SMALL;
    void *ws = noalloc_scratch();
    if (!ws) return CVATTN_ERR_HIP;
    // The kernels fully write every byte of the workspace they later read (split partials, fp16
    // copies); nothing in it has to start at zero.
    return run_single(q, k, v, mask, dst, scale, ws, kNoallocScratchBytes, stream, false);
}

// ---- the non-flash-attention node sequence ----------------------------------------------------

CVATTN_API int cvattn_supports_attn_nonfa(const cvattn_tensor *q, const cvattn_tensor *k, const cvattn_tensor *vt,
                                          const cvattn_tensor *mask) {
    FaShape sh;
    return check_fa(q, k, vt, mask, &sh, true) == CVATTN_OK ? 1 : 0;
}

CVATTN_API size_t cvattn_attn_nonfa_workspace(const cvattn_tensor *q, const cvattn_tensor *k,
                                              const cvattn_tensor *vt, const cvattn_tensor *mask) {
    SinglePlan pl;
    if (plan_single(q, k, vt, mask, &pl, true)) return 0;
    return pl.ws_bytes;
}

CVATTN_API int cvattn_attn_nonfa(const cvattn_tensor *q, const cvattn_tensor *k, const cvattn_tensor *vt,
                                 const cvattn_tensor *mask, const cvattn_tensor *dst, float scale, void *ws,
                                 size_t ws_bytes, cvattn_stream_t stream) {
    if (!std::isfinite(scale)) return CVATTN_ERR_BAD_ARGS;
    return run_single(q, k, vt, mask, dst, scale, ws, ws_bytes, stream, true);
}

// ---- batches ------------------------------------------------------------------------------

// Workspace of a prepared batch: [problem table | split-arrival counters | split partials].
struct BatchLayout {
    size_t table_bytes, counter_bytes, total_bytes;
    size_t mcls_off;   // mask tile classes after the partials (problem i at mcls_begin bytes)
    int64_t mcls_blocks;
    int64_t units, rows;
};

// n_kv_dev: plans whose n_kv is read from device memory at each launch (problem i reads
// n_kv_dev[i * n_kv_stride]); the views' ne[1] is then the capacity the splits are planned for.
static int plan_batch(const cvattn_fa_problem *probs, int n, std::vector<FaProblem> *table, FaShape *sh0,
                      BatchLayout *lay, const int32_t *n_kv_dev = nullptr, int n_kv_stride = 0) {
    if (!probs || n <= 0) return CVATTN_ERR_BAD_ARGS;
    const bool has_mask = probs[0].mask.data != nullptr;
    int rc = check_fa(&probs[0].q, &probs[0].k, &probs[0].v, has_mask ? &probs[0].mask : nullptr, sh0);
    if (rc) return rc;
    int64_t work = 0;
    for (int i = 0; i < n; i++) {
        const cvattn_fa_problem &p = probs[i];
        FaShape sh;
        if ((p.mask.data != nullptr) != has_mask) return CVATTN_ERR_BAD_ARGS;
        rc = check_fa(&p.q, &p.k, &p.v, has_mask ? &p.mask : nullptr, &sh);
        if (rc) return rc;
        rc = check_dst(&p.dst, sh);
        if (rc) return rc;
        if (p.q.type != probs[0].q.type || p.k.type != probs[0].k.type || p.v.type != probs[0].v.type)
            return CVATTN_ERR_BAD_ARGS;
        if (sh.n_q != sh0->n_q || sh.H != sh0->H || sh.H_kv != sh0->H_kv || sh.B != sh0->B) return CVATTN_ERR_BAD_ARGS;
        // one launch runs one kernel shape (e.g. a view too large for 32-bit offsets among
        // decode problems cannot join them)
        if (sh.ks.wsplit != sh0->ks.wsplit) return CVATTN_ERR_UNSUPPORTED;
        work += split_work(sh);
    }
    if (table) table->resize(n);
    choose_kh(*sh0, work, false);
    // the wide form (make_wide) when the launch's 192-row groups give every CU one
    bool wide = !sh0->ks.wsplit && sh0->ks.kh == 1 && !has_mask && rows_wide_ok(probs[0].k.type, probs[0].v.type);
    if (wide) {
        int64_t g = 0;
        for (int i = 0; i < n; i++) {
            FaShape sh;
            check_fa(&probs[i].q, &probs[i].k, &probs[i].v, nullptr, &sh);
            g += wide_groups(sh);
        }
        wide = g >= cu_count();
        if (wide) make_wide(*sh0);
    }
    // decode: a second merge round only if all workgroups of the launch stay resident
    bool two_rounds = true;
    if (sh0->ks.wsplit) {
        int64_t units = 0;
        for (int i = 0; i < n; i++) {
            const cvattn_fa_problem &p = probs[i];
            FaShape sh;
            check_fa(&p.q, &p.k, &p.v, has_mask ? &p.mask : nullptr, &sh);
            int ns, sl;
            plan_splits(sh, sh.n_kv, work, &ns, &sl);
            units += (int64_t)sh.B * sh.H_kv * sh.n_rowgroups * ns;
        }
        two_rounds = units <= kDecodePerCu * cu_count();
    }
    int64_t unit = 0, part = 0, row = 0, cnt = 0;
    for (int i = 0; i < n; i++) {
        const cvattn_fa_problem &p = probs[i];
        FaShape sh;
        check_fa(&p.q, &p.k, &p.v, has_mask ? &p.mask : nullptr, &sh);
        sh.ks.kh = sh0->ks.kh;
        if (wide) make_wide(sh);
        int ns, sl;
        plan_splits(sh, sh.n_kv, work, &ns, &sl, two_rounds);
        // (the wide form never splits: its launches have more 64-row groups than CUs, so the
        // planner's slots, one workgroup per CU, are never half idle)
        if (wide && ns != 1) return CVATTN_ERR_UNSUPPORTED;
        FaProblem fp;
        fill_problem(fp, &p.q, &p.k, &p.v, has_mask ? &p.mask : nullptr, &p.dst, sh);
        fp.n_splits = ns;
        fp.div_splits = make_fastdiv((uint32_t)ns);
        fp.split_len = sl;
        if (n_kv_dev) {
            fp.n_kv_dev = n_kv_dev + (int64_t)i * n_kv_stride;
            fp.split_unit = sh.ks.wsplit ? sh.ks.tstep * sh.ks.nw : sh.ks.tstep * sh0->ks.kh;
        }
        fp.unit_begin = unit;
        fp.part_begin = part;
        fp.row_begin = row;
        fp.cnt_begin = cnt;
        const int64_t groups = (int64_t)sh.B * sh.H_kv * sh.n_rowgroups;
        unit += groups * ns;
        if (ns > 1) {
            part += slots_per_split(sh) * ns;
            cnt += groups;
        }
        row += (int64_t)sh.B * sh.H * sh.n_q;
        if (table) (*table)[i] = fp;
    }
    lay->table_bytes = align_up(sizeof(FaProblem) * (size_t)n, kAlign);
    lay->counter_bytes = align_up(sizeof(uint32_t) * (size_t)cnt * CNT_STRIDE, kAlign);
    lay->total_bytes = lay->table_bytes + lay->counter_bytes + (size_t)part * PART_STRIDE * sizeof(float);
    // mask tile classes when every problem's mask takes them
    lay->mcls_off = 0;
    lay->mcls_blocks = 0;
    if (has_mask) {
        bool all = true;
        int64_t blocks = 0;
        for (int i = 0; i < n && all; i++) {
            FaShape sh;
            check_fa(&probs[i].q, &probs[i].k, &probs[i].v, &probs[i].mask, &sh);
            sh.ks.kh = sh0->ks.kh;
            const int nkt = mcls_tiles(sh, &probs[i].mask, probs[i].k.type, probs[i].v.type);
            all = nkt > 0;
            if (table) {
                (*table)[i].mcls_ld = nkt;
                (*table)[i].mcls_begin = blocks;
            }
            blocks += (int64_t)sh.n_rowgroups * nkt;
        }
        if (all && blocks > 0) {
            // the classes of every problem, then their prefix lengths (64 per block)
            lay->mcls_off = lay->total_bytes = align_up(lay->total_bytes, kAlign);
            lay->mcls_blocks = blocks;
            lay->total_bytes += (size_t)mcls_table_bytes(blocks);
        } else if (table) {
            for (int i = 0; i < n; i++) (*table)[i].mcls_ld = 0;
        }
    }
    if (unit > kMaxUnits) return CVATTN_ERR_UNSUPPORTED;
    lay->units = unit;
    lay->rows = row;
    return CVATTN_OK;
}

CVATTN_API size_t cvattn_fa_batch_workspace(const cvattn_fa_problem *problems, int n) {
    FaShape sh;
    BatchLayout lay;
    if (plan_batch(problems, n, nullptr, &sh, &lay)) return 0;
    return lay.total_bytes;
}

static int prepare_batch(const cvattn_fa_problem *problems, int n, float scale, const int32_t *n_kv_dev,
                         int n_kv_stride, void *ws, size_t ws_bytes, cvattn_stream_t stream, cvattn_fa_plan *plan) {
    if (!plan || !std::isfinite(scale)) return CVATTN_ERR_BAD_ARGS;
    std::vector<FaProblem> table;
    FaShape sh;
    BatchLayout lay;
    int rc = plan_batch(problems, n, &table, &sh, &lay, n_kv_dev, n_kv_stride);
    if (rc) return rc;
    if (!ws || ws_bytes < lay.total_bytes) return CVATTN_ERR_WORKSPACE_TOO_SMALL;
    if ((uintptr_t)ws & (kAlign - 1)) return CVATTN_ERR_BAD_ARGS; // tables use aligned vector stores
    BatchPlan bp;
    std::memset(&bp, 0, sizeof(bp));
    bp.magic = kPlanMagic;
    bp.ks = sh.ks;
    bp.ktype = problems[0].k.type;
    bp.vtype = problems[0].v.type;
    bp.has_mask = problems[0].mask.data != nullptr;
    fill_uniform(bp.args.u, sh, problems[0].q.type, scale);
    bp.args.u.n_problems = n;
    bp.args.u.total_units = lay.units;
    {
        const int64_t u0 = n > 1 ? table[1].unit_begin - table[0].unit_begin : lay.units;
        bool uniform = u0 > 0;
        for (int i = 0; i < n && uniform; i++) uniform = table[i].unit_begin == (int64_t)i * u0;
        bp.args.u.units_per_problem = uniform && (int64_t)n * u0 == lay.units ? u0 : 0;
        if (bp.args.u.units_per_problem > 0) bp.args.u.div_upp = make_fastdiv((uint32_t)u0);
    }
    bp.args.u.total_rows = lay.rows;
    bp.args.u.counters = (uint32_t *)((char *)ws + lay.table_bytes);
    bp.args.u.partials = (float *)((char *)ws + lay.table_bytes + lay.counter_bytes);
    if (lay.mcls_blocks > 0) {
        for (int i = 0; i < n; i++) {
            table[i].mcls = (uint8_t *)ws + lay.mcls_off + table[i].mcls_begin;
        }
        bp.args.u.mcls_blocks = lay.mcls_blocks;
    }
    bp.args.p0 = table[0];
    bp.args.table = (const FaProblem *)ws;
    fill_dec_pre(bp.args, sh, table.data(), n, problems[0].q.type, bp.has_mask != 0);
    // one upload: the table followed by zeroed counters (the kernels keep them zero afterwards)
    std::vector<unsigned char> head(lay.table_bytes + lay.counter_bytes, 0);
    std::memcpy(head.data(), table.data(), sizeof(FaProblem) * (size_t)n);
    hipError_t e = hipMemcpyAsync(ws, head.data(), head.size(), hipMemcpyHostToDevice, (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream); // `head` must outlive the copy
    if (e != hipSuccess) return CVATTN_ERR_HIP;
    std::memset(plan, 0, sizeof(*plan));
    std::memcpy(plan, &bp, sizeof(bp));
    return CVATTN_OK;
}

CVATTN_API int cvattn_fa_batch_prepare(const cvattn_fa_problem *problems, int n, float scale,
                                       void *ws, size_t ws_bytes, cvattn_stream_t stream,
                                       cvattn_fa_plan *plan) {
    return prepare_batch(problems, n, scale, nullptr, 0, ws, ws_bytes, stream, plan);
}

CVATTN_API int cvattn_fa_batch_prepare_dynamic(const cvattn_fa_problem *problems, int n, float scale,
                                               const int32_t *n_kv_dev, int n_kv_stride, void *ws,
                                               size_t ws_bytes, cvattn_stream_t stream, cvattn_fa_plan *plan) {
    if (!n_kv_dev || (n_kv_stride != 0 && n_kv_stride != 1)) return CVATTN_ERR_BAD_ARGS;
    if (((uintptr_t)n_kv_dev & 3) != 0) return CVATTN_ERR_BAD_ARGS;
    return prepare_batch(problems, n, scale, n_kv_dev, n_kv_stride, ws, ws_bytes, stream, plan);
}

CVATTN_API int cvattn_shift_n_kv(int32_t *n_kv_dev, int n, int32_t delta, cvattn_stream_t stream) {
    if (n < 0 || (n > 0 && !n_kv_dev) || ((uintptr_t)n_kv_dev & 3) != 0) return CVATTN_ERR_BAD_ARGS;
    return hip_status(shift_n_kv_launch(n_kv_dev, n, delta, (hipStream_t)stream));
}

CVATTN_API int cvattn_fa_batch_launch(const cvattn_fa_plan *plan, cvattn_stream_t stream) {
    if (!plan) return CVATTN_ERR_BAD_ARGS;
    BatchPlan bp;
    std::memcpy(&bp, plan, sizeof(bp));
    if (bp.magic != kPlanMagic) return CVATTN_ERR_BAD_ARGS;
    if (bp.args.u.mcls_blocks > 0 && mask_classify_launch(bp.args, true, (hipStream_t)stream) != hipSuccess)
        return CVATTN_ERR_HIP;
    return hip_status(fa_launch(bp.ks, bp.ktype, bp.vtype, bp.has_mask != 0, true, bp.args, (hipStream_t)stream));
}

// ---- formats ------------------------------------------------------------------------------

CVATTN_API int64_t cvattn_block_size(int type) { return is_kv_type(type) ? type_block(type) : 0; }
CVATTN_API int64_t cvattn_type_size(int type) { return is_kv_type(type) ? type_bytes(type) : 0; }

CVATTN_API int cvattn_dequantize(int type, const void *src, float *dst, int64_t n, cvattn_stream_t stream) {
    if (!is_kv_type(type)) return CVATTN_ERR_UNSUPPORTED;
    if (n < 0 || (n > 0 && (!src || !dst))) return CVATTN_ERR_BAD_ARGS;
    if (n % type_block(type)) return CVATTN_ERR_BAD_ARGS;
    return hip_status(dequant_launch(type, src, dst, n, (hipStream_t)stream));
}

// ---- KV write ------------------------------------------------------------------------------

static int check_set_rows(const cvattn_tensor *dst, const cvattn_tensor *src, const cvattn_tensor *idx) {
    if (!dst || !src || !idx) return CVATTN_ERR_BAD_ARGS;
    if (!is_kv_type(dst->type)) return CVATTN_ERR_UNSUPPORTED;
    if (src->type != T_F32 || src->nb[0] != 4) return CVATTN_ERR_UNSUPPORTED;
    if (idx->type != T_I32 && idx->type != 27 /* GGML_TYPE_I64 */) return CVATTN_ERR_UNSUPPORTED;
    if (dst->nb[0] != (size_t)type_bytes(dst->type)) return CVATTN_ERR_UNSUPPORTED;
    if (dst->ne[0] != src->ne[0] || dst->ne[0] % type_block(dst->type)) return CVATTN_ERR_BAD_ARGS;
    if (dst->ne[2] != src->ne[2] || dst->ne[3] != src->ne[3]) return CVATTN_ERR_BAD_ARGS;
    if (idx->ne[0] != src->ne[1]) return CVATTN_ERR_BAD_ARGS;
    if (idx->ne[1] <= 0 || idx->ne[2] <= 0 || src->ne[2] % idx->ne[1] || src->ne[3] % idx->ne[2])
        return CVATTN_ERR_BAD_ARGS;
    for (int i = 0; i < 4; i++)
        if (src->ne[i] < 0 || dst->ne[i] <= 0) return CVATTN_ERR_BAD_ARGS;
    if (src->ne[1] > 0 && (!dst->data || !src->data || !idx->data)) return CVATTN_ERR_BAD_ARGS;
    return CVATTN_OK;
}

CVATTN_API int cvattn_supports_set_rows(const cvattn_tensor *dst, const cvattn_tensor *src,
                                        const cvattn_tensor *idx) {
    return check_set_rows(dst, src, idx) == CVATTN_OK ? 1 : 0;
}

static void fill_set_rows(SetRowsArgs &a, const cvattn_tensor *dst, const cvattn_tensor *src,
                          const cvattn_tensor *idx) {
    std::memset(&a, 0, sizeof(a));
    a.dst = (uint8_t *)dst->data;
    a.src = (const uint8_t *)src->data;
    a.idx = (const uint8_t *)idx->data;
    a.ne0 = src->ne[0];
    a.n_rows = src->ne[1];
    a.ne2 = src->ne[2];
    a.ne3 = src->ne[3];
    a.dst_rows = dst->ne[1];
    a.dst_nb1 = (int64_t)dst->nb[1];
    a.dst_nb2 = (int64_t)dst->nb[2];
    a.dst_nb3 = (int64_t)dst->nb[3];
    a.src_nb1 = (int64_t)src->nb[1];
    a.src_nb2 = (int64_t)src->nb[2];
    a.src_nb3 = (int64_t)src->nb[3];
    a.idx_nb0 = (int64_t)idx->nb[0];
    a.idx_nb1 = (int64_t)idx->nb[1];
    a.idx_nb2 = (int64_t)idx->nb[2];
    a.idx_ne1 = idx->ne[1];
    a.idx_ne2 = idx->ne[2];
    a.idx_i64 = idx->type == 27 ? 1 : 0;
    const int64_t per = type_block(dst->type) == QK ? QK : 1;
    a.total = (src->ne[0] / per) * src->ne[1] * src->ne[2] * src->ne[3];
}

CVATTN_API int cvattn_set_rows(const cvattn_tensor *dst, const cvattn_tensor *src,
                               const cvattn_tensor *idx, cvattn_stream_t stream) {
    int rc = check_set_rows(dst, src, idx);
    if (rc) return rc;
    SetRowsArgs a;
    fill_set_rows(a, dst, src, idx);
    return hip_status(set_rows_launch(dst->type, a, (hipStream_t)stream));
}

// ---- RoPE ------------------------------------------------------------------------------------

// The rope forms cosyvoice.cpp uses (ggml_rope_ext with no frequency factors, ext_factor 0,
// attn_factor 1): NORMAL or NEOX, an even n_dims within the rope input.
static int check_rope_params(int64_t seg, int n_dims, int mode, float freq_base, float freq_scale) {
    if (mode != CVATTN_ROPE_NORMAL && mode != CVATTN_ROPE_NEOX) return CVATTN_ERR_UNSUPPORTED;
    if (seg <= 0 || (seg & 1) || n_dims <= 0 || (n_dims & 1) || n_dims > seg) return CVATTN_ERR_BAD_ARGS;
    if (!(freq_base > 0.0f) || !std::isfinite(freq_base) || !std::isfinite(freq_scale)) return CVATTN_ERR_BAD_ARGS;
    return CVATTN_OK;
}

// ggml's CPU rope takes theta_scale from the C library's powf once per op.
static float rope_theta_scale(float freq_base, int n_dims) { return powf(freq_base, -2.0f / (float)n_dims); }

CVATTN_API int cvattn_rope(const cvattn_tensor *dst, const cvattn_tensor *src, const cvattn_tensor *pos,
                           int n_dims, int mode, float freq_base, float freq_scale, cvattn_stream_t stream) {
    if (!dst || !src || !pos) return CVATTN_ERR_BAD_ARGS;
    if (src->type != T_F32 || dst->type != T_F32 || pos->type != T_I32) return CVATTN_ERR_UNSUPPORTED;
    if (src->nb[0] != 4 || dst->nb[0] != 4 || pos->nb[0] != 4) return CVATTN_ERR_UNSUPPORTED;
    for (int i = 0; i < 4; i++)
        if (src->ne[i] < 0 || dst->ne[i] != src->ne[i]) return CVATTN_ERR_BAD_ARGS;
    int rc = check_rope_params(src->ne[0], n_dims, mode, freq_base, freq_scale);
    if (rc) return rc;
    if (pos->ne[0] != src->ne[2]) return CVATTN_ERR_BAD_ARGS; // ggml_rope_ext: one position per i2
    const int64_t total = src->ne[0] * src->ne[1] * src->ne[2] * src->ne[3];
    if (total > 0 && (!dst->data || !src->data || !pos->data)) return CVATTN_ERR_BAD_ARGS;
    RopeArgs a;
    std::memset(&a, 0, sizeof(a));
    a.dst = (float *)dst->data;
    a.src = (const float *)src->data;
    a.pos = (const int32_t *)pos->data;
    a.ne0 = src->ne[0];
    a.ne1 = src->ne[1];
    a.ne2 = src->ne[2];
    a.ne3 = src->ne[3];
    a.src_nb1 = (int64_t)src->nb[1];
    a.src_nb2 = (int64_t)src->nb[2];
    a.src_nb3 = (int64_t)src->nb[3];
    a.dst_nb1 = (int64_t)dst->nb[1];
    a.dst_nb2 = (int64_t)dst->nb[2];
    a.dst_nb3 = (int64_t)dst->nb[3];
    a.rope_dims = n_dims;
    a.rope_neox = mode == CVATTN_ROPE_NEOX ? 1 : 0;
    a.theta_scale = rope_theta_scale(freq_base, n_dims);
    a.freq_scale = freq_scale;
    a.total = total;
    return hip_status(rope_launch(a, (hipStream_t)stream));
}

CVATTN_API int cvattn_rope_set_rows(const cvattn_tensor *dst, const cvattn_tensor *src, const cvattn_tensor *idx,
                                    const cvattn_tensor *pos, int64_t head, int n_dims, int mode, float freq_base,
                                    float freq_scale, cvattn_stream_t stream) {
    int rc = check_set_rows(dst, src, idx);
    if (rc) return rc;
    if (!pos) return CVATTN_ERR_BAD_ARGS;
    if (pos->type != T_I32) return CVATTN_ERR_UNSUPPORTED;
    rc = check_rope_params(head, n_dims, mode, freq_base, freq_scale);
    if (rc) return rc;
    if (src->ne[0] % head) return CVATTN_ERR_BAD_ARGS;
    // one position per source row, contiguous
    const int64_t n_pos = pos->ne[0] * pos->ne[1] * pos->ne[2] * pos->ne[3];
    if (n_pos != src->ne[1] * src->ne[2] * src->ne[3]) return CVATTN_ERR_BAD_ARGS;
    if (pos->nb[0] != 4 || pos->nb[1] != 4 * (size_t)pos->ne[0] || pos->nb[2] != pos->nb[1] * (size_t)pos->ne[1] ||
        pos->nb[3] != pos->nb[2] * (size_t)pos->ne[2])
        return CVATTN_ERR_UNSUPPORTED;
    if (n_pos > 0 && !pos->data) return CVATTN_ERR_BAD_ARGS;
    SetRowsArgs a;
    fill_set_rows(a, dst, src, idx);
    a.pos = (const int32_t *)pos->data;
    a.rope_seg = head;
    a.rope_dims = n_dims;
    a.rope_neox = mode == CVATTN_ROPE_NEOX ? 1 : 0;
    a.theta_scale = rope_theta_scale(freq_base, n_dims);
    a.freq_scale = freq_scale;
    return hip_status(set_rows_launch(dst->type, a, (hipStream_t)stream));
}

CVATTN_API const char *cvattn_status_string(int status) {
    switch (status) {
    case CVATTN_OK: return "ok";
    case CVATTN_ERR_UNSUPPORTED: return "unsupported";
    case CVATTN_ERR_BAD_ARGS: return "bad arguments";
    case CVATTN_ERR_WORKSPACE_TOO_SMALL: return "workspace too small";
    case CVATTN_ERR_HIP: return "hip error";
    default: return "unknown status";
    }
}

} // extern "C"
