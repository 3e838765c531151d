// cvattn_common.h -- types shared by the host dispatcher and the gfx950 kernels.
//
// Block formats are ggml's (ggml-common.h), as cosyvoice.cpp stores them in its KV cache
// (src/cosyvoice-kv-cache.cpp:104-119, types chosen at src/cosyvoice-loader.cpp:468-510):
//   q8_0 {f16 d; i8 qs[32]}                   34 B   x = qs*d
//   q4_0 {f16 d; u8 qs[16]}                   18 B   x = (nib-8)*d
//   q4_1 {f16 d; f16 m; u8 qs[16]}            20 B   x = nib*d + m
//   q5_0 {f16 d; u8 qh[4]; u8 qs[16]}         22 B   x = (nib|hb<<4 - 16)*d
//   q5_1 {f16 d; f16 m; u8 qh[4]; u8 qs[16]}  24 B   x = (nib|hb<<4)*d + m
// Element j<16 of a 4/5-bit block is the low nibble of qs[j], element j+16 the high nibble;
// its 5th bit is bit j (resp. j+16) of qh.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace cvattn {

enum : int {
    T_F32 = 0,
    T_F16 = 1,
    T_Q4_0 = 2,
    T_Q4_1 = 3,
    T_Q5_0 = 6,
    T_Q5_1 = 7,
    T_Q8_0 = 8,
    T_I32 = 26,
};

constexpr int QK = 32;   // elements per quantized block
constexpr int HEAD = 64; // D = Dv handled by the attention kernels

__host__ __device__ constexpr int type_block(int t) {
    return (t == T_F32 || t == T_F16) ? 1
           : (t == T_Q4_0 || t == T_Q4_1 || t == T_Q5_0 || t == T_Q5_1 || t == T_Q8_0) ? QK
                                                                                     : 0;
}
__host__ __device__ constexpr int type_bytes(int t) {
    return t == T_F32 ? 4 : t == T_F16 ? 2 : t == T_Q4_0 ? 18 : t == T_Q4_1 ? 20
         : t == T_Q5_0 ? 22 : t == T_Q5_1 ? 24 : t == T_Q8_0 ? 34 : 0;
}
// Codes are staged as fp16 "1024 + u" (u the unsigned code); the true code is u - code_off.
__host__ __device__ constexpr int code_off(int t) {
    return t == T_Q8_0 ? 128 : t == T_Q4_0 ? 8 : t == T_Q5_0 ? 16 : 0;
}
__host__ __device__ constexpr bool has_min(int t) { return t == T_Q4_1 || t == T_Q5_1; }
__host__ __device__ constexpr bool is_quant(int t) { return type_block(t) == QK; }

// V held transposed -- [n_kv, Dv] per head with the tokens contiguous, the V cache of the
// non-flash-attention path (src/cosyvoice-kv-cache.cpp:104-108,338-345) -- in f32 or f16.
// Kernel tags only, never ggml type codes.
constexpr int T_VT_F32 = 64, T_VT_F16 = 65;
__host__ __device__ constexpr bool is_vt(int t) { return t == T_VT_F32 || t == T_VT_F16; }

// Division by a runtime constant d >= 1 for 0 <= n < 2^31: q = (n * mul) >> shift with
// shift = 31 + ceil(log2 d) and mul = ceil(2^shift / d) < 2^32 (round-up method; the error term
// n*(mul*d - 2^shift) / (d*2^shift) < 1/d never carries the quotient over).  Workgroup indices
// are decomposed with these on the scalar unit instead of 64-bit division routines.
struct FastDiv {
    uint32_t mul, shift, d;
};
inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while (l < 31 && (1u << l) < d) l++;
    const uint32_t shift = 31 + l;
    const uint64_t mul = (((uint64_t)1 << shift) + d - 1) / d;
    return FastDiv{(uint32_t)mul, shift, d};
}
__host__ __device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) {
    return (uint32_t)(((uint64_t)n * f.mul) >> f.shift);
}

// One attention problem as the kernels see it (strides in bytes; nb0 is implied by the type).
struct FaProblem {
    const void *q;
    const void *k;
    const void *v;
    const void *mask; // f16 or nullptr
    float *dst;       // f32 contiguous [Dv, H, n_q, B]
    int64_t q_nb1, q_nb2, q_nb3;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t v_nb1, v_nb2, v_nb3;
    int64_t m_nb1, m_nb2, m_nb3;
    int32_t m_ne2, m_ne3;
    int32_t n_kv;
    int32_t n_splits;
    int32_t split_len;    // tokens per split (multiple of the kernel's token step)
    int32_t rk3, rv3;     // B / B_k, B / B_v
    int32_t v_align2;     // transposed V whose rows are only 2-byte aligned (odd max_seq, f16)
    int64_t unit_begin;   // first workgroup unit of this problem in the launch
    int64_t part_begin;   // first partial slot (rows) of this problem in the workspace
    int64_t row_begin;    // first output row (b, i, h) of this problem (combine indexing)
    int64_t cnt_begin;    // first split-arrival counter of this problem (prepared batches)
    FastDiv div_splits;   // n_splits
    // Plans prepared with a device-resident n_kv (cvattn_fa_batch_prepare_dynamic): each launch
    // reads n_kv here, n_kv above holds the capacity the plan was made for, and the launch spreads
    // the tokens over the planned splits in runs of a multiple of split_unit tokens.
    const int32_t *n_kv_dev;
    int32_t split_unit;
    // Mask tile classes (row-tiled kernel, masks shared by every head and sequence): byte
    // [rg * mcls_ld + kt] tells whether the mask over row group rg's query rows and keys
    // 64*kt .. 64*kt+63 is all zero (MCLS_ZERO), all -inf (MCLS_OFF), zero up to a per-row key
    // and -inf after it (MCLS_PREFIX) or none of these (MCLS_MIXED);
    // nullptr when the launch does not classify.  mcls_begin: the problem's first block in the
    // classifying launch.
    uint8_t *mcls;
    int32_t mcls_ld;
    int64_t mcls_begin;
};
// The classes of a launch's blocks (padded to 64 bytes) are followed by 64 bytes per block: for
// an MCLS_PREFIX block, the visible-prefix length of each of its query rows (row q0+i of the
// block at byte i), where q0 is the block's first query row.  mcls_blocks: the blocks of the
// whole launch.  The whole table takes mcls_table_bytes(mcls_blocks) from a 64-aligned base.
__host__ __device__ inline int64_t mcls_table_bytes(int64_t mcls_blocks) { return (mcls_blocks + 63) / 64 * 64 + 64 * mcls_blocks; }
__host__ __device__ inline uint8_t *mcls_bounds(const FaProblem &p, int64_t mcls_blocks, int64_t block) {
    return p.mcls - p.mcls_begin + (mcls_blocks + 63) / 64 * 64 + (p.mcls_begin + block) * 64;
}
// MCLS_PREFIX: every query row of the block is 0 up to some key and -inf from there on (the
// edges of causal and chunk masks); the kernel then masks with the row's prefix length.
constexpr int MCLS_ZERO = 0, MCLS_OFF = 1, MCLS_MIXED = 2, MCLS_PREFIX = 3;
constexpr int ROWS_TILE = 64;       // keys per tile of the row-tiled kernel (the class granularity)
constexpr int MCLS_MAX_TILES = 64; // key tiles a classified row group may have (n_kv <= 4096)

// Parameters shared by every problem of one launch.
struct FaUniform {
    int32_t n_q, H, H_kv, G, B;
    int32_t n_rows;      // n_q * G rows per (batch, kv head)
    int32_t n_rowgroups; // ceil(n_rows / rows per workgroup)
    int32_t q_f16;       // Q element type: 0 f32, 1 f16
    int32_t n_problems;
    float scale;         // softmax scale
    float scale_log2;    // scale * log2(e)
    float empty_row;     // output of a row whose keys are all masked: 0 (flash attention), or
                         // NaN as ggml's soft_max gives it (the non-flash-attention path)
    FastDiv div_hkv, div_rowgroups, div_upp; // H_kv, n_rowgroups, units_per_problem
    int64_t units_per_problem; // > 0 when every problem has this many workgroup units
    int64_t total_units;
    int64_t total_rows;  // sum over problems of B*H*n_q (combine grid)
    int64_t mcls_blocks; // mask tile classes to compute before the attention launch (0: none)
    float *partials;     // workspace: split partial (m, l, O[64]) per row slot
    uint32_t *counters;  // prepared batches: split-arrival counter per (problem, b, kh, row group),
                         // CNT_STRIDE words apart, zero between launches (the merging workgroup
                         // resets its counter)
};

constexpr int PART_STRIDE = 68; // floats per partial slot: O[64], m, l, pad
// Split-arrival counters sit one per 128-byte line: a group's splits increment theirs at about the
// same time, and counters sharing a line serialize each other's atomics (one line per counter took
// the 24-layer decode step from 14.6 to 14.0 us and the 16-sequence serving step from 390 to 362 us).
constexpr int CNT_STRIDE = 32; // uint32 words

// What a decode workgroup needs to address its K/V and Q loads, for launches whose problems are
// laid out at uniform strides (the layers of one cache buffer, or a single problem) with one
// sequence, one query token and one row group per kv head, no mask and f32 Q with contiguous
// heads.  The decode kernel takes these 14 dwords as its leading arguments, which the dispatcher
// preloads into scalar registers: a workgroup issues its loads and converts its Q without first
// reading its kernel arguments or a problem table from memory, which, once the other workgroups'
// K/V requests fill the memory queues, waits behind them.  G == 0: the kernel locates its problem
// as before.
struct DecPre {
    const uint8_t *k, *v, *q;  // problem 0: K and V rows of kv head 0, the Q rows
    int32_t k_ps, v_ps, q_ps;  // byte stride from one problem to the next
    uint32_t kv;               // n_kv | n_splits << 24
    uint32_t lens;             // split_len | K row bytes << 16 (kv head h at h * row / H_kv)
    uint32_t shape;            // V row bytes | H_kv << 16 | G << 24 (G = 0: not preloaded)
    uint32_t units;            // workgroups of the launch
    float scale_log2;          // softmax scale * log2(e)
};

struct FaArgs {
    FaUniform u;
    FaProblem p0;              // used when n_problems == 1
    const FaProblem *table;    // device table when n_problems > 1
    DecPre pre;                // decode launches: the preloaded addressing (pre.shape G field set)
    int64_t dst_ps;            // with pre: float stride from one problem's output to the next
};

} // namespace cvattn
