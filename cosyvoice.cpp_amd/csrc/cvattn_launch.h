// cvattn_launch.h -- internal launchers implemented in the .hip translation units.
#pragma once

#include <hip/hip_runtime.h>

#include "cvattn_common.h"

namespace cvattn {

// Workgroup shape chosen for a problem: decode-shaped (<= 64 rows per kv head, waves split the
// tokens) or row-tiled (waves split the rows).
struct FaKernelShape {
    bool wsplit;        // decode kernel (fa_decode.h)
    int nw;             // waves per workgroup
    int tstep;          // tokens per staged tile (per wave step for the decode kernel)
    int rows_per_group; // query rows per workgroup
    int max_splits;     // most token splits one workgroup can merge in-kernel
    int round_splits;   // decode: splits per merge round; a second round only when one round's
    int long_split;     //   splits would leave a workgroup more than long_split tokens
    int kh;             // row-tiled: key halves per workgroup (1, or 2 for launches with fewer row
                        // groups than CUs: 8 waves, two per row set, 128-token steps)
};
FaKernelShape fa_shape(int n_rows, bool decode_ok);
hipError_t fa_launch(const FaKernelShape &s, int ktype, int vtype, bool mask, bool batch, const FaArgs &a,
                     hipStream_t st);
// A row-tiled instance for classified mask tiles exists for this K/V type pair.
bool rows_cls_ok(int ktype, int vtype);
// The wide row-tiled form (12 waves, 192 rows per workgroup; unmasked, one key half) exists for
// this K/V type pair; fa_shape_wide turns a row-tiled shape into it.
bool rows_wide_ok(int ktype, int vtype);
void fa_shape_wide(FaKernelShape &s);
// Row-tiled attention over a transposed V (vtype T_VT_F32 / T_VT_F16), single calls.
hipError_t fa_launch_vt(int ktype, int vtype, bool mask, const FaArgs &a, hipStream_t st);

hipError_t dequant_launch(int type, const void *src, float *dst, int64_t n, hipStream_t st);
// Mask tile classes of the launch described by `a` (a.u.mcls_blocks blocks; problems' mcls set).
hipError_t mask_classify_launch(const FaArgs &a, bool batch, hipStream_t st);

// fp32 -> fp16 copy (round to nearest even, the conversion the attention kernels apply when
// they stage fp32 K/V) of a strided 4-d view [ne0, ne1, ne2, ne3] into dense rows of dst_row
// halfs (a multiple of 8; the pad of a row is written as zeros).  total < 2^31: the kernel
// indexes with 32-bit fast divisions.
struct CvtF16Args {
    const uint8_t *src;
    _Float16 *dst;
    int64_t ne0, ne1, ne2;
    int64_t nb1, nb2, nb3;
    int64_t dst_row;
    int64_t chunks;   // dst_row / 8: one thread per 8 halfs of a row
    int64_t total;    // rows * chunks
    FastDiv div_chunks, div_ne1, div_ne2;   // filled by cvt_f16_launch
};
constexpr int64_t kCvtMaxChunks = INT32_MAX;
// Copies n (1 or 2) views in one launch: the K and V copies of one attention call.
hipError_t cvt_f16_launch(CvtF16Args *a, int n, hipStream_t st);

struct SetRowsArgs {
    uint8_t *dst;
    const uint8_t *src;
    const uint8_t *idx;
    int64_t ne0, n_rows, ne2, ne3;
    int64_t dst_rows;
    int64_t dst_nb1, dst_nb2, dst_nb3;
    int64_t src_nb1, src_nb2, src_nb3;
    int64_t idx_nb0, idx_nb1, idx_nb2;
    int64_t idx_ne1, idx_ne2;
    int32_t idx_i64;
    int64_t total;
    // RoPE in front of the write (rope_dims = 0: plain set_rows)
    const int32_t *pos;   // one position per source row, flattened (i1, i2, i3)
    int64_t rope_seg;     // elements per rope input (head)
    int32_t rope_dims;    // rotated dims per input (even, <= rope_seg)
    int32_t rope_neox;    // pairing: (k, k + dims/2) instead of (2k, 2k+1)
    float theta_scale;    // powf(freq_base, -2/dims), taken on the host
    float freq_scale;
};
hipError_t set_rows_launch(int type, const SetRowsArgs &a, hipStream_t st);

// ggml_rope_ext on f32 tensors [ne0, ne1, ne2, ne3], position pos[i2].
struct RopeArgs {
    float *dst;
    const float *src;
    const int32_t *pos;
    int64_t ne0, ne1, ne2, ne3;
    int64_t src_nb1, src_nb2, src_nb3;
    int64_t dst_nb1, dst_nb2, dst_nb3;
    int32_t rope_dims, rope_neox;
    float theta_scale, freq_scale;
    int64_t total; // ne0 * ne1 * ne2 * ne3
};
hipError_t rope_launch(const RopeArgs &a, hipStream_t st);

// DiT step inputs built on the device.
constexpr int kMaxChunkBounds = 256;
struct ChunkMaskArgs {
    uint8_t *mask;    // f16 rows of n_cols, nb1 bytes apart
    int64_t nb1;
    int32_t n_rows, n_cols, n_bounds;
    uint32_t bounds[kMaxChunkBounds];
};
hipError_t chunk_mask_launch(const ChunkMaskArgs &a, hipStream_t st);
hipError_t fill_positions_launch(int32_t *pos, int64_t n, int64_t batch, int64_t nb1, int32_t base, hipStream_t st);
hipError_t shift_n_kv_launch(int32_t *n_kv, int32_t n, int32_t delta, hipStream_t st);
hipError_t v_idxs_launch(int32_t *idx, const int32_t *pos, uint32_t n_tokens, uint32_t n_per_batch, uint32_t n_embd,
                         uint32_t max_seq, hipStream_t st);

} // namespace cvattn
