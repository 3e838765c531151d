// fa_dispatch.hip -- picks the flash-attention instantiation for a launch.
#include "fa_decode_inst.h"

namespace cvattn {

static FaLaunchFn fa_pick_decode(int mask, int batch, int ki, int vi) {
    return mask ? fa_pick_decode_m1(batch, ki, vi) : fa_pick_decode_m0(batch, ki, vi);
}
FaLaunchFn fa_pick_rows(int mask, int batch, int ki, int vi);
FaLaunchFn fa_pick_rows_kh2(int mask, int batch, int ki, int vi);
FaLaunchFn fa_pick_rows_vt(int mask, int ki, int vti);
FaLaunchFn fa_pick_rows_cls(int batch, int ktype, int vtype);
FaLaunchFn fa_pick_rows_wide(int batch, int ktype, int vtype);

bool rows_cls_ok(int ktype, int vtype) { return fa_pick_rows_cls(0, ktype, vtype) != nullptr; }

static int type_index(int t) {
    switch (t) {
    case T_F32: return 0;
    case T_F16: return 1;
    case T_Q8_0: return 2;
    case T_Q4_0: return 3;
    case T_Q4_1: return 4;
    case T_Q5_0: return 5;
    case T_Q5_1: return 6;
    default: return -1;
    }
}

FaKernelShape fa_shape(int n_rows, bool decode_ok) {
    FaKernelShape s;
    // decode-shaped kernel (fa_decode.h): <= 64 rows per kv head (up to 4 groups of 16, e.g. the
    // 50 rows of a DiT streaming chunk), unless the caller rules it out (the transposed V of the
    // non-flash-attention path); everything else runs the row-tiled kernel
    s.wsplit = n_rows <= 64 && decode_ok;
    s.nw = 4;
    s.tstep = s.wsplit ? 32 : ROWS_TS;
    s.rows_per_group = s.wsplit ? 16 : ROWS_ROWS;
    s.max_splits = s.wsplit ? DEC_MAX_SPLITS : ROWS_MERGE_MAX_SPLITS;
    s.round_splits = s.wsplit ? DEC_MERGE_CHUNK : ROWS_MERGE_MAX_SPLITS;
    s.long_split = DEC_LONG_SPLIT;
    s.kh = 1;
    return s;
}

hipError_t fa_launch(const FaKernelShape &s, int ktype, int vtype, bool mask, bool batch, const FaArgs &a,
                     hipStream_t st) {
    if (!s.wsplit && s.nw == ROWS_NW_WIDE) {
        const FaLaunchFn fn = mask || s.kh != 1 ? nullptr : fa_pick_rows_wide(batch, ktype, vtype);
        return fn ? fn(a, st) : hipErrorInvalidValue;
    }
    if (mask && !s.wsplit && s.kh == 1 && a.u.mcls_blocks > 0) {
        const FaLaunchFn fn = fa_pick_rows_cls(batch, ktype, vtype);
        return fn ? fn(a, st) : hipErrorInvalidValue;
    }
    const int ki = type_index(ktype), vi = type_index(vtype);
    if (ki < 0 || vi < 0) return hipErrorInvalidValue;
    const FaLaunchFn fn = s.wsplit    ? fa_pick_decode(mask, batch, ki, vi)
                          : s.kh == 2 ? fa_pick_rows_kh2(mask, batch, ki, vi)
                                      : fa_pick_rows(mask, batch, ki, vi);
    return fn(a, st);
}

hipError_t fa_launch_vt(int ktype, int vtype, bool mask, const FaArgs &a, hipStream_t st) {
    const int ki = type_index(ktype);
    const int vti = vtype == T_VT_F32 ? 0 : vtype == T_VT_F16 ? 1 : -1;
    if (ki < 0 || vti < 0) return hipErrorInvalidValue;
    return fa_pick_rows_vt(mask, ki, vti)(a, st);
}

} // namespace cvattn
