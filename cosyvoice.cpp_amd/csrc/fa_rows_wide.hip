// fa_rows_wide.hip -- the row-tiled flash attention in its wide form: 12 waves x 16 query rows
// per workgroup (one workgroup per CU, 3 waves per SIMD) sharing each staged 64-token K/V tile,
// for unmasked fp16 K/V launches whose 192-row groups still give every CU one (the DiT call).
#include "fa_impl.h"

namespace cvattn {

FaLaunchFn fa_pick_rows_wide(int batch, int ktype, int vtype) {
    if (ktype != T_F16 || vtype != T_F16) return nullptr;
    return batch ? launch_rows<T_F16, T_F16, 0, true, 1, ROWS_NW_WIDE>
                 : launch_rows<T_F16, T_F16, 0, false, 1, ROWS_NW_WIDE>;
}

bool rows_wide_ok(int ktype, int vtype) { return fa_pick_rows_wide(0, ktype, vtype) != nullptr; }

void fa_shape_wide(FaKernelShape &s) {
    s.nw = ROWS_NW_WIDE;
    s.rows_per_group = 16 * ROWS_SETS * ROWS_NW_WIDE;
}

} // namespace cvattn
