// fa_rows_kh2.hip -- instantiates the row-tiled flash attention with two key halves: 8 waves per
// workgroup, waves w and w+4 on the same 16 rows and the two 64-token halves of each 128-token
// step, merged through LDS at the end.  Chosen for launches with fewer row groups than CUs.
#include "fa_impl.h"

namespace cvattn {

// The table lives inside a host function so the device pass never sees host pointers.
FaLaunchFn fa_pick_rows_kh2(int mask, int batch, int ki, int vi) {
    static const FaLaunchFn table[2][2][7][7] = {
        {CVATTN_TABLE(false, false, 2), CVATTN_TABLE(false, true, 2)},
        {CVATTN_TABLE(true, false, 2), CVATTN_TABLE(true, true, 2)},
    };
    return table[mask][batch][ki][vi];
}

} // namespace cvattn
