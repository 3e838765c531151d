// fa_rows.hip -- instantiates the row-tiled flash attention for prefill and DiT: 4 waves x 16
// query rows per workgroup sharing double-buffered 64-token K/V tiles (one key half).
#include "fa_impl.h"

namespace cvattn {

// The table lives inside a host function so the device pass never sees host pointers.
FaLaunchFn fa_pick_rows(int mask, int batch, int ki, int vi) {
    static const FaLaunchFn table[2][2][7][7] = {
        {CVATTN_TABLE(false, false, 1), CVATTN_TABLE(false, true, 1)},
        {CVATTN_TABLE(true, false, 1), CVATTN_TABLE(true, true, 1)},
    };
    return table[mask][batch][ki][vi];
}

} // namespace cvattn
