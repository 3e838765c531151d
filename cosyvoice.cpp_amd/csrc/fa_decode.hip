// fa_decode.hip -- instantiates the decode-shaped flash attention: at most 16 query rows per kv
// head (GQA decode, a few query tokens), 4 waves per workgroup splitting the token range.
#include "fa_impl.h"

namespace cvattn {

// The table lives inside a host function so the device pass never sees host pointers.
FaLaunchFn fa_pick_decode(int mask, int batch, int ki, int vi) {
    static const FaLaunchFn table[2][2][7][7] = {
        {CVATTN_TABLE(4, true, false, false), CVATTN_TABLE(4, true, false, true)},
        {CVATTN_TABLE(4, true, true, false), CVATTN_TABLE(4, true, true, true)},
    };
    return table[mask][batch][ki][vi];
}

} // namespace cvattn
