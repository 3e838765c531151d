// fa_rows_cls.hip -- the row-tiled flash attention with classified mask tiles (one key half):
// launches whose mask is shared by every head and sequence and was classified per 64-row group
// and 64-key tile before the launch (the DiT call with a chunk mask, long causal prefills).
#include "fa_impl.h"

namespace cvattn {

// The K/V type pairs it is built for; others run the mask-word instance unclassified.
FaLaunchFn fa_pick_rows_cls(int batch, int ktype, int vtype) {
#define CVATTN_CLS(KT, VT)                                                                         \
    if (ktype == KT && vtype == VT) return batch ? launch_rows<KT, VT, 2, true> : launch_rows<KT, VT, 2, false>;
    CVATTN_CLS(T_F16, T_F16)
    CVATTN_CLS(T_Q8_0, T_Q8_0)
    CVATTN_CLS(T_Q8_0, T_Q4_0)
    CVATTN_CLS(T_F16, T_Q8_0)
#undef CVATTN_CLS
    return nullptr;
}

} // namespace cvattn
