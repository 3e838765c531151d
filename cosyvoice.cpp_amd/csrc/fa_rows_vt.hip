// fa_rows_vt.hip -- instantiates the row-tiled attention over a transposed V cache ([n_kv, Dv]
// per head, f32 or f16): the non-flash-attention path of src/cosyvoice-kv-cache.cpp:387-395 and
// src/cosyvoice-graph.cpp:378-388 served by the same kernel (single calls only).
#include "fa_impl.h"

namespace cvattn {

#define CVATTN_VT_ROW(KT, MASK) {launch_rows<KT, T_VT_F32, MASK, false>, launch_rows<KT, T_VT_F16, MASK, false>}
#define CVATTN_VT_TABLE(MASK)                                                                          \
    {CVATTN_VT_ROW(T_F32, MASK), CVATTN_VT_ROW(T_F16, MASK), CVATTN_VT_ROW(T_Q8_0, MASK),            \
     CVATTN_VT_ROW(T_Q4_0, MASK), CVATTN_VT_ROW(T_Q4_1, MASK), CVATTN_VT_ROW(T_Q5_0, MASK),           \
     CVATTN_VT_ROW(T_Q5_1, MASK)}

// The table lives inside a host function so the device pass never sees host pointers.
FaLaunchFn fa_pick_rows_vt(int mask, int ki, int vti) {
    static const FaLaunchFn table[2][7][2] = {CVATTN_VT_TABLE(false), CVATTN_VT_TABLE(true)};
    return table[mask][ki][vti];
}

} // namespace cvattn
