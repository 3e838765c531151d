// fa_decode.hip -- instantiates the decode-shaped flash attention (fa_decode.h).
#include "fa_decode.h"

namespace cvattn {

template <int KT, int VT, bool MASK, bool BATCH>
hipError_t launch_decode(const FaArgs &a, hipStream_t st) {
    if (a.u.total_units <= 0) return hipSuccess;
    hipLaunchKernelGGL((fa_decode_kernel<KT, VT, MASK, BATCH>), dim3((unsigned)a.u.total_units), dim3(64 * DEC_NW),
                       0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // single calls merge split partials with a second launch; prepared batches merge in-kernel
    if (!BATCH && a.p0.n_splits > 1 && a.u.total_rows > 0) {
        hipLaunchKernelGGL((fa_combine_kernel<16, false>), dim3((unsigned)a.u.total_rows), dim3(64), 0, st, a);
        e = hipGetLastError();
    }
    return e;
}

#define CVATTN_DV_ROW(KT, MASK, BATCH)                                                              \
    {launch_decode<KT, T_F32, MASK, BATCH>, launch_decode<KT, T_F16, MASK, BATCH>,                 \
     launch_decode<KT, T_Q8_0, MASK, BATCH>, launch_decode<KT, T_Q4_0, MASK, BATCH>,               \
     launch_decode<KT, T_Q4_1, MASK, BATCH>, launch_decode<KT, T_Q5_0, MASK, BATCH>,               \
     launch_decode<KT, T_Q5_1, MASK, BATCH>}
#define CVATTN_DTABLE(MASK, BATCH)                                                                   \
    {CVATTN_DV_ROW(T_F32, MASK, BATCH), CVATTN_DV_ROW(T_F16, MASK, BATCH),                         \
     CVATTN_DV_ROW(T_Q8_0, MASK, BATCH), CVATTN_DV_ROW(T_Q4_0, MASK, BATCH),                       \
     CVATTN_DV_ROW(T_Q4_1, MASK, BATCH), CVATTN_DV_ROW(T_Q5_0, MASK, BATCH),                       \
     CVATTN_DV_ROW(T_Q5_1, MASK, BATCH)}

// The table lives inside a host function so the device pass never sees host pointers.
FaLaunchFn fa_pick_decode(int mask, int batch, int ki, int vi) {
    static const FaLaunchFn table[2][2][7][7] = {
        {CVATTN_DTABLE(false, false), CVATTN_DTABLE(false, true)},
        {CVATTN_DTABLE(true, false), CVATTN_DTABLE(true, true)},
    };
    return table[mask][batch][ki][vi];
}

} // namespace cvattn
