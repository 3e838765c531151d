// fa_decode_inst.h -- launchers and dispatch tables of the decode-shaped kernel; each
// dec_*.hip translation unit instantiates one mask family.
#pragma once

#include "fa_decode.h"

namespace cvattn {

template <int KT, int VT, bool MASK, bool BATCH>
hipError_t launch_decode(const FaArgs &a, hipStream_t st) {
    if (a.u.total_units <= 0) return hipSuccess;
    const DecPre &d = a.pre;
    hipLaunchKernelGGL((fa_decode_kernel<KT, VT, MASK, BATCH>), dim3((unsigned)a.u.total_units),
                       dim3(64 * DEC_NW), 0, st, d.k, d.v, d.q, d.k_ps, d.v_ps, d.q_ps, d.kv, d.lens, d.shape,
                       d.units, d.scale_log2, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // single calls merge split partials with a second launch; prepared batches merge in-kernel
    if (!BATCH && a.p0.n_splits > 1) {
        const int64_t groups = (int64_t)a.u.B * a.u.H_kv * a.u.n_rowgroups;
        hipLaunchKernelGGL(dec_combine_kernel, dim3((unsigned)groups), dim3(256), 0, st, a);
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

// The tables live inside host functions so the device pass never sees host pointers.
#define CVATTN_DECODE_PICK(NAME, MASK)                                                               \
    FaLaunchFn NAME(int batch, int ki, int vi) {                                                     \
        static const FaLaunchFn table[2][7][7] = {CVATTN_DTABLE(MASK, false), CVATTN_DTABLE(MASK, true)}; \
        return table[batch][ki][vi];                                                                 \
    }

FaLaunchFn fa_pick_decode_m0(int batch, int ki, int vi);
FaLaunchFn fa_pick_decode_m1(int batch, int ki, int vi);

} // namespace cvattn
