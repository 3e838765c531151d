// kv_blocks.h -- whole ggml blocks (32 consecutive dims of a K/V head row) moved through
// registers: 16-byte buffer loads of a block, and its unpacking into fp16 rows of an LDS tile
// plus fp32 block scales.  Shared by the decode and row-tiled attention kernels.
#pragma once

#include "cvattn_device.h"

namespace cvattn {

typedef short short4_t __attribute__((ext_vector_type(4)));

// Buffer resource over [base, base + bytes); loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(gu8 *base, int64_t bytes) {
    const int32_t n = bytes > 0x7fffffff ? 0x7fffffff : (int32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, n, 0x00020000);
}
__device__ __forceinline__ uint32_t bld_u16(__amdgpu_buffer_rsrc_t r, int v, int s) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, v, s, 0);
}
__device__ __forceinline__ uint32_t bld_u32(__amdgpu_buffer_rsrc_t r, int v, int s) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, v, s, 0);
}
__device__ __forceinline__ u4 bld_u128(__amdgpu_buffer_rsrc_t r, int v, int s) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, v, s, 0);
}

// ---- whole 32-dim blocks in registers ------------------------------------------------------

template <int T>
__host__ __device__ constexpr int blk_words() {
    return T == T_F32 || T == T_VT_F32 ? 32 : T == T_F16 || T == T_VT_F16 ? 16 : T == T_Q8_0 ? 8 : 4;
}
// bytes of 32 consecutive dims of a head row
template <int T>
__host__ __device__ constexpr int dblk_bytes() {
    return T == T_F32 ? 128 : T == T_F16 ? 64 : type_bytes(T);
}
// Registers of one block: W >= blk_words<T>() words so one buffer can hold either tensor's block.
template <int W>
struct RawBuf {
    uint32_t w[W];   // codes (quantized) or values (f16/f32)
    uint32_t dm;     // fp16 bits of d (low half) and m (high half)
    uint32_t qh;     // 5th bits (q5_0/q5_1)
};

// Issue the loads of the 32-dim block at byte offset voff + soff of the resource.
template <int T, int W>
__device__ __forceinline__ void blk_load(__amdgpu_buffer_rsrc_t rs, int voff, int soff, RawBuf<W> &r) {
    static_assert(W >= blk_words<T>(), "block buffer too small");
    r.dm = 0u;
    r.qh = 0u;
    constexpr int nq = T == T_F32 ? 8 : T == T_F16 ? 4 : T == T_Q8_0 ? 2 : 1;
    constexpr int qoff = T == T_Q8_0 ? 2 : T == T_Q4_0 ? 2 : T == T_Q4_1 ? 4 : T == T_Q5_0 ? 6 : T == T_Q5_1 ? 8 : 0;
    if constexpr (is_quant(T)) r.dm = has_min(T) ? bld_u32(rs, voff, soff) : bld_u16(rs, voff, soff);
    if constexpr (T == T_Q5_0 || T == T_Q5_1) r.qh = bld_u32(rs, voff + (T == T_Q5_0 ? 2 : 4), soff);
#pragma unroll
    for (int i = 0; i < nq; i++) {
        const u4 a = bld_u128(rs, voff + qoff + 16 * i, soff);
        r.w[4 * i + 0] = a[0];
        r.w[4 * i + 1] = a[1];
        r.w[4 * i + 2] = a[2];
        r.w[4 * i + 3] = a[3];
    }
}

// The Raw8 view (dims 8c..8c+7) of a whole block, for the shared unpackers.
template <int T, int W>
__device__ __forceinline__ Raw8<T> blk_sub(const RawBuf<W> &r, int c) {
    Raw8<T> s;
    s.dm = r.dm;
    if constexpr (T == T_F32) {
#pragma unroll
        for (int i = 0; i < 8; i++) s.w[i] = r.w[8 * c + i];
    } else if constexpr (T == T_F16) {
#pragma unroll
        for (int i = 0; i < 4; i++) s.w[i] = r.w[4 * c + i];
    } else if constexpr (T == T_Q8_0) {
        s.w[0] = r.w[2 * c];
        s.w[1] = r.w[2 * c + 1];
    } else {
        s.w[0] = r.w[2 * (c & 1)];
        s.w[1] = r.w[2 * (c & 1) + 1];
        if constexpr (T == T_Q5_0 || T == T_Q5_1) s.w[2] = r.qh;
    }
    return s;
}

// Unpack a block into 32 fp16 of an LDS row (dims 32b..32b+31 at `dst`).  EXACT: V codes are
// turned into the true small integers (u - code_off) with an exact fp16 subtraction; K keeps
// "1024 + u" (its offset is folded into the score accumulator).
template <int T, bool EXACT, int W>
__device__ __forceinline__ void blk_stage(const RawBuf<W> &r, _Float16 *dst) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
        uint32_t o[4];
        raw8_unpack<T>(blk_sub<T, W>(r, c), c, o);
        if constexpr (EXACT && is_quant(T)) {
            const _Float16 nb = (_Float16)(-(float)(1024 + code_off(T)));
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] = __builtin_bit_cast(uint32_t, as_h2(o[i]) + h2{nb, nb});
        }
        *(u4 *)(dst + 8 * c) = u4{o[0], o[1], o[2], o[3]};
    }
}

template <int T, int W>
__device__ __forceinline__ void blk_scales(const RawBuf<W> &r, float &d, float &m) {
    Raw8<T> s;
    s.dm = r.dm;
    raw8_scales<T>(s, d, m);
}

} // namespace cvattn
