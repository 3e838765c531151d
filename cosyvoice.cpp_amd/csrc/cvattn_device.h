// cvattn_device.h -- gfx950 device helpers: unaligned loads, block-format unpacking into fp16
// MFMA operands, wave reductions.  Used by every kernel so the dequantizer test entry
// (cvattn_dequantize) exercises the exact unpacking the attention kernels run.
#pragma once

#include <hip/hip_runtime.h>

#include "cvattn_common.h"

namespace cvattn {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

// Reinterpret a 32-bit word.  The argument is taken by value: with the ROCm 7.2 compiler,
// __builtin_bit_cast applied directly to an ext_vector element (v[i], i > 0) read element 0.
__device__ __forceinline__ h2 as_h2(uint32_t x) { return __builtin_bit_cast(h2, x); }
__device__ __forceinline__ float as_f32(uint32_t x) { return __builtin_bit_cast(float, x); }
__device__ __forceinline__ h8 as_h8(u4 x) { return __builtin_bit_cast(h8, x); }
__device__ __forceinline__ uint32_t as_u32(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ u4 as_u4(f4 x) { return __builtin_bit_cast(u4, x); }
__device__ __forceinline__ f4 as_f4(u4 x) { return __builtin_bit_cast(f4, x); }

// Device memory is read through address-space-1 pointers so the compiler emits global (not
// flat) loads; flat loads would make every LDS wait also wait for outstanding memory reads.
typedef const __attribute__((address_space(1))) uint8_t gu8;
__device__ __forceinline__ gu8 *gptr(const void *p) { return (gu8 *)p; }

// Little-endian loads at any byte alignment (gfx950 global loads accept unaligned addresses).
__device__ __forceinline__ uint32_t ldg_u32(gu8 *p) {
    uint32_t v;
    __builtin_memcpy(&v, (const __attribute__((address_space(1))) void *)p, 4);
    return v;
}
// 8- and 16-byte loads are typed loads through byte-aligned vector types.  (Copying into a
// vector local with __builtin_memcpy was miscompiled by the ROCm 7.2 compiler in some kernels:
// only the first lane of the loaded vector survived.)
typedef u2 u2_a1 __attribute__((aligned(1)));
typedef u4 u4_a1 __attribute__((aligned(1)));
__device__ __forceinline__ u2 ldg_u64(gu8 *p) { return *(const __attribute__((address_space(1))) u2_a1 *)p; }
__device__ __forceinline__ u4 ldg_u128(gu8 *p) { return *(const __attribute__((address_space(1))) u4_a1 *)p; }
__device__ __forceinline__ float ldg_half(gu8 *p) {
    _Float16 v;
    __builtin_memcpy(&v, (const __attribute__((address_space(1))) void *)p, 2);
    return (float)v;
}

// byte_perm(hi, lo, sel): result byte i = byte sel_i of the 8-byte value {hi:lo} (lo = bytes 0-3).
__device__ __forceinline__ uint32_t byte_perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// Bytes u0..u3 of w -> fp16 pairs (1024+u0, 1024+u1), (1024+u2, 1024+u3).  fp16 0x64XX is
// exactly 1024 + XX because the ulp of fp16 on [1024, 2048) is 1.
__device__ __forceinline__ void bytes_to_h1024(uint32_t w, uint32_t &a, uint32_t &b) {
    a = byte_perm(0x64646464u, w, 0x04010400u);
    b = byte_perm(0x64646464u, w, 0x04030402u);
}

// 4 bits -> one bit per byte (bit k -> bit 4 of byte k), used for the q5 high bits.
__device__ __forceinline__ uint32_t spread4_hi(uint32_t x) {
    return (((x & 0xfu) * 0x00204081u) & 0x01010101u) << 4;
}

// Raw words of dims [32*b + 8*c, +8) of one head row, sized for the type so prefetched tiles
// cost only the registers they need.  Loads only fill integer registers; every conversion
// happens in raw8_unpack/raw8_scales so prefetched tiles do not force a wait.
template <int T>
__host__ __device__ constexpr int raw_words() {
    return T == T_F32 ? 8 : T == T_F16 ? 4 : (T == T_Q5_0 || T == T_Q5_1) ? 3 : 2;
}
template <int T>
struct Raw8 {
    uint32_t w[raw_words<T>()];
    uint32_t dm; // quantized: fp16 bits of d (low half) and m (high half)
};

__device__ __forceinline__ uint32_t ldg_u16(gu8 *p) {
    uint16_t v;
    __builtin_memcpy(&v, (const __attribute__((address_space(1))) void *)p, 2);
    return v;
}

// Issue the loads for dims [32*b + 8*c, +8) of a head row starting at `row`.
template <int T>
__device__ __forceinline__ void raw8_load(gu8 *row, int b, int c, Raw8<T> &r) {
    r.dm = 0u;
    if constexpr (T == T_F32) {
        const u4 a = ldg_u128(row + (32 * b + 8 * c) * 4);
        const u4 e = ldg_u128(row + (32 * b + 8 * c) * 4 + 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            r.w[i] = a[i];
            r.w[4 + i] = e[i];
        }
    } else if constexpr (T == T_F16) {
        const u4 a = ldg_u128(row + (32 * b + 8 * c) * 2);
#pragma unroll
        for (int i = 0; i < 4; i++) r.w[i] = a[i];
    } else {
        gu8 *blk = row + b * type_bytes(T);
        if constexpr (has_min(T))
            r.dm = ldg_u32(blk); // d and m are adjacent
        else
            r.dm = ldg_u16(blk);
        constexpr int qs_off = T == T_Q8_0 ? 2 : T == T_Q4_0 ? 2 : T == T_Q4_1 ? 4 : T == T_Q5_0 ? 6 : 8;
        const u2 q = ldg_u64(blk + qs_off + (T == T_Q8_0 ? 8 * c : 8 * (c & 1)));
        r.w[0] = q[0];
        r.w[1] = q[1];
        if constexpr (T == T_Q5_0 || T == T_Q5_1) r.w[2] = ldg_u32(blk + (T == T_Q5_0 ? 2 : 4));
    }
}

// Block scale d and min m of the loaded block (1 and 0 for f16/f32).
template <int T>
__device__ __forceinline__ void raw8_scales(const Raw8<T> &r, float &d, float &m) {
    if constexpr (is_quant(T)) {
        const h2 h = as_h2(r.dm);
        d = (float)h[0];
        m = has_min(T) ? (float)h[1] : 0.0f;
    } else {
        d = 1.0f;
        m = 0.0f;
    }
}

// Unpack to 8 fp16 in natural dim order (4 dwords).  Quantized types give 1024 + u where u is
// the unsigned code (true code = u - code_off(T)); f16 gives the values, f32 rounds to fp16.
template <int T>
__device__ __forceinline__ void raw8_unpack(const Raw8<T> &r, int c, uint32_t o[4]) {
    if constexpr (T == T_F32) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            h2 h = {(_Float16)as_f32(r.w[2 * i]), (_Float16)as_f32(r.w[2 * i + 1])};
            o[i] = __builtin_bit_cast(uint32_t, h);
        }
    } else if constexpr (T == T_F16) {
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = r.w[i];
    } else if constexpr (T == T_Q8_0) {
        bytes_to_h1024(r.w[0] ^ 0x80808080u, o[0], o[1]);
        bytes_to_h1024(r.w[1] ^ 0x80808080u, o[2], o[3]);
    } else {
        uint32_t w0 = r.w[0], w1 = r.w[1];
        if (c >= 2) {
            w0 >>= 4;
            w1 >>= 4;
        }
        w0 &= 0x0f0f0f0fu;
        w1 &= 0x0f0f0f0fu;
        if constexpr (T == T_Q5_0 || T == T_Q5_1) {
            const uint32_t bits = r.w[2] >> (8 * (c & 1) + 16 * (c >> 1));
            w0 |= spread4_hi(bits);
            w1 |= spread4_hi(bits >> 4);
        }
        bytes_to_h1024(w0, o[0], o[1]);
        bytes_to_h1024(w1, o[2], o[3]);
    }
}

// Offset that turns the staged fp16 into the true code (exact in fp16).
template <int T>
__device__ __forceinline__ constexpr float stage_bias() {
    return is_quant(T) ? (float)(1024 + code_off(T)) : 0.0f;
}

// Reductions over the four lanes l, l^16, l^32, l^48 that share a row (MFMA column).  They stay
// in the VALU: v_permlane32_swap exchanges the wave halves of two registers and
// v_permlane16_swap the odd rows of one with the even rows of the other, so with both operands
// holding v each lane ends with its own value and its partner's (no LDS round trip).
__device__ __forceinline__ float wave_max16x4(float v) {
    const uint32_t u = as_u32(v);
    const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = fmaxf(as_f32(a[0]), as_f32(a[1]));
    const uint32_t w = as_u32(v);
    const auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    return fmaxf(as_f32(b[0]), as_f32(b[1]));
}
__device__ __forceinline__ float wave_sum16x4(float v) {
    const uint32_t u = as_u32(v);
    const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = as_f32(a[0]) + as_f32(a[1]);
    const uint32_t w = as_u32(v);
    const auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    return as_f32(b[0]) + as_f32(b[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Device-coherent (agent scope) stores/loads for data one workgroup hands to another.  On
// gfx950 each XCD has its own L2; these go through to the coherent level (sc1) without the
// whole-L2 write-back/invalidate a device-scope fence costs.
__device__ __forceinline__ void st_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every memory operation this thread issued has completed.
__device__ __forceinline__ void wait_memory() { __builtin_amdgcn_s_waitcnt(0); }

// Workgroup -> unit with consecutive units on one XCD (workgroups are dealt round-robin over
// the 8 XCDs, so ids w and w+8 share an L2).
__device__ __forceinline__ uint32_t xcd_unit(uint32_t w, uint32_t n) {
    const uint32_t x = w & 7, i = w >> 3, q = n >> 3, r = n & 7;
    return x * q + (x < r ? x : r) + i;
}

} // namespace cvattn
