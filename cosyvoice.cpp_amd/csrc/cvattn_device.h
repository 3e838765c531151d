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

__device__ __forceinline__ uint32_t ldg_u32(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}
__device__ __forceinline__ uint32_t ldg_u16(const uint8_t *p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}
__device__ __forceinline__ float ldg_half(const uint8_t *p) {
    _Float16 v;
    __builtin_memcpy(&v, p, 2);
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

// Raw bytes of dims [32*b + 8*c, +8) of one head row, enough to finish unpacking later.
struct Raw8 {
    uint32_t w[8]; // f32: 8 words; f16: 4 words; quantized: codes in w[0..1], hi bits in w[2]
    float d, m;
};

// Issue the loads for dims [32*b + 8*c, +8) of a head row starting at `row`.
template <int T>
__device__ __forceinline__ void raw8_load(const uint8_t *row, int b, int c, Raw8 &r) {
    // every field is defined on every path so the struct stays in registers
#pragma unroll
    for (int i = 0; i < 8; i++) r.w[i] = 0u;
    if constexpr (T == T_F32) {
        const uint8_t *p = row + (32 * b + 8 * c) * 4;
#pragma unroll
        for (int i = 0; i < 8; i++) r.w[i] = ldg_u32(p + 4 * i);
        r.d = 1.0f;
        r.m = 0.0f;
    } else if constexpr (T == T_F16) {
        const uint8_t *p = row + (32 * b + 8 * c) * 2;
#pragma unroll
        for (int i = 0; i < 4; i++) r.w[i] = ldg_u32(p + 4 * i);
        r.d = 1.0f;
        r.m = 0.0f;
    } else {
        const uint8_t *blk = row + b * type_bytes(T);
        r.d = ldg_half(blk);
        r.m = has_min(T) ? ldg_half(blk + 2) : 0.0f;
        if constexpr (T == T_Q8_0) {
            const uint8_t *p = blk + 2 + 8 * c;
            r.w[0] = ldg_u32(p);
            r.w[1] = ldg_u32(p + 4);
        } else {
            constexpr int qs_off = T == T_Q4_0 ? 2 : T == T_Q4_1 ? 4 : T == T_Q5_0 ? 6 : 8;
            const uint8_t *p = blk + qs_off + 8 * (c & 1);
            r.w[0] = ldg_u32(p);
            r.w[1] = ldg_u32(p + 4);
            if constexpr (T == T_Q5_0 || T == T_Q5_1) {
                constexpr int qh_off = T == T_Q5_0 ? 2 : 4;
                r.w[2] = ldg_u32(blk + qh_off);
            }
        }
    }
}

// Unpack to 8 fp16 in natural dim order (4 dwords).  Quantized types give 1024 + u where u is
// the unsigned code (true code = u - code_off(T)); f16 gives the values, f32 rounds to fp16.
template <int T>
__device__ __forceinline__ void raw8_unpack(const Raw8 &r, int c, uint32_t o[4]) {
    if constexpr (T == T_F32) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float x0, x1;
            __builtin_memcpy(&x0, &r.w[2 * i], 4);
            __builtin_memcpy(&x1, &r.w[2 * i + 1], 4);
            h2 h = {(_Float16)x0, (_Float16)x1};
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

__device__ __forceinline__ float wave_max16x4(float v) {
    // reduce over the four lanes l, l^16, l^32, l^48 that share a row
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}
__device__ __forceinline__ float wave_sum16x4(float v) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup -> unit with consecutive units on one XCD (workgroups are dealt round-robin over
// the 8 XCDs, so ids w and w+8 share an L2).
__device__ __forceinline__ int64_t xcd_unit(int64_t w, int64_t n) {
    const int64_t x = w & 7, i = w >> 3, q = n >> 3, r = n & 7;
    return x * q + (x < r ? x : r) + i;
}

} // namespace cvattn
