// dm_device.h -- device helpers shared by the gfx950 kernels.
//
// All kernels are compiled with -ffp-contract=off: every fused multiply-add
// is an explicit __builtin_fmaf, and every other product/sum rounds on its
// own, as the reference's Rust code does (Rust never contracts).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dm {

constexpr uint32_t kF32 = 0, kF16 = 1, kQ5_0 = 6, kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14, kBF16 = 30;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2), aligned(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// Exact binary16 -> binary32, src/cpu.rs:647-660 (subnormals as frac*2^-24,
// Inf/NaN keep their payload; no quieting).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t value) {
    uint32_t sign = (value & 0x8000u) << 16;
    uint32_t exponent = (value >> 10) & 0x1fu;
    uint32_t fraction = value & 0x03ffu;
    if (exponent == 0) {
        float magnitude = (float)fraction * 5.9604644775390625e-08f;
        return sign ? -magnitude : magnitude;
    }
    uint32_t bits = exponent == 0x1f ? (sign | 0x7f800000u | (fraction << 13))
                                     : (sign | ((exponent + 112u) << 23) | (fraction << 13));
    return __uint_as_float(bits);
}

// Order-preserving map of a float onto uint32 (Rust total_cmp order for
// every non-NaN value, -0 < +0).
__device__ __forceinline__ uint32_t ordered_key(float v) {
    uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// 64-bit argmax key: larger value wins; on equal values the lower index wins.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t index) {
    return ((uint64_t)ordered_key(v) << 32) | (uint64_t)(0xffffffffu - index);
}

__device__ __forceinline__ uint32_t argmax_key_index(uint64_t key) {
    return 0xffffffffu - (uint32_t)(key & 0xffffffffu);
}

// Buffer resource over [base, base + bytes): loads past the end return zero
// instead of faulting.  The base is the caller's aligned-down address.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             0x00020000);
}

__device__ __forceinline__ u32x4 rsrc_load16(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0));
}

__device__ __forceinline__ uint32_t rsrc_load4(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, offset, 0, 0);
}

__device__ __forceinline__ u32x2 rsrc_load8(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, offset, 0, 0));
}

// Bytes [o, o+4) from two consecutive aligned dwords lo (at o - s) and hi,
// s = misalignment in bytes (0..3).
__device__ __forceinline__ uint32_t funnel(uint32_t lo, uint32_t hi, uint32_t s) {
    return __builtin_amdgcn_alignbyte(hi, lo, s);
}

// Wave-wide sum (64 lanes) through cross-lane shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        uint64_t o = __shfl_xor(v, m, 64);
        v = o > v ? o : v;
    }
    return v;
}

// Q4_K 6-bit (scale, min) unpack, src/cpu.rs:607-616.
__device__ __forceinline__ void scale_min_q4_k(int j, const uint8_t *s, uint32_t &sc, uint32_t &m) {
    if (j < 4) {
        sc = s[j] & 63u;
        m = s[j + 4] & 63u;
    } else {
        sc = (s[j + 4] & 0x0fu) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

}  // namespace dm
