// kernels_qmv_valu.hip -- VALU decode GEMV for gfx950: batch 1 over Q4_K rows
// of 1, 2, 4, 8 or 16 super-blocks (256 to 4096 columns).
//
// y[r] = sum_c W[r][c] * x[c] (src/cpu.rs:345-399 semantics, fp32 products and
// fp32 accumulation in a different order than the CPU's sequential fold).
//
// This is the latency-bound form of the decode GEMV: a launch that streams a
// few MB (a 4096 x 4096 Q4_K matrix is 9.4 MB) is over in a few microseconds,
// so what matters is that every wave has all of its weight bytes requested
// the moment it starts, and that nothing waits on a workgroup barrier or an
// LDS round trip before the last bytes arrive.
//
//  * Lane mapping: four lanes per 256-value super-block (144 bytes).  Lane
//    quarter q of block b takes the block header (d, dmin, the 12 scale
//    bytes) and qs bytes [32q, 32q + 32): their low nibbles are values
//    64q .. 64q + 31 (sub-block 2q), their high nibbles values 64q + 32 ..
//    64q + 63 (sub-block 2q + 1) (src/cpu.rs:585-605).  A row of B blocks
//    takes 4B lanes; a wave covers 64 / 4B rows per pass.
//  * Every lane keeps its 64 activation values in registers for the whole
//    launch (the same columns in every row), plus their two sub-block sums:
//    the "- dmin * m * x" term of a sub-block is dmin * m * sum(x).
//  * A weight is its 4-bit code converted to fp32 (v_cvt_f32_ubyte after a
//    nibble mask) and multiplied into the running sum with an fma; the
//    sub-block scales d * sc and dmin * m apply once per sub-block.
//  * The partial sums of a row's lanes are added with cross-lane shuffles
//    (xor butterflies inside the row's lane group); lane 0 of the group
//    writes y[r].
//  * Each wave owns a contiguous range of rows and has the loads of its next
//    two passes in flight while it computes the current one.
#include "dm_device.h"
#include "dm_qmv.h"

namespace dm {

namespace {

// The three 16-byte pieces of one block a lane needs.
struct RawQ4 {
    u32x4 h;     // d | dmin | scales[0..12)
    u32x4 a, b;  // qs [32q, 32q + 16) and [32q + 16, 32q + 32)
};

__device__ __forceinline__ float f16_low(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
}

__device__ __forceinline__ void load_q4(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t q, RawQ4 &raw) {
    raw.h = rsrc_load16(r, off);
    raw.a = rsrc_load16(r, off + 16 + 32 * q);
    raw.b = rsrc_load16(r, off + 32 + 32 * q);
}

// Byte J of v as fp32 (v_cvt_f32_ubyteJ).  Written as instructions because
// the compiler otherwise extracts each nibble of a masked word with its own
// bit-field extract before converting byte 0.
template <int J>
__device__ __forceinline__ float byte_f(uint32_t v) {
    float r;
    if constexpr (J == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (J == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (J == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// This lane's share of one block: d * (sc0 * S0 + sc1 * S1) - dmin * (m0 * X0 + m1 * X1)
// with S the code . x dot of each sub-block and X its activation sum.
__device__ __forceinline__ float block_part(const RawQ4 &raw, const float (&xv)[64], float x0, float x1,
                                            uint32_t q) {
    const float d = f16_low(raw.h[0]);
    const float dmin = f16_low(raw.h[0] >> 16);
    // (scale, min) of sub-blocks 2q and 2q + 1 (src/cpu.rs:607-616): below 4
    // the low 6 bits of scales[j] and scales[j + 4]; from 4 on the nibbles of
    // scales[j + 4] with the top bits of scales[j - 4] and scales[j].
    float sc[2], mn[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t sh = 8 * ((2 * q + j) & 3u);
        const uint32_t b1 = raw.h[1] >> sh, b2 = raw.h[2] >> sh, b3 = raw.h[3] >> sh;
        const uint32_t s_lo = b1 & 63u, m_lo = b2 & 63u;
        const uint32_t s_hi = (b3 & 15u) | ((b1 >> 2) & 0x30u);
        const uint32_t m_hi = ((b3 >> 4) & 15u) | ((b2 >> 2) & 0x30u);
        sc[j] = (float)(q >= 2 ? s_hi : s_lo);
        mn[j] = (float)(q >= 2 ? m_hi : m_lo);
    }
    const uint32_t qs[8] = {raw.a[0], raw.a[1], raw.a[2], raw.a[3], raw.b[0], raw.b[1], raw.b[2], raw.b[3]};
    // two accumulators per sub-block: independent fma chains
    float s0a = 0.0f, s0b = 0.0f, s1a = 0.0f, s1b = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t lo = qs[k] & 0x0f0f0f0fu;
        const uint32_t hi = (qs[k] >> 4) & 0x0f0f0f0fu;
        float &s0 = (k & 1) ? s0b : s0a;
        float &s1 = (k & 1) ? s1b : s1a;
        s0 = __builtin_fmaf(byte_f<0>(lo), xv[4 * k], s0);
        s1 = __builtin_fmaf(byte_f<0>(hi), xv[32 + 4 * k], s1);
        s0 = __builtin_fmaf(byte_f<1>(lo), xv[4 * k + 1], s0);
        s1 = __builtin_fmaf(byte_f<1>(hi), xv[32 + 4 * k + 1], s1);
        s0 = __builtin_fmaf(byte_f<2>(lo), xv[4 * k + 2], s0);
        s1 = __builtin_fmaf(byte_f<2>(hi), xv[32 + 4 * k + 2], s1);
        s0 = __builtin_fmaf(byte_f<3>(lo), xv[4 * k + 3], s0);
        s1 = __builtin_fmaf(byte_f<3>(hi), xv[32 + 4 * k + 3], s1);
    }
    const float part = __builtin_fmaf(sc[1], s1a + s1b, sc[0] * (s0a + s0b));
    const float mins = __builtin_fmaf(mn[1], x1, mn[0] * x0);
    return __builtin_fmaf(d, part, -(dmin * mins));
}

constexpr uint32_t kValuWaves = 4;  // waves per workgroup
constexpr uint32_t kValuAhead = 2;  // passes in flight per wave

// Wave v handles passes [v * per_wave, (v + 1) * per_wave) (a pass is 64 / 4B
// rows), clipped to the matrix.
template <uint32_t BLOCKS>
__global__ void __launch_bounds__(64 * kValuWaves) qmv_valu_q4k_kernel(
    const uint8_t *__restrict__ w, uint32_t rows, uint32_t total_bytes, const float *__restrict__ x,
    float *__restrict__ y, uint32_t per_wave) {
    constexpr uint32_t L = 4 * BLOCKS;   // lanes per row
    constexpr uint32_t P = 64 / L;       // rows per pass
    constexpr uint32_t RB = 144 * BLOCKS;  // row bytes
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = blockIdx.x * kValuWaves + (threadIdx.x >> 6);
    const uint32_t sub = lane / L, li = lane % L;
    const uint32_t blk = li >> 2, q = li & 3u;
    const uint32_t passes = (rows + P - 1) / P;
    const uint32_t p0 = wave * per_wave;
    const uint32_t p1 = p0 + per_wave < passes ? p0 + per_wave : passes;
    if (p0 >= p1) return;

    const uint32_t records = (total_bytes + 3u) & ~3u;
    const uint32_t nowhere = records + 256;
    const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(w, records);
    auto block_off = [&](uint32_t pass) -> uint32_t {
        const uint32_t row = pass * P + sub;
        return (pass < p1 && row < rows) ? row * RB + blk * 144 : nowhere;
    };

    // The weights of the first passes are requested before anything else.
    RawQ4 raw[kValuAhead];
#pragma unroll
    for (uint32_t i = 0; i < kValuAhead; i++) load_q4(rsrc, block_off(p0 + i), q, raw[i]);

    float xv[64];
    const float4 *xs = (const float4 *)(x + blk * 256 + 64 * q);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float4 v = xs[i];
        xv[4 * i] = v.x;
        xv[4 * i + 1] = v.y;
        xv[4 * i + 2] = v.z;
        xv[4 * i + 3] = v.w;
    }
    float x0 = 0.0f, x1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        x0 += xv[i];
        x1 += xv[32 + i];
    }

    for (uint32_t p = p0; p < p1; p += kValuAhead) {
#pragma unroll
        for (uint32_t i = 0; i < kValuAhead; i++) {
            const uint32_t pass = p + i;
            if (pass >= p1) break;
            float v = block_part(raw[i], xv, x0, x1, q);
            // the next load into this slot goes out before the reduction
            load_q4(rsrc, block_off(pass + kValuAhead), q, raw[i]);
#pragma unroll
            for (uint32_t m = 1; m < L; m <<= 1) v += __shfl_xor(v, (int)m, 64);
            const uint32_t row = pass * P + sub;
            if (li == 0 && row < rows) y[row] = v;
        }
    }
}

template <uint32_t BLOCKS>
hipError_t run_valu_q4k(dmhip_ctx *ctx, uint32_t rows, const void *w, const float *x, float *y) {
    constexpr uint32_t P = 64 / (4 * BLOCKS);
    const uint32_t passes = (rows + P - 1) / P;
    // About eight waves per compute unit, each with an even share of passes.
    const uint32_t cus = ctx->compute_units > 0 ? (uint32_t)ctx->compute_units : 256u;
    const uint32_t target = 8 * cus;
    uint32_t per_wave = (passes + target - 1) / target;
    if (per_wave == 0) per_wave = 1;
    const uint32_t waves = (passes + per_wave - 1) / per_wave;
    const uint32_t grid = (waves + kValuWaves - 1) / kValuWaves;
    return launch_kernel(ctx, qmv_valu_q4k_kernel<BLOCKS>, dim3(grid), dim3(64 * kValuWaves), 0,
                         (const uint8_t *)w, rows, rows * 144u * BLOCKS, x, y, per_wave);
}

}  // namespace

bool qmv_valu_supported(uint32_t type, size_t rows, size_t columns, const void *w, const float *x,
                        size_t batch) {
    if (type != kQ4_K || batch != 1 || rows == 0) return false;
    if (((uintptr_t)w & 15u) != 0 || ((uintptr_t)x & 15u) != 0) return false;
    const size_t blocks = columns / 256;
    if (columns % 256 || !(blocks == 1 || blocks == 2 || blocks == 4 || blocks == 8 || blocks == 16)) return false;
    return (uint64_t)rows * blocks * 144u < (1ull << 32) - 512;
}

hipError_t launch_qmv_valu(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns, const void *w,
                           const float *x, float *y) {
    (void)type;
    switch (columns / 256) {
    case 1: return run_valu_q4k<1>(ctx, rows, w, x, y);
    case 2: return run_valu_q4k<2>(ctx, rows, w, x, y);
    case 4: return run_valu_q4k<4>(ctx, rows, w, x, y);
    case 8: return run_valu_q4k<8>(ctx, rows, w, x, y);
    default: return run_valu_q4k<16>(ctx, rows, w, x, y);
    }
}

// A kernel of this file: resolving it loads the file's code object.
const void *module_anchor_qmv_valu() { return (const void *)qmv_valu_q4k_kernel<16>; }

}  // namespace dm
