// kernels_dense.hip -- GEMV over F32, F16 and Q5_0 rows for gfx950.
//
// y[t][r] = sum_c W[r][c] * x[t][c] for up to 4 tokens (src/cpu.rs:345-399
// semantics; the sum runs in a different order than the reference's
// sequential fold, within the dot-product tolerance).  HBM-bound: one pass
// over W at full width.
//
// A workgroup of 4 waves stages the tokens' activations in LDS once (fp32,
// tokens x columns), then walks row groups (persistent): each wave takes
// kRows rows at a time, lane l reads the 16-byte chunks l, l + 64, ... of
// every row (4 F32 or 8 F16 weights each), kChunkGroup chunks of each
// row in flight per step, folds them with fma against the activations read
// from LDS, and ends each row with a wave sum.
//
// Q5_0 rows (22-byte blocks of 32 values, src/cpu.rs:560-574) take the same
// walk with one block per lane: its 22 bytes sit 2 bytes off a dword
// boundary in every other block, so the lane reads the 6 aligned dwords
// around it through a range-checked buffer resource (reads past the end
// of W return zeros) and aligns them with funnel shifts.  The value
// d (q - 16) is exact in fp32; the kernel sums x q over the block, subtracts
// 16 times the block's activation sum (staged once per workgroup) and
// multiplies by d once (a different rounding order, within the tolerance).
#include "dm_device.h"
#include "dm_kernels.h"

namespace dm {

namespace {

constexpr uint32_t kDenseWaves = 4, kRows = 2, kChunkGroup = 8;
constexpr uint32_t kXU = 8;  // activation loads per thread in flight while staging

// Elements of one 16-byte chunk.
template <uint32_t TYPE> constexpr uint32_t kPerChunk = TYPE == kF32 ? 4u : 8u;

// The weights of chunk v as floats.
template <uint32_t TYPE>
__device__ __forceinline__ void widen(const u32x4 &v, float (&out)[kPerChunk<TYPE>]) {
    if constexpr (TYPE == kF32) {
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = __uint_as_float(v[i]);
    } else {
        // binary16 -> binary32 is exact (src/cpu.rs:647-660)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            out[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v[i] & 0xffffu));
            out[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v[i] >> 16));
        }
    }
}

}  // namespace

template <uint32_t TYPE, int TOK>
__global__ void __launch_bounds__(64 * kDenseWaves) dense_gemv_kernel(const uint8_t *__restrict__ w, uint32_t rows,
                                                                      uint32_t columns, size_t row_bytes,
                                                                      const float *__restrict__ x,
                                                                      float *__restrict__ y, uint32_t y_stride) {
    constexpr uint32_t E = kPerChunk<TYPE>, XP = E + 4;  // LDS floats per chunk
    // [TOK][chunks][E + 4]: lanes reading consecutive chunks start 4 banks
    // apart, so a 16-byte read of 16 lanes touches all 64 banks once.
    extern __shared__ __attribute__((aligned(16))) float xs[];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t chunks = columns / E;  // per row
    // kXU loads of each thread in flight before their stores
    for (uint32_t i0 = 0; i0 < TOK * columns / 4; i0 += kXU * 64 * kDenseWaves) {
        floatx4 v[kXU];
#pragma unroll
        for (uint32_t j = 0; j < kXU; j++) {
            const uint32_t i = i0 + j * 64 * kDenseWaves + threadIdx.x;
            v[j] = i < TOK * columns / 4 ? ((const floatx4 *)x)[i] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (uint32_t j = 0; j < kXU; j++) {
            const uint32_t i = i0 + j * 64 * kDenseWaves + threadIdx.x;
            if (i >= TOK * columns / 4) break;
            const uint32_t t = i / (columns / 4), k = i % (columns / 4);
            *(floatx4 *)&xs[(t * chunks + k / (E / 4)) * XP + 4 * (k % (E / 4))] = v[j];
        }
    }
    __syncthreads();
    const uint32_t step = gridDim.x * kDenseWaves * kRows;
    for (uint32_t r0 = (blockIdx.x * kDenseWaves + wave) * kRows; r0 < rows; r0 += step) {
        float acc[kRows][TOK];
#pragma unroll
        for (uint32_t r = 0; r < kRows; r++)
#pragma unroll
            for (int t = 0; t < TOK; t++) acc[r][t] = 0.0f;
        for (uint32_t c0 = 0; c0 < chunks; c0 += 64 * kChunkGroup) {
            u32x4 v[kRows][kChunkGroup];
#pragma unroll
            for (uint32_t r = 0; r < kRows; r++)
#pragma unroll
                for (uint32_t j = 0; j < kChunkGroup; j++) {
                    const uint32_t c = c0 + 64 * j + lane;
                    v[r][j] = r0 + r < rows && c < chunks
                                  ? *(const u32x4 *)(w + (size_t)(r0 + r) * row_bytes + (size_t)c * 16)
                                  : u32x4{0, 0, 0, 0};
                }
#pragma unroll
            for (uint32_t j = 0; j < kChunkGroup; j++) {
                const uint32_t c = c0 + 64 * j + lane;
                if (c >= chunks) break;
                float xv[TOK][E];
#pragma unroll
                for (int t = 0; t < TOK; t++)
#pragma unroll
                    for (uint32_t q = 0; q < E / 4; q++) {
                        const floatx4 f = *(const floatx4 *)&xs[(t * chunks + c) * XP + 4 * q];
#pragma unroll
                        for (int e = 0; e < 4; e++) xv[t][4 * q + e] = f[e];
                    }
#pragma unroll
                for (uint32_t r = 0; r < kRows; r++) {
                    float wv[E];
                    widen<TYPE>(v[r][j], wv);
#pragma unroll
                    for (int t = 0; t < TOK; t++)
#pragma unroll
                        for (uint32_t e = 0; e < E; e++) acc[r][t] = __builtin_fmaf(wv[e], xv[t][e], acc[r][t]);
                }
            }
        }
#pragma unroll
        for (uint32_t r = 0; r < kRows; r++)
#pragma unroll
            for (int t = 0; t < TOK; t++) {
                const float s = wave_sum(acc[r][t]);
                if (lane == 0 && r0 + r < rows) y[(size_t)t * y_stride + r0 + r] = s;
            }
    }
}

// The 4 bits of h (0..15) as bit 4 of bytes 0..3: the product places copies
// of h at bits 0, 7, 14 and 21, which never overlap, so bit i of h lands at
// bit 4 + 8 i after the shift.
// (A 24-bit multiply: h < 16 and the constant < 2^24.)
__device__ __forceinline__ uint32_t spread4(uint32_t h) { return (__umul24(h, 0x00204081u) << 4) & 0x10101010u; }

constexpr uint32_t kQ5Ld = 36;  // LDS floats per staged block of 32 activations

template <int TOK>
__global__ void __launch_bounds__(64 * kDenseWaves) q5_0_gemv_kernel(const uint8_t *__restrict__ w, uint32_t w_bytes,
                                                                     uint32_t rows, uint32_t columns, uint32_t row_bytes,
                                                                     const float *__restrict__ x,
                                                                     float *__restrict__ y, uint32_t y_stride) {
    // LDS: the tokens' activations, kQ5Ld floats per 32-value block (lane l
    // reads block b + l: the padding spreads neighbouring lanes' 16-byte
    // reads over all banks), then per block the sum of its 32 activations
    // (the "- 16" of every code is -16 times that sum).
    extern __shared__ float xs[];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t blocks = columns / 32;
    float *xsum = xs + TOK * blocks * kQ5Ld;
    for (uint32_t i0 = 0; i0 < TOK * columns / 4; i0 += kXU * 64 * kDenseWaves) {
        floatx4 v[kXU];
#pragma unroll
        for (uint32_t j = 0; j < kXU; j++) {
            const uint32_t i = i0 + j * 64 * kDenseWaves + threadIdx.x;
            v[j] = i < TOK * columns / 4 ? ((const floatx4 *)x)[i] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (uint32_t j = 0; j < kXU; j++) {
            const uint32_t i = i0 + j * 64 * kDenseWaves + threadIdx.x;
            if (i >= TOK * columns / 4) break;
            const uint32_t blk = i / 8, q = i % 8;  // 8 float4s per block
            *(floatx4 *)&xs[blk * kQ5Ld + 4 * q] = v[j];
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < TOK * blocks; i += 64 * kDenseWaves) {
        floatx4 q[8];
#pragma unroll
        for (int e = 0; e < 8; e++) q[e] = *(const floatx4 *)&xs[i * kQ5Ld + 4 * e];  // all reads before the sum
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; e++) s += q[e / 4][e % 4];
        xsum[i] = s;
    }
    __syncthreads();
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(w, w_bytes);
    constexpr uint32_t kGroup = 2;  // blocks per lane in flight, per row
    const uint32_t step = gridDim.x * kDenseWaves * kRows;
    for (uint32_t r0 = (blockIdx.x * kDenseWaves + wave) * kRows; r0 < rows; r0 += step) {
        float acc[kRows][TOK];
#pragma unroll
        for (uint32_t r = 0; r < kRows; r++)
#pragma unroll
            for (int t = 0; t < TOK; t++) acc[r][t] = 0.0f;
        for (uint32_t b0 = 0; b0 < blocks; b0 += 64 * kGroup) {
            uint32_t d[kRows][kGroup][6];
#pragma unroll
            for (uint32_t r = 0; r < kRows; r++)
#pragma unroll
                for (uint32_t j = 0; j < kGroup; j++) {
                    const uint32_t b = b0 + 64 * j + lane;
                    // rows past the end and blocks past the row read past W: zeros
                    const uint32_t at = r0 + r < rows && b < blocks ? (r0 + r) * row_bytes + 22 * b : w_bytes;
                    const u32x4 lo = rsrc_load16(rs, at & ~3u);
                    const u32x2 hi = rsrc_load8(rs, (at & ~3u) + 16);
#pragma unroll
                    for (int i = 0; i < 4; i++) d[r][j][i] = lo[i];
                    d[r][j][4] = hi[0];
                    d[r][j][5] = hi[1];
                }
#pragma unroll
            for (uint32_t j = 0; j < kGroup; j++) {
                const uint32_t b = b0 + 64 * j + lane;
                if (b >= blocks) break;
                float xv[TOK][32], xb[TOK];
#pragma unroll
                for (int t = 0; t < TOK; t++) {
#pragma unroll
                    for (int q = 0; q < 8; q++) {
                        const floatx4 f = *(const floatx4 *)&xs[(t * blocks + b) * kQ5Ld + 4 * q];
#pragma unroll
                        for (int e = 0; e < 4; e++) xv[t][4 * q + e] = f[e];
                    }
                    xb[t] = xsum[t * blocks + b];
                }
#pragma unroll
                for (uint32_t r = 0; r < kRows; r++) {
                    // the block's bytes 4k .. 4k + 3 as v[k] (bytes 0-1 d, 2-5
                    // high bits, 6-21 nibbles)
                    const uint32_t sh = ((r0 + r) * row_bytes + 22 * b) & 3u;
                    uint32_t v[6];
#pragma unroll
                    for (int i = 0; i < 5; i++) v[i] = funnel(d[r][j][i], d[r][j][i + 1], sh);
                    v[5] = d[r][j][5] >> (8 * sh);
                    const float delta = f16_bits_to_f32(v[0] & 0xffffu);
                    const uint32_t high = (v[0] >> 16) | (v[1] << 16);
                    float s[TOK];
#pragma unroll
                    for (int t = 0; t < TOK; t++) s[t] = 0.0f;
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        // nibble bytes 6 + 4k .. 9 + 4k: the codes of elements
                        // 4k .. 4k + 3 (low nibbles) and 16 + 4k .. (high
                        // nibbles), each with its fifth bit from `high`
                        const uint32_t qs = funnel(v[k + 1], v[k + 2], 2);
                        const uint32_t lo = (qs & 0x0f0f0f0fu) | spread4((high >> (4 * k)) & 15u);
                        const uint32_t hi = ((qs >> 4) & 0x0f0f0f0fu) | spread4((high >> (16 + 4 * k)) & 15u);
                        float ql[4], qh[4];  // byte e as a float: one v_cvt_f32_ubyte each
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            ql[e] = (float)((lo >> (8 * e)) & 0xffu);
                            qh[e] = (float)((hi >> (8 * e)) & 0xffu);
                        }
#pragma unroll
                        for (int t = 0; t < TOK; t++)
#pragma unroll
                            for (int e = 0; e < 4; e++) {
                                s[t] = __builtin_fmaf(ql[e], xv[t][4 * k + e], s[t]);
                                s[t] = __builtin_fmaf(qh[e], xv[t][16 + 4 * k + e], s[t]);
                            }
                    }
#pragma unroll
                    for (int t = 0; t < TOK; t++)
                        acc[r][t] = __builtin_fmaf(delta, __builtin_fmaf(-16.0f, xb[t], s[t]), acc[r][t]);
                }
            }
        }
#pragma unroll
        for (uint32_t r = 0; r < kRows; r++)
#pragma unroll
            for (int t = 0; t < TOK; t++) {
                const float sum = wave_sum(acc[r][t]);
                if (lane == 0 && r0 + r < rows) y[(size_t)t * y_stride + r0 + r] = sum;
            }
    }
}

namespace {

template <uint32_t TYPE, int TOK>
hipError_t launch_dense_t(hipStream_t s, int cus, const uint8_t *w, uint32_t rows, uint32_t columns, size_t row_bytes,
                          const float *x, float *y, uint32_t y_stride) {
    const uint32_t lds = TOK * (columns / kPerChunk<TYPE>) * (kPerChunk<TYPE> + 4) * 4;
    static LdsLimit limit;
    hipError_t e = limit.ensure((const void *)dense_gemv_kernel<TYPE, TOK>, lds);
    if (e != hipSuccess) return e;
    const uint32_t groups = (rows + kDenseWaves * kRows - 1) / (kDenseWaves * kRows);
    // enough workgroups to cover the CUs a few times; each stages x once
    const uint32_t cap = (uint32_t)(cus > 0 ? cus : 256) * 4;
    const uint32_t grid = groups < cap ? groups : cap;
    hipLaunchKernelGGL((dense_gemv_kernel<TYPE, TOK>), dim3(grid), dim3(64 * kDenseWaves), lds, s, w, rows, columns,
                       row_bytes, x, y, y_stride);
    return hipGetLastError();
}

template <int TOK>
hipError_t launch_q5_0_t(hipStream_t s, int cus, const uint8_t *w, uint32_t w_bytes, uint32_t rows, uint32_t columns,
                         uint32_t row_bytes, const float *x, float *y, uint32_t y_stride) {
    const uint32_t lds = TOK * (columns / 32) * (kQ5Ld + 1) * 4;
    static LdsLimit limit;
    hipError_t e = limit.ensure((const void *)q5_0_gemv_kernel<TOK>, lds);
    if (e != hipSuccess) return e;
    const uint32_t groups = (rows + kDenseWaves * kRows - 1) / (kDenseWaves * kRows);
    const uint32_t cap = (uint32_t)(cus > 0 ? cus : 256) * 4;
    const uint32_t grid = groups < cap ? groups : cap;
    hipLaunchKernelGGL((q5_0_gemv_kernel<TOK>), dim3(grid), dim3(64 * kDenseWaves), lds, s, w, w_bytes, rows, columns,
                       row_bytes, x, y, y_stride);
    return hipGetLastError();
}

template <uint32_t TYPE>
hipError_t launch_dense_type(hipStream_t s, int cus, const uint8_t *w, uint32_t rows, uint32_t columns,
                             size_t row_bytes, uint32_t batch, const float *x, float *y) {
    for (uint32_t t0 = 0; t0 < batch; t0 += 4) {
        const uint32_t n = batch - t0 < 4 ? batch - t0 : 4;
        const float *xt = x + (size_t)t0 * columns;
        float *yt = y + (size_t)t0 * rows;
        hipError_t e;
        switch (n) {
        case 1: e = launch_dense_t<TYPE, 1>(s, cus, w, rows, columns, row_bytes, xt, yt, rows); break;
        case 2: e = launch_dense_t<TYPE, 2>(s, cus, w, rows, columns, row_bytes, xt, yt, rows); break;
        case 3: e = launch_dense_t<TYPE, 3>(s, cus, w, rows, columns, row_bytes, xt, yt, rows); break;
        default: e = launch_dense_t<TYPE, 4>(s, cus, w, rows, columns, row_bytes, xt, yt, rows); break;
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

bool dense_supported(uint32_t type, size_t rows, size_t columns, const void *w, const float *x, size_t batch) {
    const size_t tok = batch < 4 ? batch : 4;
    if (rows == 0 || columns == 0 || (columns / 32) * (kQ5Ld + 1) * tok * 4 > 64 * 1024 || ((uintptr_t)x & 15u) != 0)
        return false;
    if (type == kQ5_0)  // whole blocks, dword-aligned rows, W within the 32-bit buffer range
        return columns % 64 == 0 && ((uintptr_t)w & 3u) == 0 && (uint64_t)rows * (columns / 32) * 22 < 0x7fffffffull;
    if (!(type == kF32 || type == kF16)) return false;
    const size_t e = type == kF32 ? 4 : 8;
    return columns % e == 0 && rows < (1u << 31) && ((uintptr_t)w & 15u) == 0;
}

hipError_t launch_dense_gemv(hipStream_t s, int cus, uint32_t type, const void *w, uint32_t rows, uint32_t columns,
                             size_t row_bytes, uint32_t batch, const float *x, float *y) {
    const uint8_t *wb = (const uint8_t *)w;
    if (type == kQ5_0) {
        const uint32_t w_bytes = (uint32_t)(rows * row_bytes);
        for (uint32_t t0 = 0; t0 < batch; t0 += 4) {
            const uint32_t n = batch - t0 < 4 ? batch - t0 : 4;
            const float *xt = x + (size_t)t0 * columns;
            float *yt = y + (size_t)t0 * rows;
            hipError_t e;
            switch (n) {
            case 1: e = launch_q5_0_t<1>(s, cus, wb, w_bytes, rows, columns, (uint32_t)row_bytes, xt, yt, rows); break;
            case 2: e = launch_q5_0_t<2>(s, cus, wb, w_bytes, rows, columns, (uint32_t)row_bytes, xt, yt, rows); break;
            case 3: e = launch_q5_0_t<3>(s, cus, wb, w_bytes, rows, columns, (uint32_t)row_bytes, xt, yt, rows); break;
            default: e = launch_q5_0_t<4>(s, cus, wb, w_bytes, rows, columns, (uint32_t)row_bytes, xt, yt, rows); break;
            }
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    if (type == kF32) return launch_dense_type<kF32>(s, cus, wb, rows, columns, row_bytes, batch, x, y);
    return launch_dense_type<kF16>(s, cus, wb, rows, columns, row_bytes, batch, x, y);
}

// A kernel of this file: resolving it loads the file's code object.
const void *module_anchor_dense() { return (const void *)dense_gemv_kernel<kF32, 1>; }

}  // namespace dm
