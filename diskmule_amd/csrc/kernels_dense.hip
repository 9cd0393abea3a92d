// kernels_dense.hip -- GEMV over unquantized rows (F32, F16) for gfx950.
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
#include "dm_device.h"
#include "dm_kernels.h"

namespace dm {

namespace {

constexpr uint32_t kDenseWaves = 4, kRows = 2, kChunkGroup = 8;

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
    constexpr uint32_t E = kPerChunk<TYPE>;
    extern __shared__ float xs[];  // [TOK][columns]
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    for (uint32_t i = threadIdx.x; i < TOK * columns / 4; i += 64 * kDenseWaves)
        ((floatx4 *)xs)[i] = ((const floatx4 *)x)[i];
    __syncthreads();
    const uint32_t chunks = columns / E;  // per row
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
                        const floatx4 f = *(const floatx4 *)&xs[t * columns + c * E + 4 * q];
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

namespace {

template <uint32_t TYPE, int TOK>
hipError_t launch_dense_t(hipStream_t s, int cus, const uint8_t *w, uint32_t rows, uint32_t columns, size_t row_bytes,
                          const float *x, float *y, uint32_t y_stride) {
    const uint32_t lds = TOK * columns * 4;
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
    if (!(type == kF32 || type == kF16)) return false;
    const size_t e = type == kF32 ? 4 : 8;
    const size_t tok = batch < 4 ? batch : 4;
    return rows > 0 && columns > 0 && columns % e == 0 && columns * tok * 4 <= 64 * 1024 && rows < (1u << 31) &&
           ((uintptr_t)w & 15u) == 0 && ((uintptr_t)x & 15u) == 0;
}

hipError_t launch_dense_gemv(hipStream_t s, int cus, uint32_t type, const void *w, uint32_t rows, uint32_t columns,
                             size_t row_bytes, uint32_t batch, const float *x, float *y) {
    const uint8_t *wb = (const uint8_t *)w;
    if (type == kF32) return launch_dense_type<kF32>(s, cus, wb, rows, columns, row_bytes, batch, x, y);
    return launch_dense_type<kF16>(s, cus, wb, rows, columns, row_bytes, batch, x, y);
}

// A kernel of this file: resolving it loads the file's code object.
const void *module_anchor_dense() { return (const void *)dense_gemv_kernel<kF32, 1>; }

}  // namespace dm
