// kernels_safetensor.hip -- GEMV over GLM safetensors matrices for gfx950
// (MetalContext::matvec_safetensor / _mapped, src/metal.rs:738-1146;
// metal/kernels.metal:243-344).
//
// Formats (src/glm52/cpu.rs:1180-1420):
//  * BF16 rows: w = bits << 16 (exact);
//  * F8_E4M3FN rows with one f32 scale per 128 x 128 block: the byte decodes
//    on the hardware converter (gfx950 converts the OCP E4M3 format: the NaN
//    codes 0x7f / 0xff give NaN, as metal/kernels.metal:260-271 does);
//  * row INT8: signed bytes, one scale per row;
//  * grouped INT4: two codes per byte (low nibble first), (n - 8) times the
//    scale of the column's group, rows of ceil(columns / 2) bytes.
//
// st_gemv_kernel is the wide-load form (rows of whole 16-byte chunks, the
// activation in LDS): a workgroup of 4 waves stages x once and walks row
// pairs persistently; lane l reads chunks l, l + 64, ... of each row, eight
// per row in flight.  The block or group scale multiplies a chunk's partial
// sum (one rounding order; the sum runs in a different order than the
// reference's sequential fold, within the dot-product tolerance).  INT4
// chunks sum n * x with one v_cvt_f32_ubyte per code and subtract 8 times
// the chunk's activation sum, staged once per workgroup.
//
// st_gemv_generic_kernel takes every other shape (odd INT4 columns, groups
// of 48, unaligned rows): one wave per row, each weight the reference's
// product decode(code) * scale, then fma with x.
#include "dm_device.h"
#include "dm_kernels.h"

namespace dm {

namespace {

constexpr uint32_t kStWaves = 4;

template <uint32_t FMT> constexpr uint32_t kStPerChunk = FMT == kStBf16 ? 8u : FMT == kStI4 ? 32u : 16u;

__device__ __forceinline__ float bf16_bits(uint32_t h) { return __uint_as_float(h << 16); }

typedef float float2v __attribute__((ext_vector_type(2)));

// Four E4M3FN bytes of v as floats (hardware conversion).
__device__ __forceinline__ void fp8x4(uint32_t v, float *out) {
    const float2v lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)v, false);
    const float2v hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)v, true);
    out[0] = lo.x;
    out[1] = lo.y;
    out[2] = hi.x;
    out[3] = hi.y;
}

// E4M3FN by the reference's formula (src/glm52/cpu.rs:1397-1410), NaN for
// the two NaN codes (metal/kernels.metal:260-271).
__device__ __forceinline__ float fp8_formula(uint32_t b) {
    const float sign = (b & 0x80u) ? -1.0f : 1.0f;
    const uint32_t e = (b >> 3) & 15u, f = b & 7u;
    if (e == 15u && f == 7u) return __builtin_nanf("");
    // 2^(e - 7) exactly, from its exponent field
    const float m = e == 0 ? (float)f * 0.001953125f : (1.0f + (float)f * 0.125f) * __uint_as_float((e + 120u) << 23);
    return sign * m;
}

}  // namespace

// y[r] = sum_c W[r][c] x[c], one token.  scales: F8 [ceil(rows/128)][sc],
// INT8 [rows], INT4 [rows][sc] with `group` columns per scale.
// R rows per wave step, C chunks of each row in flight per lane.
template <uint32_t FMT, uint32_t kStRows, uint32_t kStChunks>
__global__ void __launch_bounds__(64 * kStWaves)
st_gemv_kernel(const uint8_t *__restrict__ w, uint32_t rows, uint32_t columns, size_t row_bytes,
               const float *__restrict__ scales, uint32_t scale_columns, uint32_t group, const float *__restrict__ x,
               float *__restrict__ y) {
    constexpr uint32_t E = kStPerChunk<FMT>, XP = E + 4;  // LDS floats per chunk
    // [chunks][E + 4]: lanes reading consecutive chunks start 4 banks apart,
    // so a 16-byte read of 16 lanes touches all 64 banks once.  INT4: then a
    // sum per 16 columns.
    extern __shared__ __attribute__((aligned(16))) float xs[];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t chunks = columns / E;
    {
        // every load of a thread in flight before the first store (columns <= 16384;
        // measured at 12288 x 6144: F8 16.6 -> 15.9 us, INT8 16.3 -> 15.5 us, BF16
        // 26.2 -> 25.6 us per launch against one load in flight at a time)
        constexpr uint32_t kXU = 16;
        const uint32_t n4 = columns / 4;
        floatx4 t[kXU];
#pragma unroll
        for (uint32_t j = 0; j < kXU; j++) {
            const uint32_t i = j * 64 * kStWaves + threadIdx.x;
            t[j] = i < n4 ? ((const floatx4 *)x)[i] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (uint32_t j = 0; j < kXU; j++) {
            const uint32_t i = j * 64 * kStWaves + threadIdx.x;
            if (i < n4) *(floatx4 *)&xs[(i / (E / 4)) * XP + 4 * (i % (E / 4))] = t[j];
        }
    }
    float *xsum = xs + chunks * XP;
    if constexpr (FMT == kStI4) {
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < columns / 16; i += 64 * kStWaves) {
            const float *src = xs + (i / 2) * XP + 16 * (i % 2);
            floatx4 q[4];
#pragma unroll
            for (int k = 0; k < 4; k++) q[k] = *(const floatx4 *)&src[4 * k];  // all reads before the sum
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; k++) s += q[k / 4][k % 4];
            xsum[i] = s;
        }
    }
    __syncthreads();
    const uint32_t step = gridDim.x * kStWaves * kStRows;
    for (uint32_t r0 = (blockIdx.x * kStWaves + wave) * kStRows; r0 < rows; r0 += step) {
        float acc[kStRows] = {};
        for (uint32_t c0 = 0; c0 < chunks; c0 += 64 * kStChunks) {
            // the chunks' weights and their block / group scales, all in flight
            // before the first is used
            constexpr int NS = FMT == kStF8 || FMT == kStI4 ? (FMT == kStI4 ? 2 : 1) : 0;
            u32x4 v[kStRows][kStChunks];
            float sv[kStRows][kStChunks][NS > 0 ? NS : 1];
#pragma unroll
            for (uint32_t r = 0; r < kStRows; r++)
#pragma unroll
                for (uint32_t j = 0; j < kStChunks; j++) {
                    const uint32_t c = c0 + 64 * j + lane;
                    const bool ok = r0 + r < rows && c < chunks;
                    v[r][j] = ok ? *(const u32x4 *)(w + (size_t)(r0 + r) * row_bytes + (size_t)c * 16)
                                 : u32x4{0, 0, 0, 0};
                    if constexpr (FMT == kStF8) {
                        // the chunk's 16 columns lie in one 128-column block
                        sv[r][j][0] = ok ? scales[((r0 + r) / 128) * scale_columns + c / 8] : 0.0f;
                    } else if constexpr (FMT == kStI4) {
                        const float *srow = scales + (size_t)(r0 + r) * scale_columns;
                        // group 16: a scale per half chunk; else one per chunk
                        sv[r][j][0] = ok ? srow[group == 16 ? 2 * c : (32 * c) / group] : 0.0f;
                        sv[r][j][1] = ok && group == 16 ? srow[2 * c + 1] : 0.0f;
                    }
                }
#pragma unroll
            for (uint32_t j = 0; j < kStChunks; j++) {
                const uint32_t c = c0 + 64 * j + lane;
                if (c >= chunks) break;
                float xv[E];
#pragma unroll
                for (uint32_t q = 0; q < E / 4; q++) {
                    const floatx4 f = *(const floatx4 *)&xs[c * XP + 4 * q];
#pragma unroll
                    for (int e = 0; e < 4; e++) xv[4 * q + e] = f[e];
                }
#pragma unroll
                for (uint32_t r = 0; r < kStRows; r++) {
                    if constexpr (FMT == kStBf16) {
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            acc[r] = __builtin_fmaf(bf16_bits(v[r][j][i] & 0xffffu), xv[2 * i], acc[r]);
                            acc[r] = __builtin_fmaf(bf16_bits(v[r][j][i] >> 16), xv[2 * i + 1], acc[r]);
                        }
                    } else if constexpr (FMT == kStI8) {
#pragma unroll
                        for (int i = 0; i < 4; i++)
#pragma unroll
                            for (int b = 0; b < 4; b++) {
                                const float q = (float)(int32_t)((int32_t)(v[r][j][i] << (24 - 8 * b)) >> 24);
                                acc[r] = __builtin_fmaf(q, xv[4 * i + b], acc[r]);
                            }
                    } else if constexpr (FMT == kStF8) {
                        float s = 0.0f;
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            float d[4];
                            fp8x4(v[r][j][i], d);
#pragma unroll
                            for (int b = 0; b < 4; b++) s = __builtin_fmaf(d[b], xv[4 * i + b], s);
                        }
                        acc[r] = __builtin_fmaf(sv[r][j][0], s, acc[r]);
                    } else {
                        // 32 codes: dword i holds columns 8i .. 8i + 7, low nibble first
                        float s[2] = {0.0f, 0.0f};
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const uint32_t even = v[r][j][i] & 0x0f0f0f0fu, odd = (v[r][j][i] >> 4) & 0x0f0f0f0fu;
#pragma unroll
                            for (int b = 0; b < 4; b++) {
                                s[i >> 1] = __builtin_fmaf((float)((even >> (8 * b)) & 0xffu), xv[8 * i + 2 * b], s[i >> 1]);
                                s[i >> 1] = __builtin_fmaf((float)((odd >> (8 * b)) & 0xffu), xv[8 * i + 2 * b + 1], s[i >> 1]);
                            }
                        }
                        const float h0 = __builtin_fmaf(-8.0f, xsum[2 * c], s[0]);
                        const float h1 = __builtin_fmaf(-8.0f, xsum[2 * c + 1], s[1]);
                        if (group == 16) {
                            acc[r] = __builtin_fmaf(sv[r][j][0], h0, acc[r]);
                            acc[r] = __builtin_fmaf(sv[r][j][1], h1, acc[r]);
                        } else {
                            // group a multiple of 32: one scale for the chunk
                            acc[r] = __builtin_fmaf(sv[r][j][0], h0 + h1, acc[r]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (uint32_t r = 0; r < kStRows; r++) {
            float s = wave_sum(acc[r]);
            if (lane == 0 && r0 + r < rows) {
                if constexpr (FMT == kStI8) s *= scales[r0 + r];
                y[r0 + r] = s;
            }
        }
    }
}

template <uint32_t FMT>
__global__ void __launch_bounds__(256)
st_gemv_generic_kernel(const uint8_t *__restrict__ w, uint32_t rows, uint32_t columns, const float *__restrict__ scales,
                       uint32_t scale_columns, uint32_t group, const float *__restrict__ x, float *__restrict__ y) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float acc = 0.0f;
    for (uint32_t c = lane; c < columns; c += 64) {
        float wv;
        if constexpr (FMT == kStBf16) {
            const uint8_t *p = w + ((size_t)row * columns + c) * 2;
            wv = bf16_bits((uint32_t)p[0] | ((uint32_t)p[1] << 8));
        } else if constexpr (FMT == kStF8) {
            wv = fp8_formula(w[(size_t)row * columns + c]) * scales[(row / 128) * scale_columns + c / 128];
        } else if constexpr (FMT == kStI8) {
            wv = (float)(int8_t)w[(size_t)row * columns + c] * scales[row];
        } else {
            const uint8_t b = w[(size_t)row * ((columns + 1) / 2) + c / 2];
            const uint32_t n = (c & 1u) ? (b >> 4) : (b & 15u);
            wv = ((float)n - 8.0f) * scales[(size_t)row * scale_columns + c / group];
        }
        acc = __builtin_fmaf(wv, x[c], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

namespace {

template <uint32_t FMT, uint32_t R, uint32_t C>
hipError_t launch_st_rc(hipStream_t s, int cus, const uint8_t *w, uint32_t rows, uint32_t columns, size_t row_bytes,
                        const float *scales, uint32_t scale_columns, uint32_t group, const float *x, float *y) {
    const uint32_t lds = (columns / kStPerChunk<FMT>) * (kStPerChunk<FMT> + 4) * 4 + (FMT == kStI4 ? (columns / 16) * 4 : 0);
    static LdsLimit limit;
    hipError_t e = limit.ensure((const void *)st_gemv_kernel<FMT, R, C>, lds);
    if (e != hipSuccess) return e;
    const uint32_t groups = (rows + kStWaves * R - 1) / (kStWaves * R);
    const uint32_t cap = (uint32_t)(cus > 0 ? cus : 256) * 4;
    const uint32_t grid = groups < cap ? groups : cap;
    hipLaunchKernelGGL((st_gemv_kernel<FMT, R, C>), dim3(grid), dim3(64 * kStWaves), lds, s, w, rows, columns,
                       row_bytes, scales, scale_columns, group, x, y);
    return hipGetLastError();
}

template <uint32_t FMT>
hipError_t launch_st_t(hipStream_t s, int cus, const uint8_t *w, uint32_t rows, uint32_t columns, size_t row_bytes,
                       const float *scales, uint32_t scale_columns, uint32_t group, const float *x, float *y) {
    // (4 rows x 4 chunks for rows of at most 4 chunks per lane measured slower:
    // INT4 12288 x 6144 in 19.3 against 16.5 us, fewer workgroups; so did
    // 3 rows x 8 chunks for every format, e.g. INT4 18.0 against 16.3 us and
    // F8 18.7 against 17.0 us)
    return launch_st_rc<FMT, 2, 8>(s, cus, w, rows, columns, row_bytes, scales, scale_columns, group, x, y);
}

template <uint32_t FMT>
hipError_t launch_st_generic_t(hipStream_t s, const uint8_t *w, uint32_t rows, uint32_t columns, const float *scales,
                               uint32_t scale_columns, uint32_t group, const float *x, float *y) {
    hipLaunchKernelGGL((st_gemv_generic_kernel<FMT>), dim3((rows + 3) / 4), dim3(256), 0, s, w, rows, columns, scales,
                       scale_columns, group, x, y);
    return hipGetLastError();
}

}  // namespace

bool st_wide_supported(uint32_t fmt, size_t rows, size_t columns, size_t group, const void *w, const float *x) {
    if (rows == 0 || columns == 0 || columns > 16384 || rows >= (1u << 31)) return false;
    if (((uintptr_t)w & 15u) != 0 || ((uintptr_t)x & 15u) != 0) return false;
    switch (fmt) {
    case kStBf16: return columns % 8 == 0;
    case kStF8: case kStI8: return columns % 16 == 0;
    case kStI4: return columns % 32 == 0 && (group == 16 || group % 32 == 0);
    default: return false;
    }
}

hipError_t launch_st_gemv(hipStream_t s, int cus, uint32_t fmt, const void *w, uint32_t rows, uint32_t columns,
                          const float *scales, uint32_t scale_columns, uint32_t group, const float *x, float *y,
                          bool wide) {
    const uint8_t *wb = (const uint8_t *)w;
    if (wide) {
        const size_t row_bytes = fmt == kStBf16 ? (size_t)columns * 2 : fmt == kStI4 ? columns / 2 : columns;
        switch (fmt) {
        case kStBf16: return launch_st_t<kStBf16>(s, cus, wb, rows, columns, row_bytes, scales, scale_columns, group, x, y);
        case kStF8: return launch_st_t<kStF8>(s, cus, wb, rows, columns, row_bytes, scales, scale_columns, group, x, y);
        case kStI8: return launch_st_t<kStI8>(s, cus, wb, rows, columns, row_bytes, scales, scale_columns, group, x, y);
        default: return launch_st_t<kStI4>(s, cus, wb, rows, columns, row_bytes, scales, scale_columns, group, x, y);
        }
    }
    switch (fmt) {
    case kStBf16: return launch_st_generic_t<kStBf16>(s, wb, rows, columns, scales, scale_columns, group, x, y);
    case kStF8: return launch_st_generic_t<kStF8>(s, wb, rows, columns, scales, scale_columns, group, x, y);
    case kStI8: return launch_st_generic_t<kStI8>(s, wb, rows, columns, scales, scale_columns, group, x, y);
    default: return launch_st_generic_t<kStI4>(s, wb, rows, columns, scales, scale_columns, group, x, y);
    }
}

// A kernel of this file: resolving it loads the file's code object.
const void *module_anchor_safetensor() { return (const void *)st_gemv_kernel<kStBf16, 2, 8>; }

}  // namespace dm

// ---------------------------------------------------------------------------
// MetalContext::matvec_safetensor / matvec_safetensor_mapped (src/metal.rs:
// 738-1146): the same checks in the same order, then one launch.
// ---------------------------------------------------------------------------
#include "runtime.h"

#include <algorithm>

namespace dm {
namespace {

// SafeDtype (src/safetensors.rs:171-187), in declaration order.
enum : uint32_t {
    kSafeBool = 0, kSafeU8 = 1, kSafeI8 = 2, kSafeU16 = 3, kSafeI16 = 4, kSafeF16 = 5, kSafeBf16 = 6,
    kSafeU32 = 7, kSafeI32 = 8, kSafeF32 = 9, kSafeU64 = 10, kSafeI64 = 11, kSafeF64 = 12,
    kSafeF8E4M3 = 13, kSafeF8E5M2 = 14
};

int st_fail_bytes(const char *kind, size_t expected, size_t actual) {
    fail(DMHIP_ERR_INVALID_BYTE_LENGTH, "%s requires %zu encoded bytes, got %zu", kind, expected, actual);
    last_detail().kind = kind;
    last_detail().expected = expected;
    last_detail().actual = actual;
    return DMHIP_ERR_INVALID_BYTE_LENGTH;
}

int st_fail_unsupported(const char *kind) {
    fail(DMHIP_ERR_UNSUPPORTED_TENSOR_TYPE, "HIP matrix-vector multiplication does not support %s", kind);
    last_detail().kind = kind;
    return DMHIP_ERR_UNSUPPORTED_TENSOR_TYPE;
}

int st_overflow() { return fail(DMHIP_ERR_OVERFLOW, "matrix dimensions or encoded byte length overflowed"); }

bool mul_ovf(size_t a, size_t b, size_t *out) { return __builtin_mul_overflow(a, b, out); }

size_t sat_mul(size_t a, size_t b) {
    size_t r;
    return mul_ovf(a, b, &r) ? SIZE_MAX : r;
}

// u8_matrix_encoding (src/metal.rs:1893-1942).
int st_u8_encoding(size_t rows, size_t columns, size_t encoded_length, size_t scale_length, uint32_t *fmt,
                   size_t *group, size_t *scale_columns) {
    size_t int8_bytes, row_scale_bytes, int4_bytes;
    if (mul_ovf(rows, columns, &int8_bytes) || mul_ovf(rows, 4, &row_scale_bytes)) return st_overflow();
    if (encoded_length == int8_bytes && scale_length == row_scale_bytes) {
        *fmt = kStI8;
        *group = columns;
        *scale_columns = 1;
        return DMHIP_OK;
    }
    if (mul_ovf(rows, (columns + 1) / 2, &int4_bytes)) return st_overflow();
    if (encoded_length != int4_bytes) return st_fail_bytes("U8 quantized matrix", int4_bytes, encoded_length);
    *fmt = kStI4;
    if (scale_length == row_scale_bytes) {
        *group = std::max<size_t>(columns, 1);
        *scale_columns = 1;
        return DMHIP_OK;
    }
    for (size_t g : {16, 32, 48, 64, 96, 128, 192, 256}) {
        if (g > columns) break;
        const size_t sc = (columns + g - 1) / g;
        size_t want;
        if (mul_ovf(rows, sc, &want) || mul_ovf(want, 4, &want)) return st_overflow();
        if (scale_length == want) {
            *group = g;
            *scale_columns = sc;
            return DMHIP_OK;
        }
    }
    return st_fail_bytes("U8 quantization scales", row_scale_bytes, scale_length);
}

int st_mapped_range(const dmhip_buf *mapping, size_t offset, size_t length) {
    size_t end;
    if (__builtin_add_overflow(offset, length, &end)) return st_overflow();
    if (end > mapping->len) return fail_mapped_range(offset, end, mapping->len);
    return DMHIP_OK;
}

int st_count_u32(size_t n) {
    if (n > 0xffffffffull) return fail(DMHIP_ERR_VECTOR_TOO_LARGE, "HIP vector length exceeds the 32-bit kernel limit");
    return DMHIP_OK;
}

// Enqueues y = W x for a validated matrix on the context stream.  Scales not
// 4-byte aligned are first copied into aligned scratch.
int st_enqueue(dmhip_ctx *ctx, uint32_t fmt, size_t rows, size_t columns, const void *w, const float *scales,
               size_t scale_count, size_t group, size_t scale_columns, const float *x, float *y) {
    DM_CHECK_STATUS(st_count_u32(rows));
    DM_CHECK_STATUS(st_count_u32(columns));
    if (scales && ((uintptr_t)scales & 3u) != 0) {
        DM_CHECK_STATUS(ctx->aux.ensure(scale_count * 4));
        DM_HIP(hipMemcpyAsync(ctx->aux.ptr, scales, scale_count * 4, hipMemcpyDeviceToDevice, ctx->stream));
        scales = (const float *)ctx->aux.ptr;
    }
    const bool wide = st_wide_supported(fmt, rows, columns, group, w, x);
    DM_HIP(launch_st_gemv(ctx->stream, ctx->compute_units, fmt, w, (uint32_t)rows, (uint32_t)columns, scales,
                          (uint32_t)scale_columns, (uint32_t)std::min<size_t>(group, 0xffffffffu), x, y, wide));
    return DMHIP_OK;
}

// The host-slice (and device) form's checks: src/metal.rs:883-993 for BF16 /
// F8_E4M3FN, :1070-1146 for U8.  Fills the launch parameters; *empty when
// there are no rows (Ok without work).
int st_host_checks(uint32_t dtype, size_t rows, size_t columns, size_t encoded_len, const float *scales,
                   size_t scales_len, size_t input_len, size_t output_len, uint32_t *fmt, size_t *group,
                   size_t *scale_columns, size_t *scale_count, bool *empty) {
    *empty = false;
    if (dtype == kSafeU8) {
        if (input_len != columns) return fail_input_length(columns, input_len);
        if (output_len != rows) return fail_output_length(rows, output_len);
        if (!scales) return fail_vector_length("safetensors U8 matvec", "scales", rows, 0);
        size_t scale_length;
        if (mul_ovf(scales_len, 4, &scale_length)) return st_overflow();
        DM_CHECK_STATUS(st_u8_encoding(rows, columns, encoded_len, scale_length, fmt, group, scale_columns));
        *scale_count = scales_len;
        if (rows == 0) return *empty = true, DMHIP_OK;
        if (input_len == 0) return fail_empty("safetensors U8 matvec");
        return DMHIP_OK;
    }
    if (dtype != kSafeBf16 && dtype != kSafeF8E4M3) return st_fail_unsupported("safetensors dtype");
    if (input_len != columns) return fail_input_length(columns, input_len);
    if (output_len != rows) return fail_output_length(rows, output_len);
    const size_t width = dtype == kSafeBf16 ? 2 : 1;
    size_t expected;
    if (mul_ovf(rows, columns, &expected) || mul_ovf(expected, width, &expected)) return st_overflow();
    if (encoded_len != expected) return st_fail_bytes(dtype == kSafeBf16 ? "BF16" : "F8_E4M3FN", expected, encoded_len);
    if (rows == 0) return *empty = true, DMHIP_OK;
    if (input_len == 0) return fail_empty("safetensors matvec");
    *fmt = dtype == kSafeBf16 ? kStBf16 : kStF8;
    *group = 128;
    *scale_columns = (columns + 127) / 128;
    *scale_count = 0;
    if (dtype == kSafeF8E4M3) {
        size_t expected_scales;
        if (mul_ovf((rows + 127) / 128, *scale_columns, &expected_scales)) return st_overflow();
        if (!scales) return fail_vector_length("F8_E4M3FN matvec", "scales", expected_scales, 0);
        if (scales_len != expected_scales)
            return fail_vector_length("F8_E4M3FN matvec", "scales", expected_scales, scales_len);
        *scale_count = scales_len;
    }
    return DMHIP_OK;
}

}  // namespace
}  // namespace dm

using namespace dm;

#define DM_ST_REQUIRE(ptr)                                                               \
    do {                                                                                 \
        if (!(ptr)) return fail(DMHIP_ERR_INVALID_ARGUMENT, "%s must not be null", #ptr); \
    } while (0)

extern "C" {

int dmhip_matvec_safetensor_mapped(dmhip_ctx *ctx, uint32_t dtype, size_t rows, size_t columns,
                                   const dmhip_buf *mapping, size_t encoded_offset, size_t encoded_length,
                                   const dmhip_buf *scale_mapping, size_t scale_offset, size_t scale_length,
                                   const float *input, size_t input_len, float *output, size_t output_len) {
    DM_ST_REQUIRE(ctx);
    DM_ST_REQUIRE(mapping);
    if (dtype == kSafeF32 || dtype == kSafeF16)
        return dmhip_matvec_mapped(ctx, dtype == kSafeF32 ? 0 : 1, rows, columns, mapping, encoded_offset,
                                   encoded_length, input, input_len, output, output_len);
    uint32_t fmt = kStBf16;
    size_t group = 0, scale_columns = 0;
    if (dtype == kSafeU8) {
        // matvec_u8_mapped (src/metal.rs:995-1068)
        if (input_len != columns) return fail_input_length(columns, input_len);
        if (output_len != rows) return fail_output_length(rows, output_len);
        if (!scale_mapping) return st_fail_bytes("U8 quantization scales", sat_mul(rows, 4), 0);
        DM_CHECK_STATUS(st_u8_encoding(rows, columns, encoded_length, scale_length, &fmt, &group, &scale_columns));
        DM_CHECK_STATUS(st_mapped_range(mapping, encoded_offset, encoded_length));
        DM_CHECK_STATUS(st_mapped_range(scale_mapping, scale_offset, scale_length));
        if (rows == 0) return DMHIP_OK;
        if (input_len == 0) return fail_empty("safetensors U8 matvec");
    } else {
        if (dtype != kSafeBf16 && dtype != kSafeF8E4M3) return st_fail_unsupported("safetensors dtype");
        if (input_len != columns) return fail_input_length(columns, input_len);
        if (output_len != rows) return fail_output_length(rows, output_len);
        const size_t width = dtype == kSafeBf16 ? 2 : 1;
        size_t expected;
        if (mul_ovf(rows, columns, &expected) || mul_ovf(expected, width, &expected)) return st_overflow();
        if (encoded_length != expected)
            return st_fail_bytes(dtype == kSafeBf16 ? "BF16" : "F8_E4M3FN", expected, encoded_length);
        DM_CHECK_STATUS(st_mapped_range(mapping, encoded_offset, encoded_length));
        if (rows == 0) return DMHIP_OK;
        if (input_len == 0) return fail_empty("safetensors matvec");
        fmt = dtype == kSafeBf16 ? kStBf16 : kStF8;
        scale_columns = (columns + 127) / 128;
        group = 128;
        if (dtype == kSafeF8E4M3) {
            const size_t shown = sat_mul(sat_mul((rows + 127) / 128, scale_columns), 4);
            if (!scale_mapping) return st_fail_bytes("F8_E4M3FN scale", shown, 0);
            size_t expected_scale;
            if (mul_ovf((rows + 127) / 128, scale_columns, &expected_scale) || mul_ovf(expected_scale, 4, &expected_scale))
                return st_overflow();
            if (scale_length != expected_scale) return st_fail_bytes("F8_E4M3FN scale", expected_scale, scale_length);
            DM_CHECK_STATUS(st_mapped_range(scale_mapping, scale_offset, scale_length));
        }
    }
    DM_ST_REQUIRE(input);
    DM_ST_REQUIRE(output);
    DM_CHECK_STATUS(set_device(ctx));
    DM_CHECK_STATUS(ctx->in.ensure(columns * 4));
    DM_CHECK_STATUS(ctx->out.ensure(rows * 4));
    HostCall hc(ctx);
    DM_CHECK_STATUS(hc.begin(columns * 4 + rows * 4));
    DM_CHECK_STATUS(hc.in(ctx->in.ptr, input, columns * 4));
    const uint8_t *w = (const uint8_t *)mapping->dev + encoded_offset;
    const float *sc = fmt == kStBf16 ? nullptr : (const float *)((const uint8_t *)scale_mapping->dev + scale_offset);
    // the kernel writes y straight into the pinned bounce buffer
    float *o = (float *)hc.out_direct(output, rows * 4);
    DM_CHECK_STATUS(st_enqueue(ctx, fmt, rows, columns, w, sc, scale_length / 4, group, scale_columns,
                               (const float *)ctx->in.ptr, o ? o : (float *)ctx->out.ptr));
    if (!o) DM_CHECK_STATUS(hc.out(output, ctx->out.ptr, rows * 4));
    return hc.finish();
}

int dmhip_matvec_safetensor(dmhip_ctx *ctx, uint32_t dtype, size_t rows, size_t columns, const uint8_t *encoded,
                            size_t encoded_len, const float *scales, size_t scales_len, const float *input,
                            size_t input_len, float *output, size_t output_len) {
    DM_ST_REQUIRE(ctx);
    if (dtype == kSafeF32 || dtype == kSafeF16)
        return dmhip_matvec(ctx, dtype == kSafeF32 ? 0 : 1, rows, columns, encoded, encoded_len, input, input_len,
                            output, output_len);
    uint32_t fmt = kStBf16;
    size_t group = 0, scale_columns = 0, scale_count = 0;
    bool empty = false;
    DM_CHECK_STATUS(st_host_checks(dtype, rows, columns, encoded_len, scales, scales_len, input_len, output_len, &fmt,
                                   &group, &scale_columns, &scale_count, &empty));
    if (empty) return DMHIP_OK;
    DM_ST_REQUIRE(encoded);
    DM_ST_REQUIRE(input);
    DM_ST_REQUIRE(output);
    DM_CHECK_STATUS(set_device(ctx));
    const size_t enc_span = (encoded_len + 255) & ~(size_t)255;
    DM_CHECK_STATUS(ctx->enc.ensure(enc_span + scale_count * 4));
    DM_CHECK_STATUS(ctx->in.ensure(columns * 4));
    DM_CHECK_STATUS(ctx->out.ensure(rows * 4));
    uint8_t *dw = (uint8_t *)ctx->enc.ptr;
    float *ds = scale_count ? (float *)(dw + enc_span) : nullptr;
    DM_HIP(hipMemcpyAsync(dw, encoded, encoded_len, hipMemcpyHostToDevice, ctx->stream));
    if (scale_count) DM_HIP(hipMemcpyAsync(ds, scales, scale_count * 4, hipMemcpyHostToDevice, ctx->stream));
    DM_HIP(hipMemcpyAsync(ctx->in.ptr, input, columns * 4, hipMemcpyHostToDevice, ctx->stream));
    DM_CHECK_STATUS(st_enqueue(ctx, fmt, rows, columns, dw, ds, scale_count, group, scale_columns,
                               (const float *)ctx->in.ptr, (float *)ctx->out.ptr));
    DM_HIP(hipMemcpyAsync(output, ctx->out.ptr, rows * 4, hipMemcpyDeviceToHost, ctx->stream));
    DM_HIP(hipStreamSynchronize(ctx->stream));  // a copy into pageable memory precedes
    return DMHIP_OK;
}

int dmhip_matvec_safetensor_device(dmhip_ctx *ctx, uint32_t dtype, size_t rows, size_t columns, const void *weights,
                                   size_t weights_len, const float *scales, size_t scales_len, const float *x,
                                   float *y) {
    DM_ST_REQUIRE(ctx);
    if (dtype == kSafeF32 || dtype == kSafeF16) {
        const uint32_t type = dtype == kSafeF32 ? 0 : 1;
        size_t expected;
        if (mul_ovf(rows, columns, &expected) || mul_ovf(expected, type == 0 ? 4 : 2, &expected))
            return st_overflow();
        if (weights_len != expected) return fail_byte_length(type, expected, weights_len);
        return dmhip_matvec_device(ctx, type, rows, columns, weights, 1, x, y);
    }
    uint32_t fmt = kStBf16;
    size_t group = 0, scale_columns = 0, scale_count = 0;
    bool empty = false;
    DM_CHECK_STATUS(st_host_checks(dtype, rows, columns, weights_len, scales, scales_len, columns, rows, &fmt, &group,
                                   &scale_columns, &scale_count, &empty));
    if (empty) return DMHIP_OK;
    DM_ST_REQUIRE(weights);
    DM_ST_REQUIRE(x);
    DM_ST_REQUIRE(y);
    DM_CHECK_STATUS(set_device(ctx));
    return st_enqueue(ctx, fmt, rows, columns, weights, scale_count ? scales : nullptr, scale_count, group,
                      scale_columns, x, y);
}

}  // extern "C"
