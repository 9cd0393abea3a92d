// kernels_qmv.hip -- MFMA quantized matvec for gfx950 (decode, batch 1..16).
//
// y[b][r] = sum_c W[r][c] * x[b][c] for Q4_K / Q6_K rows (src/cpu.rs:345-399
// semantics, fp32 accumulation).
//
// Operands of v_mfma_f32_16x16x32_f16, all exact:
//  * B (weights): 16 rows x 32 columns per step.  Each weight enters as the
//    fp16 integer sc*q (Q4_K: 0..945) or sc*(q-32) (Q6_K: |.| <= 1984 when
//    |sc| <= 62), built from the packed bits with the "1024 + q" exponent
//    trick and one packed fp16 FMA (exact: the result is representable and
//    the FMA rounds once).  The super-block scale d (and dmin) multiply the
//    fp32 block result afterwards.  Q6_K blocks with a larger |sc| split the
//    scale into 8*sh + sl and run two exact MFMAs.
//  * A (activations): 16 rows = 8 tokens x {hi, lo}.  Each token is scaled
//    by a power of two so |x| < 2^15, then x = hi + lo with hi, lo fp16
//    (22 significant bits).  Products are exact; MFMA accumulates in fp32.
//  * Q4_K's "- dmin * m * x" term is a ninth MFMA step per block whose B
//    column carries 64*m and whose A row carries the sub-block sums of x
//    (scaled by 2^-6, hi/lo), accumulated separately and scaled by dmin.
//
// Lanes: n = lane & 15 is the weight row within a 16-row tile (B column)
// and the A row; kg = lane >> 4 picks which quarter of each 32-column step
// the lane supplies.  C[m][n] sits in lane n + 16*(m/4), element m%4, so
// lane (n, g4) accumulates tokens 2*g4 and 2*g4+1 of row n.
//
// Data movement: a wave stages G = 2 consecutive blocks of each of its row
// tiles in its own LDS area with contiguous 16-byte loads (out-of-range rows
// read zero), the next group in flight while the current one is computed,
// and every lane takes its pieces from there.  For batch 1-2 the activation
// fragments of the whole row are staged once per workgroup in LDS and read
// with ds_read_b128; for larger batches they come from L2, the next block's
// while a block is computed.  Short matrices split K over up to 8 waves of a
// workgroup.
#include "dm_device.h"
#include "dm_qmv.h"


namespace dm {

namespace {

constexpr uint32_t kBias16 = 0x64006400u;    // fp16 pair (1024, 1024)
constexpr uint32_t kBiasBytes = 0x64646464u;  // source of the 0x64 high bytes

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

__device__ __forceinline__ half2_t h2_fma(half2_t a, half2_t b, half2_t c) {
    return __builtin_elementwise_fma(a, b, c);
}

// (v, v) as fp16 from a small integer (exact: |v| < 2048).
__device__ __forceinline__ half2_t h2_int(int v) {
    const _Float16 h = (_Float16)(short)v;
    half2_t r;
    r[0] = h;
    r[1] = h;
    return r;
}

__device__ __forceinline__ half2_t h2_splat(float v) {
    half2_t h;
    h[0] = (_Float16)v;
    h[1] = (_Float16)v;
    return h;
}

__device__ __forceinline__ float f16_lo(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
}

__device__ __forceinline__ floatx4 mfma(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8 frag(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4 v = {a, b, c, d};
    return __builtin_bit_cast(half8, v);
}

// Steps of 32 columns per 256-column block, including Q4_K's min step.
template <uint32_t TYPE> struct Steps;
template <> struct Steps<kQ4_K> { static constexpr uint32_t value = 9; };
template <> struct Steps<kQ6_K> { static constexpr uint32_t value = 8; };

// Column (0..255) of a block that fragment position j of lane-group kg
// carries at step t (t < 8).
template <uint32_t TYPE>
__device__ __forceinline__ uint32_t fragment_column(uint32_t kg, uint32_t t, uint32_t j) {
    const uint32_t perm = (j & 3u) == 1 ? 2u : ((j & 3u) == 2 ? 1u : (j & 3u));
    if (TYPE == kQ4_K) return 64 * kg + 32 * (j >> 2) + 4 * t + perm;
    // Q6_K: kg = 2h + c; k = t >> 1; dw = 2 * (t & 1) + (j >> 2).
    const uint32_t h = kg >> 1, c = kg & 1u, k = t >> 1, dw = 2 * (t & 1u) + (j >> 2);
    return 128 * h + 32 * k + 16 * c + 4 * dw + perm;
}

// Power-of-two exponent e with max|x| * 2^-e in [2^14, 2^15) (0 for an
// all-zero or non-finite row, whose result is then non-finite anyway).
__device__ __forceinline__ int token_exponent(float mx) {
    int e = 0;
    if (mx > 0.0f && __builtin_isfinite(mx)) {
        int ex;
        (void)frexpf(mx, &ex);  // mx = f * 2^ex, f in [0.5, 1)
        e = ex - 15;
        if (e < -126) e = -126;
        if (e > 127) e = 127;
    }
    return e;
}

// The hi/lo fp16 halves of fragment (blk, t, kg) of one token row `xt`
// scaled by `down` (a power of two).
template <uint32_t TYPE>
__device__ __forceinline__ void build_fragment(const float *xt, uint32_t blk, uint32_t t, uint32_t kg,
                                               float down, half8 &hi, half8 &lo) {
    const float *xb = xt + (size_t)blk * 256;
    // the halves are gathered in scalars and the vectors built once (element
    // inserts across the branch put the vectors in private memory)
    _Float16 h[8], l[8];
    if (TYPE == kQ4_K && t == 8) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const float *sb = xb + 32 * (2 * kg + j);
            float q[32];
#pragma unroll
            for (int i = 0; i < 32; i++) q[i] = sb[i];  // every read issued before the sum
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++) s += q[i] * down;
            s = s * 0.015625f;  // 2^-6 keeps |sum| inside fp16
            h[j] = (_Float16)s;
            l[j] = (_Float16)(s - (float)h[j]);
        }
#pragma unroll
        for (int j = 2; j < 8; j++) h[j] = l[j] = (_Float16)0.0f;
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float v = xb[fragment_column<TYPE>(kg, t, j)] * down;
            h[j] = (_Float16)v;
            l[j] = (_Float16)(v - (float)h[j]);
        }
    }
    hi = half8{h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]};
    lo = half8{l[0], l[1], l[2], l[3], l[4], l[5], l[6], l[7]};
}

}  // namespace

// ---------------------------------------------------------------------------
// Activation preparation: per token a power-of-two scale 2^-e with
// max|x| * 2^-e in [2^14, 2^15), the hi/lo fp16 fragments in step order,
// and (Q4_K) the 32-column sums.  yscale[t] = 2^e (times the RMSNorm factor
// when `normalize`).  Grid: (blocks of fragments, tokens).
// ---------------------------------------------------------------------------
// With STAGED the token row is copied into LDS (columns <= kPrepareLdsColumns)
// and the fragments are built from there; the row is read from global memory
// once, every load of a thread in flight at once (16-byte loads when the row
// is 16-byte aligned).  The 32-column sums of Q4_K issue all their LDS reads
// before the sequential sum (measured at C3, 4 tokens: 48.5 -> 46.3 us per
// layer against one read in flight at a time).
constexpr uint32_t kPrepareLdsColumns = 16384;

template <uint32_t TYPE, bool STAGED>
__global__ void __launch_bounds__(256) qmv_prepare_kernel(const float *__restrict__ x,
                                                          uint32_t columns, uint32_t batch,
                                                          int normalize, float epsilon,
                                                          _Float16 *__restrict__ xp,
                                                          float *__restrict__ yscale) {
    constexpr uint32_t SPB = Steps<TYPE>::value;
    constexpr uint32_t U = 16;
    extern __shared__ float s_row[];
    __shared__ float red_max[4], red_ss[4];
    const uint32_t token = blockIdx.y;
    const float *xt = x + (size_t)token * columns;
    float mx = 0.0f, ss = 0.0f;
    if (STAGED && ((uintptr_t)xt & 15u) == 0) {
        // 16-byte loads, every one in flight at once (columns <= 16384 is 16 per thread)
        const uint32_t n4 = columns / 4;
        floatx4 v[U];
#pragma unroll
        for (uint32_t j = 0; j < U; j++) {
            const uint32_t i = 256 * j + threadIdx.x;
            v[j] = i < n4 ? ((const floatx4 *)xt)[i] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (uint32_t j = 0; j < U; j++) {
            const uint32_t i = 256 * j + threadIdx.x;
            if (i < n4) ((floatx4 *)s_row)[i] = v[j];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                mx = fmaxf(mx, fabsf(v[j][e]));
                ss = __builtin_fmaf(v[j][e], v[j][e], ss);
            }
        }
    } else
    for (uint32_t i0 = 0; i0 < columns; i0 += 256 * U) {
        float v[U];
#pragma unroll
        for (uint32_t j = 0; j < U; j++) {
            const uint32_t i = i0 + 256 * j + threadIdx.x;
            v[j] = i < columns ? xt[i] : 0.0f;
        }
#pragma unroll
        for (uint32_t j = 0; j < U; j++) {
            const uint32_t i = i0 + 256 * j + threadIdx.x;
            if (STAGED && i < columns) s_row[i] = v[j];
            mx = fmaxf(mx, fabsf(v[j]));
            ss = __builtin_fmaf(v[j], v[j], ss);
        }
    }
    mx = wave_max(mx);
    ss = wave_sum(ss);
    if ((threadIdx.x & 63u) == 0) {
        red_max[threadIdx.x >> 6] = mx;
        red_ss[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    mx = fmaxf(fmaxf(red_max[0], red_max[1]), fmaxf(red_max[2], red_max[3]));
    ss = red_ss[0] + red_ss[1] + red_ss[2] + red_ss[3];
    const int e = token_exponent(mx);
    const float down = ldexpf(1.0f, -e);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        float up = ldexpf(1.0f, e);
        if (normalize) up = up * (1.0f / __builtin_sqrtf(ss / (float)columns + epsilon));
        yscale[token] = up;
    }
    // One fragment (8 halves) per thread: fragment f = ((blk*SPB + t)*4 + kg).
    const uint32_t blocks = columns / 256;
    const uint32_t m2 = 2 * batch;
    const uint32_t fragments = blocks * SPB * 4;
    half8 *dst = (half8 *)xp;
    for (uint32_t f = blockIdx.x * blockDim.x + threadIdx.x; f < fragments;
         f += gridDim.x * blockDim.x) {
        const uint32_t kg = f & 3u, t = (f >> 2) % SPB, blk = (f >> 2) / SPB;
        half8 hi, lo;
        build_fragment<TYPE>(STAGED ? s_row : xt, blk, t, kg, down, hi, lo);
        dst[(size_t)f * m2 + 2 * token] = hi;
        dst[(size_t)f * m2 + 2 * token + 1] = lo;
    }
}

// ---------------------------------------------------------------------------
// Raw bytes of one block of one row as a lane holds them, and the block's
// contribution to the lane's accumulators.
// ---------------------------------------------------------------------------
template <uint32_t TYPE> struct Raw;
template <> struct Raw<kQ4_K> {
    u32x4 hdr, q0, q1;  // d|dmin|scales, then qs bytes [32kg, 32kg+32)
};
template <> struct Raw<kQ6_K> {
    u32x4 a1, a2, a3, a4;          // aligned dwords under ql/ql+32/qh/scales
    uint32_t e1, e2, e3, e4, e4b;  // the dword after each (for the byte shift)
    uint32_t s;                    // block start mod 4
};

template <int NT>
__device__ __forceinline__ void block_dot(const Raw<kQ4_K> &raw, const half8 (&a)[9][NT], uint32_t kg,
                                          float (&acc)[NT][2]) {
    const u32x4 hdr = raw.hdr;
    const float dscale = f16_lo(hdr[0]);
    const float mscale = f16_lo(hdr[0] >> 16);
    // (scale, min) of sub-blocks 2kg and 2kg+1 (src/cpu.rs:607-616): for
    // sub-block j < 4 the low 6 bits of scales[j], scales[j+4]; for j >= 4
    // nibbles of scales[j+4] with the top bits of scales[j-4], scales[j].
    const bool high_half = kg >= 2;
    uint32_t sc[2], mn[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t sh = 8 * ((2 * kg + j) & 3u);
        const uint32_t b1 = hdr[1] >> sh, b2 = hdr[2] >> sh, b3 = hdr[3] >> sh;
        const uint32_t sc_lo = b1 & 63u, mn_lo = b2 & 63u;
        const uint32_t sc_hi = (b3 & 15u) | ((b1 >> 2) & 0x30u);
        const uint32_t mn_hi = ((b3 >> 4) & 15u) | ((b2 >> 2) & 0x30u);
        sc[j] = high_half ? sc_hi : sc_lo;
        mn[j] = high_half ? mn_hi : mn_lo;
    }
    const half2_t sl = h2_int((int)sc[0]);
    const half2_t bl = sl * h2_splat(-1024.0f);
    const half2_t shi = h2_int((int)sc[1]);
    const half2_t sh = shi * h2_splat(0.0625f);
    const half2_t bh = shi * h2_splat(-64.0f);
    floatx4 cm[NT];
#pragma unroll
    for (int g = 0; g < NT; g++) cm[g] = floatx4{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const uint32_t d = t < 4 ? raw.q0[t] : raw.q1[t - 4];
        const uint32_t d8 = d >> 8;
        const uint32_t p0 = as_u(h2_fma(as_h2((d & 0x000f000fu) | kBias16), sl, bl));
        const uint32_t p1 = as_u(h2_fma(as_h2((d8 & 0x000f000fu) | kBias16), sl, bl));
        const uint32_t p2 = as_u(h2_fma(as_h2((d & 0x00f000f0u) | kBias16), sh, bh));
        const uint32_t p3 = as_u(h2_fma(as_h2((d8 & 0x00f000f0u) | kBias16), sh, bh));
        const half8 b = frag(p0, p1, p2, p3);
#pragma unroll
        for (int g = 0; g < NT; g++) cm[g] = mfma(a[t][g], b, cm[g]);
    }
    // min step: B = (64 m_lo, 64 m_hi, 0...), A = sub-block sums * 2^-6.
    const uint32_t mm = (as_u(h2_int((int)(64 * mn[0]))) & 0xffffu) |
                        (as_u(h2_int((int)(64 * mn[1]))) << 16);
    const half8 bmin = frag(mm, 0u, 0u, 0u);
#pragma unroll
    for (int g = 0; g < NT; g++) {
        const floatx4 cmin = mfma(a[8][g], bmin, floatx4{0, 0, 0, 0});
        acc[g][0] = __builtin_fmaf(dscale, cm[g][0] + cm[g][1], acc[g][0]);
        acc[g][0] = __builtin_fmaf(-mscale, cmin[0] + cmin[1], acc[g][0]);
        acc[g][1] = __builtin_fmaf(dscale, cm[g][2] + cm[g][3], acc[g][1]);
        acc[g][1] = __builtin_fmaf(-mscale, cmin[2] + cmin[3], acc[g][1]);
    }
}

template <int NT>
__device__ __forceinline__ void block_dot(const Raw<kQ6_K> &raw, const half8 (&a)[8][NT], uint32_t kg,
                                          float (&acc)[NT][2]) {
    const uint32_t s = raw.s;
    uint32_t L1[4], L2[4], H[4], T[5];
    if (__builtin_amdgcn_ballot_w64(s != 0) == 0) {
        // every row of the tile starts this block on a dword boundary
#pragma unroll
        for (int i = 0; i < 4; i++) {
            L1[i] = raw.a1[i];
            L2[i] = raw.a2[i];
            H[i] = raw.a3[i];
            T[i] = raw.a4[i];
        }
        T[4] = raw.e4;
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            L1[i] = funnel(raw.a1[i], i < 3 ? raw.a1[i + 1] : raw.e1, s);
            L2[i] = funnel(raw.a2[i], i < 3 ? raw.a2[i + 1] : raw.e2, s);
            H[i] = funnel(raw.a3[i], i < 3 ? raw.a3[i + 1] : raw.e3, s);
            T[i] = funnel(raw.a4[i], i < 3 ? raw.a4[i + 1] : raw.e4, s);
        }
        T[4] = funnel(raw.e4, raw.e4b, s);
    }
    const float dscale = f16_lo(T[4]);
    // int8 scales sc[8h + 2k + c], k = 0..3: bytes c and c+2 of scale words
    // 2h (k = 0, 1) and 2h+1 (k = 2, 3).
    const uint32_t h = kg >> 1, c = kg & 1u;
    const uint32_t w01 = h ? T[2] : T[0], w23 = h ? T[3] : T[1];
    int sck[4];
    sck[0] = (int)(int8_t)(w01 >> (8 * c));
    sck[1] = (int)(int8_t)(w01 >> (8 * c + 16));
    sck[2] = (int)(int8_t)(w23 >> (8 * c));
    sck[3] = (int)(int8_t)(w23 >> (8 * c + 16));
    bool fast = true;
#pragma unroll
    for (int k = 0; k < 4; k++) fast = fast && sck[k] <= 62 && sck[k] >= -62;
    const bool all_fast = __builtin_amdgcn_ballot_w64(!fast) == 0;
    floatx4 cm[NT];
#pragma unroll
    for (int g = 0; g < NT; g++) cm[g] = floatx4{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const int k = t >> 1;
        uint32_t pr[4];
#pragma unroll
        for (int half_dw = 0; half_dw < 2; half_dw++) {
            const int dw = 2 * (t & 1) + half_dw;
            const uint32_t src = (k & 1) ? L2[dw] : L1[dw];
            const uint32_t nib = (k & 2) ? (src >> 4) : src;
            // bits 2k..2k+1 of each qh byte moved to bits 4..5
            const uint32_t hsh = k == 0 ? H[dw] << 4 : (k == 1 ? H[dw] << 2 : (k == 2 ? H[dw] : H[dw] >> 2));
            const uint32_t q4 = (nib & 0x0f0f0f0fu) | (hsh & 0x30303030u);  // four 6-bit q
            // fp16 pairs (1024 + q) of bytes (0, 2) and (1, 3)
            pr[2 * half_dw] = __builtin_amdgcn_perm(q4, kBiasBytes, 0x00060004u);
            pr[2 * half_dw + 1] = __builtin_amdgcn_perm(q4, kBiasBytes, 0x00070005u);
        }
        if (all_fast) {
            const half2_t scl = h2_int(sck[k]);
            const half2_t bias = scl * h2_splat(-1056.0f);
            const half8 b = frag(as_u(h2_fma(as_h2(pr[0]), scl, bias)), as_u(h2_fma(as_h2(pr[1]), scl, bias)),
                                 as_u(h2_fma(as_h2(pr[2]), scl, bias)), as_u(h2_fma(as_h2(pr[3]), scl, bias)));
#pragma unroll
            for (int g = 0; g < NT; g++) cm[g] = mfma(a[t][g], b, cm[g]);
        } else {
            // sc = 8*sh + sl, sl in 0..7: both products exact in fp16.
            const int shi = sck[k] >> 3, slo = sck[k] & 7;
            const half2_t off = h2_splat(-1056.0f);
            const half2_t one = h2_splat(1.0f);
            const half2_t f_hi = h2_int(8 * shi);
            const half2_t f_lo = h2_int(slo);
            half2_t qm[4];
#pragma unroll
            for (int i = 0; i < 4; i++) qm[i] = h2_fma(as_h2(pr[i]), one, off);  // q - 32
            const half8 b_hi = frag(as_u(qm[0] * f_hi), as_u(qm[1] * f_hi), as_u(qm[2] * f_hi),
                                    as_u(qm[3] * f_hi));
            const half8 b_lo = frag(as_u(qm[0] * f_lo), as_u(qm[1] * f_lo), as_u(qm[2] * f_lo),
                                    as_u(qm[3] * f_lo));
#pragma unroll
            for (int g = 0; g < NT; g++) {
                cm[g] = mfma(a[t][g], b_hi, cm[g]);
                cm[g] = mfma(a[t][g], b_lo, cm[g]);
            }
        }
    }
#pragma unroll
    for (int g = 0; g < NT; g++) {
        acc[g][0] = __builtin_fmaf(dscale, cm[g][0] + cm[g][1], acc[g][0]);
        acc[g][1] = __builtin_fmaf(dscale, cm[g][2] + cm[g][3], acc[g][1]);
    }
}

// ---------------------------------------------------------------------------
// Weight staging.  A wave fetches G consecutive blocks of each of its 16-row
// tiles as whole 16-byte chunks (row r of the tile: `chunks` chunks from the
// dword at or below its first block; Q4_K runs start 16-aligned), consecutive
// lanes on consecutive chunks of a row, and parks them in its own LDS area;
// each lane then takes its operand pieces from there.  Every load
// instruction covers a few long runs of rows instead of 16 rows' separate
// 16-byte pieces.
// ---------------------------------------------------------------------------
typedef uint32_t v4u __attribute__((ext_vector_type(4)));  // 16-byte aligned (LDS)

template <uint32_t TYPE, uint32_t G> struct StageQ {
    static constexpr uint32_t chunks = TYPE == kQ4_K ? 9 * G : (210 * G + 2 + 15) / 16;
    static constexpr uint32_t items = 16 * chunks;        // chunks of one tile
    static constexpr uint32_t loads = (items + 63) / 64;  // 16-byte loads per lane
};

// Lane (n, kg)'s raw bytes of the block at byte `off` of row n's run.
__device__ __forceinline__ void take_raw(const v4u *stage, uint32_t ch, uint32_t n, uint32_t kg, uint32_t off,
                                         Raw<kQ4_K> &raw) {
    const v4u *sr = stage + n * ch + off / 16;
    raw.hdr = __builtin_bit_cast(u32x4, sr[0]);
    raw.q0 = __builtin_bit_cast(u32x4, sr[1 + 2 * kg]);
    raw.q1 = __builtin_bit_cast(u32x4, sr[2 + 2 * kg]);
}

__device__ __forceinline__ void take_raw(const v4u *stage, uint32_t ch, uint32_t n, uint32_t kg, uint32_t off,
                                         Raw<kQ6_K> &raw) {
    // dwords of row n from the one holding the block's first byte
    const uint32_t *sw = (const uint32_t *)(stage + n * ch) + (off >> 2);
    const uint32_t h = kg >> 1, c = kg & 1u;
    const uint32_t o1 = 16 * h + 4 * c, o2 = o1 + 8, o3 = 32 + 8 * h + 4 * c;
    raw.s = off & 3u;
    raw.a1 = u32x4{sw[o1], sw[o1 + 1], sw[o1 + 2], sw[o1 + 3]};
    raw.a2 = u32x4{sw[o2], sw[o2 + 1], sw[o2 + 2], sw[o2 + 3]};
    raw.a3 = u32x4{sw[o3], sw[o3 + 1], sw[o3 + 2], sw[o3 + 3]};
    raw.a4 = u32x4{sw[48], sw[49], sw[50], sw[51]};
    raw.e1 = sw[o1 + 4];
    raw.e2 = sw[o2 + 4];
    raw.e3 = sw[o3 + 4];
    raw.e4 = sw[52];
    raw.e4b = sw[53];
}

// ---------------------------------------------------------------------------
// Main kernel.  A workgroup has 4 waves; S waves split one group of R row
// tiles along K, so a workgroup covers (4/S)*R tiles of 16 rows.
// MB > 0: the activation fragments (MB = 2*batch rows) live in LDS.
// MODE 0: y = W x.  MODE 1: also a per-wave argmax candidate.  MODE 2:
// gate/up pair, act = silu(gate) * up.
// ---------------------------------------------------------------------------
template <uint32_t TYPE, int NT, int R, int S, int MODE, int MB, uint32_t G>
__global__ void __launch_bounds__(64 * (S > 4 ? S : 4)) qmv_kernel(
    const uint8_t *__restrict__ w, const uint8_t *__restrict__ w2, uint32_t rows,
    uint32_t columns, uint32_t row_bytes, uint32_t total_bytes, const float *__restrict__ x,
    int normalize, float epsilon, const _Float16 *__restrict__ xp,
    const float *__restrict__ yscale_global, uint32_t batch, float *__restrict__ y,
    ArgmaxPartial *__restrict__ partials) {
    constexpr uint32_t SPB = Steps<TYPE>::value;
    constexpr uint32_t BB = TYPE == kQ4_K ? 144u : 210u;
    constexpr int RR = MODE == 2 ? 2 * R : R;  // gate/up: R tiles of each matrix
    constexpr uint32_t WAVES = S > 4 ? S : 4;
    __shared__ float partial[S > 1 ? WAVES * RR * NT * 64 * 2 : 1];
    __shared__ float token_scale[2][4];
    extern __shared__ half8 lds_a[];

    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 15u, kg = lane >> 4;
    const uint32_t group = wave / S, kpart = wave % S;
    const uint32_t first_tile = (blockIdx.x * (WAVES / S) + group) * R;
    const uint32_t blocks = columns / 256;
    const uint32_t groups = (blocks + G - 1) / G;
    const uint32_t g_begin = kpart * groups / S, g_end = (kpart + 1) * groups / S;
    const uint32_t m2 = 2 * batch;
    const float *yscale = yscale_global;

    // Lanes whose A row carries no token read a zeroed copy of one block's
    // fragments, so every lane runs the same loads.
    const half8 *a_lane = nullptr;
    uint32_t a_block_stride = 0;
    if constexpr (MB > 0) {
        // Copy every activation fragment of the row (written by the
        // preparation kernel) into LDS, followed by one zeroed block.
        const uint32_t count = blocks * SPB * 4 * MB;
        const half8 *src = (const half8 *)xp;
        for (uint32_t i = threadIdx.x; i < count; i += 64 * WAVES) lds_a[i] = src[i];
        for (uint32_t i = threadIdx.x; i < SPB * 4 * MB; i += 64 * WAVES)
            lds_a[count + i] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        if (threadIdx.x < MB / 2) token_scale[threadIdx.x][0] = yscale_global[threadIdx.x];
        __syncthreads();
        a_lane = n < (uint32_t)MB ? lds_a + kg * MB + n : lds_a + count + kg * MB;
        a_block_stride = n < (uint32_t)MB ? SPB * 4 * MB : 0;
    }

    // Whole dwords: the last dword of the matrix may extend up to 3 bytes past
    // its end (inside the allocation's granularity); loads beyond it read 0.
    const uint32_t records = (total_bytes + 3u) & ~3u;
    const uint32_t nowhere = records + 256;  // every load from here reads 0
    const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(w, records);
    const __amdgpu_buffer_rsrc_t rsrc2 = make_rsrc(MODE == 2 ? w2 : w, records);

    float acc[RR][NT][2];
#pragma unroll
    for (int r = 0; r < RR; r++)
#pragma unroll
        for (int g = 0; g < NT; g++) acc[r][g][0] = acc[r][g][1] = 0.0f;

    // Row of tile r handled by this lane (may be >= rows: loads return 0).
    uint32_t row_base[RR];
#pragma unroll
    for (int r = 0; r < RR; r++) {
        const uint32_t tile = first_tile + (MODE == 2 ? r % R : r);
        const uint32_t row = tile * 16 + n;
        row_base[r] = row < rows ? row * row_bytes : nowhere;
    }

    // Staging: the wave's area holds RR tiles of ITEMS chunks; load j of
    // this lane is chunk src_chunk[j] of row (item / CH) of each tile.
    using ST = StageQ<TYPE, G>;
    constexpr uint32_t CH = ST::chunks, NL = ST::loads, ITEMS = ST::items;
    const size_t a_bytes = MB > 0 ? ((size_t)blocks + 1) * SPB * 4 * MB * 16 : 0;
    v4u *stage = (v4u *)((uint8_t *)lds_a + a_bytes) + (size_t)wave * RR * ITEMS;
    uint32_t src_row[RR][NL], src_chunk[NL];
#pragma unroll
    for (uint32_t j = 0; j < NL; j++) {
        const uint32_t item = j * 64 + lane, ri = item / CH;
        src_chunk[j] = 16 * (item - ri * CH);
#pragma unroll
        for (int r = 0; r < RR; r++) {
            const uint32_t row = (first_tile + (MODE == 2 ? r % R : r)) * 16 + ri;
            src_row[r][j] = (item < ITEMS && row < rows) ? row * row_bytes : nowhere;
        }
    }
    v4u st[RR][NL];
    auto fetch = [&](uint32_t grp) {
#pragma unroll
        for (int r = 0; r < RR; r++)
#pragma unroll
            for (uint32_t j = 0; j < NL; j++) {
                const uint32_t off =
                    src_row[r][j] == nowhere ? nowhere : ((src_row[r][j] + grp * G * BB) & ~3u) + src_chunk[j];
                st[r][j] = __builtin_bit_cast(v4u, rsrc_load16((MODE == 2 && r >= R) ? rsrc2 : rsrc, off));
            }
    };
    // A wave reads only its own area and its LDS operations run in order; the
    // wavefront-scope fences keep the compiler from moving another lane's
    // reads across these writes.
    auto put = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int r = 0; r < RR; r++)
#pragma unroll
            for (uint32_t j = 0; j < NL; j++)
                if (j + 1 < NL || j * 64 + lane < ITEMS) stage[r * ITEMS + j * 64 + lane] = st[r][j];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    };
    // Activation fragments of block blk (from LDS, or from the prepared
    // fragments in global memory one block ahead of their use).
    auto load_a = [&](uint32_t blk, half8 (&a)[SPB][NT]) {
#pragma unroll
        for (int t = 0; t < (int)SPB; t++)
#pragma unroll
            for (int g = 0; g < NT; g++) {
                const uint32_t m = 16 * g + n;
                if constexpr (MB > 0) {
                    // one address per block, then immediate offsets per step
                    a[t][g] = a_lane[blk * a_block_stride + t * 4 * MB];
                } else if (m < m2) {
                    const size_t f = ((size_t)blk * SPB + t) * 4 + kg;
                    a[t][g] = *(const half8 *)(xp + (f * m2 + m) * 8);
                } else {
                    a[t][g] = half8{0, 0, 0, 0, 0, 0, 0, 0};
                }
            }
    };

    // The loads of group g+1 are in flight while group g is computed, and
    // the activation fragments of the next block while a block is computed.
    if (g_begin < g_end) {
        const uint32_t blk_end = g_end * G < blocks ? g_end * G : blocks;
        half8 a[SPB][NT];
        load_a(g_begin * G, a);
        fetch(g_begin);
        for (uint32_t grp = g_begin; grp < g_end; grp++) {
            put();
            if (grp + 1 < g_end) fetch(grp + 1);
#pragma unroll
            for (uint32_t b = 0; b < G; b++) {
                const uint32_t blk = grp * G + b;
                if (blk >= blk_end) break;
                half8 a_next[SPB][NT];
                if (blk + 1 < blk_end) load_a(blk + 1, a_next);
                Raw<TYPE> raw[RR];
#pragma unroll
                for (int r = 0; r < RR; r++) {
                    // the run of row n starts 0 or 2 bytes into its first dword (Q6_K)
                    const uint32_t s0 = row_base[r] == nowhere ? 0u : ((row_base[r] + grp * G * BB) & 3u);
                    take_raw(stage + r * ITEMS, CH, n, kg, s0 + b * BB, raw[r]);
                }
#pragma unroll
                for (int r = 0; r < RR; r++) block_dot<NT>(raw[r], a, kg, acc[r]);
                if (blk + 1 < blk_end) {
#pragma unroll
                    for (int t = 0; t < (int)SPB; t++)
#pragma unroll
                        for (int g = 0; g < NT; g++) a[t][g] = a_next[t][g];
                }
            }
        }
    }

    // --- split-K reduction through LDS --------------------------------------
    if constexpr (S > 1) {
#pragma unroll
        for (int r = 0; r < RR; r++)
#pragma unroll
            for (int g = 0; g < NT; g++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    partial[((((wave * RR + r) * NT + g) * 64) + lane) * 2 + j] = acc[r][g][j];
        __syncthreads();
        if (kpart != 0) return;
#pragma unroll
        for (int r = 0; r < RR; r++)
#pragma unroll
            for (int g = 0; g < NT; g++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    float v = 0.0f;
                    for (int p = 0; p < S; p++)
                        v += partial[(((((wave + p) * RR + r) * NT + g) * 64) + lane) * 2 + j];
                    acc[r][g][j] = v;
                }
    }

    // --- epilogue --------------------------------------------------------------
    uint64_t best = 0;
    uint32_t bad = 0;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t row = (first_tile + r) * 16 + n;
        if (row >= rows) continue;
#pragma unroll
        for (int g = 0; g < NT; g++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t token = 8 * g + 2 * kg + j;
                if (token >= batch) continue;
                const float sc = MB > 0 ? token_scale[token][0] : yscale[token];
                float v = acc[r][g][j] * sc;
                if constexpr (MODE == 2) {
                    const float u = acc[R + r][g][j] * sc;
                    // silu(gate) * up, stable sigmoid (src/qwen35/cpu.rs:982-993)
                    float sig;
                    if (v >= 0.0f) {
                        sig = 1.0f / (1.0f + expf(-v));
                    } else {
                        const float ex = expf(v);
                        sig = ex / (1.0f + ex);
                    }
                    v = v * sig * u;
                }
                y[(size_t)token * rows + row] = v;
                if constexpr (MODE == 1) {
                    if (!__builtin_isfinite(v)) bad = 1;
                    const uint64_t key = argmax_key(v, row);
                    best = key > best ? key : best;
                }
            }
    }
    if constexpr (MODE == 1) {
        // No atomics and no device-wide fence here: each wave writes its own
        // candidate and a one-workgroup pass reduces them.
        best = wave_max_u64(best);
        bad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;
        if (lane == 0) {
            ArgmaxPartial p;
            p.key = best;
            p.non_finite = bad;
            p.pad = 0;
            partials[blockIdx.x * (WAVES / S) + group] = p;
        }
    }
}

// Reduces the per-wave candidates: the largest key wins (value, then lowest
// row); any non-finite row marks the result.
// 1024 threads with eight loads in flight each: a C2-sized candidate list
// (9496 entries) takes two rounds of memory latency.
constexpr uint32_t kArgmaxThreads = 1024;

__global__ void __launch_bounds__(kArgmaxThreads) argmax_partials_kernel(
    const ArgmaxPartial *__restrict__ partials, uint32_t count, ArgmaxState *state, uint32_t *index_out) {
    constexpr uint32_t U = 8, WAVES = kArgmaxThreads / 64;
    __shared__ unsigned long long keys[WAVES];
    __shared__ uint32_t flags[WAVES];
    uint64_t best = 0;
    uint32_t bad = 0;
    for (uint32_t i0 = 0; i0 < count; i0 += kArgmaxThreads * U) {
        ArgmaxPartial p[U];
#pragma unroll
        for (uint32_t j = 0; j < U; j++) {
            const uint32_t i = i0 + kArgmaxThreads * j + threadIdx.x;
            p[j] = i < count ? partials[i] : ArgmaxPartial{0, 0, 0};
        }
#pragma unroll
        for (uint32_t j = 0; j < U; j++) {
            best = p[j].key > best ? p[j].key : best;
            bad |= p[j].non_finite;
        }
    }
    best = wave_max_u64(best);
    bad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;
    if ((threadIdx.x & 63u) == 0) {
        keys[threadIdx.x >> 6] = best;
        flags[threadIdx.x >> 6] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = keys[0];
        uint32_t f = flags[0];
        for (uint32_t i = 1; i < WAVES; i++) {
            b = keys[i] > b ? keys[i] : b;
            f |= flags[i];
        }
        state->key = b;
        state->non_finite = f;
        state->done = count;
        *index_out = argmax_key_index(b);
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

bool qmv_supported(uint32_t type, size_t rows, size_t columns, const void *w, size_t batch) {
    if (type == kQ8_0) {
        // Q8_0 has the int8 kernel only: batch 1-4 (records permitting),
        // whole 8-block super-blocks (272 bytes, 16-byte aligned rows),
        // 32-bit offsets with slack.
        if (columns == 0 || columns % 256 || batch < 1 || batch > 4 || rows == 0) return false;
        const uint64_t row_bytes = (uint64_t)(columns / 256) * 272;
        if (row_bytes * (rows + 2) + 1024 >= 0xffffffffull || ((uintptr_t)w & 15u)) return false;
        return qmv8_supported(type, rows, columns, batch);
    }
    if (type != kQ4_K && type != kQ6_K) return false;
    if (columns == 0 || columns % 256 || batch < 1 || batch > 16) return false;
    const uint64_t row_bytes = (uint64_t)(columns / 256) * (type == kQ4_K ? 144 : 210);
    // Offsets are 32-bit: the matrix plus two rows of slack must fit.
    if (rows == 0 || row_bytes * (rows + 2) + 1024 >= 0xffffffffull) return false;
    const uintptr_t a = (uintptr_t)w;
    if (type == kQ4_K ? (a & 15u) : (a & 3u)) return false;
    return true;
}

namespace {

constexpr size_t kMaxLdsA = 56 * 1024;  // staged activation fragments; + split-K scratch <= 64 KiB

struct Plan {
    int nt, r, s, mb, g;
};

Plan choose_plan(uint32_t type, uint32_t rows, uint32_t blocks, uint32_t batch, int mode) {
    Plan p;
    p.nt = batch > 8 ? 2 : 1;
    const uint32_t tiles = (rows + 15) / 16;
    const uint32_t spb = type == kQ4_K ? 9 : 8;
    const size_t a_lds = ((size_t)blocks + 1) * spb * 4 * 2 * batch * 16;
    p.mb = (batch <= 2 && a_lds <= kMaxLdsA) ? (int)(2 * batch) : 0;
    // Two tiles per wave share each activation fragment load (batches above
    // 2, one matrix, tall matrices); short matrices need the waves more.
    p.r = (batch > 2 && mode != 2 && tiles >= 2048) ? 2 : 1;
    const uint32_t rr = mode == 2 ? 2 * p.r : p.r;
    // Blocks per staged group: 2 (runs of 2 blocks stream faster), or 1 when
    // the row has a single block or LDS is short.
    p.g = blocks >= 2 ? 2 : 1;
    // Split each tile's block groups over S waves of a workgroup until the
    // launch has about 4096 waves, with at least two groups per wave (S = 8
    // only for prepared activations of up to 8 tokens, else S <= 4).
    const uint32_t waves = (tiles + p.r - 1) / p.r;
    const uint32_t s_max = (p.mb == 0 && p.nt == 1) ? 8 : 4;
    uint32_t s = 1;
    while (s < s_max && (size_t)waves * s < 4096 && (blocks + p.g - 1) / p.g >= 4 * s) s *= 2;
    // Dynamic (activations, staging) plus static (split-K partials) LDS
    // within the 160 KiB of a workgroup: first one block per group, then a
    // narrower split.
    for (;;) {
        const uint32_t wv = s > 4 ? s : 4;
        const size_t items = 16 * (type == kQ4_K ? 9 * p.g : (210 * p.g + 2 + 15) / 16);
        const size_t lds = (p.mb > 0 ? a_lds : 0) + (size_t)wv * rr * items * 16 +
                           (s > 1 ? (size_t)wv * rr * p.nt * 64 * 2 * 4 : 4) + 256;
        if (lds <= 160 * 1024 || s == 1) break;
        if (p.g == 2) {
            p.g = 1;
        } else {
            s /= 2;
        }
    }
    p.s = (int)s;
    return p;
}

struct Args {
    const void *w, *w2;
    uint32_t rows, columns, row_bytes, total;
    const float *x;
    int normalize;
    float epsilon;
    const _Float16 *xp;
    const float *ysc;
    uint32_t batch;
    float *y;
    ArgmaxPartial *partials;
};

template <uint32_t TYPE, int NT, int R, int S, int MODE, int MB, uint32_t G>
hipError_t run(dmhip_ctx *ctx, const Args &a, uint32_t *waves_out) {
    constexpr uint32_t SPB = Steps<TYPE>::value;
    constexpr int RR = MODE == 2 ? 2 * R : R;
    constexpr uint32_t WAVES = S > 4 ? S : 4;
    const uint32_t tiles = (a.rows + 15) / 16;
    const uint32_t per_wg = (WAVES / S) * R;
    const uint32_t grid = (tiles + per_wg - 1) / per_wg;
    // fragments of every block plus one zeroed block for the idle A rows,
    // then each wave's weight staging area
    const size_t lds = (MB > 0 ? ((size_t)(a.columns / 256) + 1) * SPB * 4 * MB * 16 : 0) +
                       (size_t)WAVES * RR * StageQ<TYPE, G>::items * 16;
    if (waves_out) *waves_out = grid * (WAVES / S);
    auto kernel = qmv_kernel<TYPE, NT, R, S, MODE, MB, G>;
    if (lds > 64 * 1024) {
        static LdsLimit limit;
        hipError_t e = limit.ensure((const void *)kernel, lds);
        if (e != hipSuccess) return e;
    }
    return launch_kernel(ctx, kernel, dim3(grid), dim3(64 * WAVES), (uint32_t)lds, (const uint8_t *)a.w,
                         (const uint8_t *)a.w2, a.rows, a.columns, a.row_bytes, a.total, a.x, a.normalize, a.epsilon,
                         a.xp, a.ysc, a.batch, a.y, a.partials);
}

template <uint32_t TYPE, int NT, int R, int MODE, int MB, uint32_t G>
hipError_t run_sg(dmhip_ctx *ctx, const Plan &p, const Args &a, uint32_t *w) {
    if (p.s == 1) return run<TYPE, NT, R, 1, MODE, MB, G>(ctx, a, w);
    if (p.s == 2) return run<TYPE, NT, R, 2, MODE, MB, G>(ctx, a, w);
    if constexpr (MB == 0 && NT == 1) {
        // the 8-wave split serves short matrices with prepared activations of
        // up to 8 tokens (wider splits or two token groups outgrow the
        // registers of the larger workgroup)
        if (p.s == 8) return run<TYPE, NT, R, 8, MODE, MB, G>(ctx, a, w);
    }
    return run<TYPE, NT, R, 4, MODE, MB, G>(ctx, a, w);
}

template <uint32_t TYPE, int NT, int R, int MODE, int MB>
hipError_t run_s(dmhip_ctx *ctx, const Plan &p, const Args &a, uint32_t *w) {
    if (p.g == 2) return run_sg<TYPE, NT, R, MODE, MB, 2>(ctx, p, a, w);
    return run_sg<TYPE, NT, R, MODE, MB, 1>(ctx, p, a, w);
}

template <uint32_t TYPE, int MODE>
hipError_t dispatch(dmhip_ctx *ctx, const Plan &p, const Args &a, uint32_t *w) {
    if (p.mb == 2) return run_s<TYPE, 1, 1, MODE, 2>(ctx, p, a, w);
    if (p.mb == 4) return run_s<TYPE, 1, 1, MODE, 4>(ctx, p, a, w);
    if constexpr (MODE == 2) {
        // the gate/up pair already streams two matrices: one tile per wave
        return p.nt == 1 ? run_s<TYPE, 1, 1, MODE, 0>(ctx, p, a, w) : run_s<TYPE, 2, 1, MODE, 0>(ctx, p, a, w);
    } else {
        if (p.nt == 1)
            return p.r == 1 ? run_s<TYPE, 1, 1, MODE, 0>(ctx, p, a, w) : run_s<TYPE, 1, 2, MODE, 0>(ctx, p, a, w);
        return p.r == 1 ? run_s<TYPE, 2, 1, MODE, 0>(ctx, p, a, w) : run_s<TYPE, 2, 2, MODE, 0>(ctx, p, a, w);
    }
}

// Activation fragments for batches above 2 go to the context's aux scratch
// (or, during an allocation-free call, to the scratch it lent the context):
// [xp | yscale], written by the preparation kernel.
hipError_t prepare(dmhip_ctx *ctx, uint32_t type, uint32_t columns, uint32_t batch, const float *x,
                   int normalize, float eps, _Float16 **xp_out, float **ysc_out) {
    const uint32_t spb = type == kQ4_K ? 9 : 8;
    const size_t frags = (size_t)(columns / 256) * spb * 4;
    const size_t xp_bytes = frags * 2 * batch * 8 * sizeof(_Float16);
    const size_t need = ((xp_bytes + 255) & ~(size_t)255) + 64 * sizeof(float);
    void *base;
    if (ctx->aux_lent) {
        if (need > ctx->aux_lent_bytes) return hipErrorOutOfMemory;
        base = ctx->aux_lent;
    } else {
        if (ctx->aux.ensure(need) != DMHIP_OK) return hipErrorOutOfMemory;
        base = ctx->aux.ptr;
    }
    _Float16 *xp = (_Float16 *)base;
    float *ysc = (float *)((char *)base + ((xp_bytes + 255) & ~(size_t)255));
    uint32_t gx = (uint32_t)((frags + 255) / 256);
    if (gx > 64) gx = 64;
    const dim3 grid(gx, batch);
    if (columns <= kPrepareLdsColumns) {
        const size_t lds = (size_t)columns * sizeof(float);
        if (type == kQ4_K)
            hipLaunchKernelGGL((qmv_prepare_kernel<kQ4_K, true>), grid, dim3(256), lds, ctx->stream, x,
                               columns, batch, normalize, eps, xp, ysc);
        else
            hipLaunchKernelGGL((qmv_prepare_kernel<kQ6_K, true>), grid, dim3(256), lds, ctx->stream, x,
                               columns, batch, normalize, eps, xp, ysc);
    } else if (type == kQ4_K) {
        hipLaunchKernelGGL((qmv_prepare_kernel<kQ4_K, false>), grid, dim3(256), 0, ctx->stream, x,
                           columns, batch, normalize, eps, xp, ysc);
    } else {
        hipLaunchKernelGGL((qmv_prepare_kernel<kQ6_K, false>), grid, dim3(256), 0, ctx->stream, x,
                           columns, batch, normalize, eps, xp, ysc);
    }
    *xp_out = xp;
    *ysc_out = ysc;
    return hipGetLastError();
}

}  // namespace

size_t qmv_prepare_bytes(uint32_t type, size_t columns, size_t batch) {
    const size_t spb = type == kQ4_K ? 9 : 8;
    const size_t xp_bytes = (columns / 256) * spb * 4 * 2 * batch * 8 * sizeof(_Float16);
    return ((xp_bytes + 255) & ~(size_t)255) + 64 * sizeof(float);
}

namespace {

Args make_args(uint32_t type, uint32_t rows, uint32_t columns, const void *w, const void *w2,
               uint32_t batch, const float *x, int normalize, float epsilon, float *y) {
    Args a;
    const uint32_t blocks = columns / 256;
    a.w = w;
    a.w2 = w2;
    a.rows = rows;
    a.columns = columns;
    a.row_bytes = blocks * (type == kQ4_K ? 144u : 210u);
    a.total = a.row_bytes * rows;
    a.x = x;
    a.normalize = normalize;
    a.epsilon = epsilon;
    a.xp = nullptr;
    a.ysc = nullptr;
    a.batch = batch;
    a.y = y;
    a.partials = nullptr;
    return a;
}

}  // namespace

hipError_t launch_qmv(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns, const void *w,
                      uint32_t batch, const float *x, float *y, ArgmaxState *argmax,
                      uint32_t *index_out) {
    const bool int8_path = qmv8_supported(type, rows, columns, batch);
    if (!argmax && int8_path) return launch_qmv8(ctx, type, rows, columns, w, batch, x, y, nullptr, nullptr);
    Args a = make_args(type, rows, columns, w, w, batch, x, 0, 0.0f, y);
    const Plan p = choose_plan(type, rows, columns / 256, batch, argmax ? 1 : 0);
    if (!int8_path) {
        hipError_t pe = prepare(ctx, type, columns, batch, x, 0, 0.0f, (_Float16 **)&a.xp, (float **)&a.ysc);
        if (pe != hipSuccess) return pe;
    }
    if (!argmax)
        return type == kQ4_K ? dispatch<kQ4_K, 0>(ctx, p, a, nullptr) : dispatch<kQ6_K, 0>(ctx, p, a, nullptr);
    // One candidate per epilogue wave (at most one per 16-row tile), then a
    // one-workgroup reduction.
    const size_t candidates = (size_t)(rows + 15) / 16 + 4;
    if (ctx->partials.ensure(candidates * sizeof(ArgmaxPartial)) != DMHIP_OK) return hipErrorOutOfMemory;
    a.partials = (ArgmaxPartial *)ctx->partials.ptr;
    uint32_t count = 0;
    hipError_t e;
    if (int8_path) {
        // the int8 kernel's last workgroup publishes the argmax itself
        return launch_qmv8(ctx, type, rows, columns, w, batch, x, y, a.partials, &count,
                           ArgmaxFinish{argmax, index_out, ctx->argmax_ticket,
                                        (unsigned long long *)(ctx->argmax_ticket + 2)});
    }
    e = type == kQ4_K ? dispatch<kQ4_K, 1>(ctx, p, a, &count) : dispatch<kQ6_K, 1>(ctx, p, a, &count);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_partials_kernel, dim3(1), dim3(kArgmaxThreads), 0, ctx->stream, a.partials, count,
                       argmax, index_out);
    return hipGetLastError();
}

hipError_t launch_qmv_gate_up(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns,
                              const void *gate, const void *up, uint32_t batch, const float *x,
                              float *act, int normalize, float epsilon) {
    Args a = make_args(type, rows, columns, gate, up, batch, x, normalize, epsilon, act);
    const Plan p = choose_plan(type, rows, columns / 256, batch, 2);
    hipError_t e = prepare(ctx, type, columns, batch, x, normalize, epsilon, (_Float16 **)&a.xp,
                           (float **)&a.ysc);
    if (e != hipSuccess) return e;
    return type == kQ4_K ? dispatch<kQ4_K, 2>(ctx, p, a, nullptr) : dispatch<kQ6_K, 2>(ctx, p, a, nullptr);
}

// A kernel of this file: resolving it loads the file's code object.
const void *module_anchor_qmv() { return (const void *)argmax_partials_kernel; }

}  // namespace dm
