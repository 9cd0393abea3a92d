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
#include "dm_device.h"
#include "dm_qmv.h"

namespace dm {

namespace {

constexpr uint32_t kBias16 = 0x64006400u;  // fp16 pair (1024, 1024)

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

__device__ __forceinline__ half2_t h2_fma(half2_t a, half2_t b, half2_t c) {
    return __builtin_elementwise_fma(a, b, c);
}

__device__ __forceinline__ half2_t h2_splat(float v) {
    half2_t h;
    h[0] = (_Float16)v;
    h[1] = (_Float16)v;
    return h;
}

__device__ __forceinline__ floatx4 mfma(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8 frag(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4 v = {a, b, c, d};
    return __builtin_bit_cast(half8, v);
}

// Byte i (0..15) of four little-endian words.
__device__ __forceinline__ uint32_t byte_of(u32x4 w, uint32_t i) {
    uint32_t word = i < 4 ? w[0] : (i < 8 ? w[1] : (i < 12 ? w[2] : w[3]));
    return (word >> (8 * (i & 3))) & 0xffu;
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

}  // namespace

// ---------------------------------------------------------------------------
// Activation preparation: per token a power-of-two scale 2^-e with
// max|x| * 2^-e in [2^14, 2^15), the hi/lo fp16 fragments in step order,
// and (Q4_K) the 32-column sums.  yscale[t] = 2^e (times the RMSNorm factor
// when `normalize`).  Grid: (blocks of fragments, tokens).
// ---------------------------------------------------------------------------
template <uint32_t TYPE>
__global__ void __launch_bounds__(256) qmv_prepare_kernel(const float *__restrict__ x,
                                                          uint32_t columns, uint32_t batch,
                                                          int normalize, float epsilon,
                                                          _Float16 *__restrict__ xp,
                                                          float *__restrict__ yscale) {
    constexpr uint32_t SPB = Steps<TYPE>::value;
    __shared__ float red_max[4], red_ss[4];
    const uint32_t token = blockIdx.y;
    const float *xt = x + (size_t)token * columns;
    float mx = 0.0f, ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < columns; i += blockDim.x) {
        float v = xt[i];
        mx = fmaxf(mx, fabsf(v));
        if (fabsf(v) != fabsf(v)) mx = v;  // keep NaN visible
        ss = __builtin_fmaf(v, v, ss);
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
    int e = 0;
    if (mx > 0.0f && __builtin_isfinite(mx)) {
        int ex;
        (void)frexpf(mx, &ex);  // mx = f * 2^ex, f in [0.5, 1)
        e = ex - 15;            // mx * 2^-e in [2^14, 2^15)
        if (e < -126) e = -126;
        if (e > 127) e = 127;
    }
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
    for (uint32_t f = blockIdx.x * blockDim.x + threadIdx.x; f < fragments;
         f += gridDim.x * blockDim.x) {
        const uint32_t kg = f & 3u, t = (f >> 2) % SPB, blk = (f >> 2) / SPB;
        const float *xb = xt + (size_t)blk * 256;
        _Float16 hi[8], lo[8];
        if (TYPE == kQ4_K && t == 8) {
#pragma unroll
            for (int j = 0; j < 8; j++) { hi[j] = (_Float16)0.0f; lo[j] = (_Float16)0.0f; }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float *sb = xb + 32 * (2 * kg + j);
                float s = 0.0f;
                for (int i = 0; i < 32; i++) s += sb[i] * down;
                s = s * 0.015625f;  // 2^-6 keeps |sum| inside fp16
                _Float16 h = (_Float16)s;
                hi[j] = h;
                lo[j] = (_Float16)(s - (float)h);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                float v = xb[fragment_column<TYPE>(kg, t, j)] * down;
                _Float16 h = (_Float16)v;
                hi[j] = h;
                lo[j] = (_Float16)(v - (float)h);
            }
        }
        _Float16 *dst = xp + ((size_t)f * m2 + 2 * token) * 8;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            dst[j] = hi[j];
            dst[8 + j] = lo[j];
        }
    }
}

// ---------------------------------------------------------------------------
// Main kernel.  A workgroup has 4 waves; S waves split one group of R row
// tiles along K, so a workgroup covers (4/S)*R tiles of 16 rows.
// MODE 0: y = W x.  MODE 1: argmax epilogue.  MODE 2: gate/up pair,
// act = silu(gate) * up.
// ---------------------------------------------------------------------------
template <uint32_t TYPE, int NT, int R, int S, int MODE>
__global__ void __launch_bounds__(256) qmv_kernel(
    const uint8_t *__restrict__ w, const uint8_t *__restrict__ w2, uint32_t rows,
    uint32_t columns, uint32_t row_bytes, uint32_t total_bytes,
    const _Float16 *__restrict__ xp, const float *__restrict__ yscale, uint32_t batch,
    float *__restrict__ y, ArgmaxState *argmax) {
    constexpr uint32_t SPB = Steps<TYPE>::value;
    constexpr int RR = MODE == 2 ? 2 * R : R;  // gate/up: R tiles of each matrix
    __shared__ float partial[S > 1 ? 4 * RR * NT * 64 * 2 : 1];

    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 15u, kg = lane >> 4;
    const uint32_t group = wave / S, kpart = wave % S;
    const uint32_t first_tile = (blockIdx.x * (4 / S) + group) * R;
    const uint32_t blocks = columns / 256;
    const uint32_t b_begin = kpart * blocks / S, b_end = (kpart + 1) * blocks / S;
    const uint32_t m2 = 2 * batch;

    // Whole dwords: the last dword of the matrix may extend up to 3 bytes past
    // its end (inside the allocation's granularity); loads beyond it read 0.
    const uint32_t records = (total_bytes + 3u) & ~3u;
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
        row_base[r] = row < rows ? row * row_bytes : records + 256;  // out of range -> zeros
    }

    for (uint32_t blk = b_begin; blk < b_end; blk++) {
        // --- activations: SPB steps x NT token groups ------------------------
        half8 a[SPB][NT];
#pragma unroll
        for (int t = 0; t < (int)SPB; t++)
#pragma unroll
            for (int g = 0; g < NT; g++) {
                const uint32_t m = 16 * g + n;
                if (m < m2) {
                    const size_t f = ((size_t)blk * SPB + t) * 4 + kg;
                    a[t][g] = *(const half8 *)(xp + (f * m2 + m) * 8);
                } else {
                    a[t][g] = half8{0, 0, 0, 0, 0, 0, 0, 0};
                }
            }

#pragma unroll
        for (int r = 0; r < RR; r++) {
            const __amdgpu_buffer_rsrc_t rs = (MODE == 2 && r >= R) ? rsrc2 : rsrc;
            floatx4 cm[NT];
#pragma unroll
            for (int g = 0; g < NT; g++) cm[g] = floatx4{0, 0, 0, 0};
            float dscale, mscale = 0.0f;
            if constexpr (TYPE == kQ4_K) {
                const uint32_t off = row_base[r] + blk * 144u;
                const u32x4 hdr = rsrc_load16(rs, off);
                const u32x4 q0 = rsrc_load16(rs, off + 16 + 32 * kg);
                const u32x4 q1 = rsrc_load16(rs, off + 32 + 32 * kg);
                dscale = f16_bits_to_f32(hdr[0] & 0xffffu);
                mscale = f16_bits_to_f32(hdr[0] >> 16);
                // (scale, min) of sub-blocks 2kg and 2kg+1 (src/cpu.rs:607-616).
                uint32_t sc[2], mn[2];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const uint32_t idx = 2 * kg + j;
                    if (idx < 4) {
                        sc[j] = (hdr[1] >> (8 * idx)) & 63u;
                        mn[j] = (hdr[2] >> (8 * idx)) & 63u;
                    } else {
                        const uint32_t b = idx - 4;
                        const uint32_t s8 = (hdr[3] >> (8 * b)) & 0xffu;
                        sc[j] = (s8 & 15u) | (((hdr[1] >> (8 * b)) >> 6 & 3u) << 4);
                        mn[j] = (s8 >> 4) | (((hdr[2] >> (8 * b)) >> 6 & 3u) << 4);
                    }
                }
                const half2_t sl = h2_splat((float)sc[0]);
                const half2_t bl = h2_splat(-1024.0f * (float)sc[0]);
                const half2_t sh = h2_splat((float)sc[1] * 0.0625f);
                const half2_t bh = h2_splat(-64.0f * (float)sc[1]);
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const uint32_t d = t < 4 ? q0[t] : q1[t - 4];
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
                half2_t mm;
                mm[0] = (_Float16)(64.0f * (float)mn[0]);
                mm[1] = (_Float16)(64.0f * (float)mn[1]);
                const half8 bmin = frag(as_u(mm), 0u, 0u, 0u);
                floatx4 cmin[NT];
#pragma unroll
                for (int g = 0; g < NT; g++) cmin[g] = mfma(a[8][g], bmin, floatx4{0, 0, 0, 0});
#pragma unroll
                for (int g = 0; g < NT; g++) {
                    acc[r][g][0] = __builtin_fmaf(dscale, cm[g][0] + cm[g][1], acc[r][g][0]);
                    acc[r][g][0] = __builtin_fmaf(-mscale, cmin[g][0] + cmin[g][1], acc[r][g][0]);
                    acc[r][g][1] = __builtin_fmaf(dscale, cm[g][2] + cm[g][3], acc[r][g][1]);
                    acc[r][g][1] = __builtin_fmaf(-mscale, cmin[g][2] + cmin[g][3], acc[r][g][1]);
                }
            } else {  // Q6_K
                const uint32_t boff = row_base[r] + blk * 210u;
                const uint32_t s = boff & 3u;
                const uint32_t base = boff - s;
                const uint32_t h = kg >> 1, c = kg & 1u;
                uint32_t L1[4], L2[4], H[4], T[5];
                {
                    const uint32_t o1 = base + 64 * h + 16 * c;
                    const uint32_t o2 = o1 + 32;
                    const uint32_t o3 = base + 128 + 32 * h + 16 * c;
                    const uint32_t o4 = base + 192;
                    const u32x4 a1 = rsrc_load16(rs, o1), a2 = rsrc_load16(rs, o2),
                                a3 = rsrc_load16(rs, o3), a4 = rsrc_load16(rs, o4);
                    const uint32_t e1 = rsrc_load4(rs, o1 + 16), e2 = rsrc_load4(rs, o2 + 16),
                                   e3 = rsrc_load4(rs, o3 + 16), e4 = rsrc_load4(rs, o4 + 16);
                    const uint32_t e4b = rsrc_load4(rs, o4 + 20);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        L1[i] = funnel(a1[i], i < 3 ? a1[i + 1] : e1, s);
                        L2[i] = funnel(a2[i], i < 3 ? a2[i + 1] : e2, s);
                        H[i] = funnel(a3[i], i < 3 ? a3[i + 1] : e3, s);
                        T[i] = funnel(a4[i], i < 3 ? a4[i + 1] : e4, s);
                    }
                    T[4] = funnel(e4, e4b, s);
                }
                dscale = f16_bits_to_f32(T[4] & 0xffffu);
                // int8 scales sc[8h + 2k + c], k = 0..3.
                int sck[4];
                bool fast = true;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t bi = 8 * h + 2 * k + c;
                    sck[k] = (int)(int8_t)((T[bi >> 2] >> (8 * (bi & 3u))) & 0xffu);
                    fast = fast && sck[k] <= 62 && sck[k] >= -62;
                }
                const bool all_fast = __builtin_amdgcn_ballot_w64(!fast) == 0;
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const int k = t >> 1;
                    uint32_t pr[4];
#pragma unroll
                    for (int half_dw = 0; half_dw < 2; half_dw++) {
                        const int dw = 2 * (t & 1) + half_dw;
                        const uint32_t src = (k & 1) ? L2[dw] : L1[dw];
                        const uint32_t nib = (k & 2) ? (src >> 4) : src;
                        const uint32_t hb = H[dw] >> (2 * k);
                        pr[2 * half_dw] = (nib & 0x000f000fu) | ((hb << 4) & 0x00300030u) | kBias16;
                        pr[2 * half_dw + 1] =
                            ((nib >> 8) & 0x000f000fu) | ((hb >> 4) & 0x00300030u) | kBias16;
                    }
                    if (all_fast) {
                        const half2_t scl = h2_splat((float)sck[k]);
                        const half2_t bias = h2_splat(-1056.0f * (float)sck[k]);
                        const half8 b = frag(as_u(h2_fma(as_h2(pr[0]), scl, bias)),
                                             as_u(h2_fma(as_h2(pr[1]), scl, bias)),
                                             as_u(h2_fma(as_h2(pr[2]), scl, bias)),
                                             as_u(h2_fma(as_h2(pr[3]), scl, bias)));
#pragma unroll
                        for (int g = 0; g < NT; g++) cm[g] = mfma(a[t][g], b, cm[g]);
                    } else {
                        // sc = 8*sh + sl, sl in 0..7: both products exact in fp16.
                        const int shi = sck[k] >> 3, slo = sck[k] & 7;
                        const half2_t off = h2_splat(-1056.0f);
                        const half2_t one = h2_splat(1.0f);
                        const half2_t f_hi = h2_splat(8.0f * (float)shi);
                        const half2_t f_lo = h2_splat((float)slo);
                        half2_t qm[4];
#pragma unroll
                        for (int i = 0; i < 4; i++) qm[i] = h2_fma(as_h2(pr[i]), one, off);  // q - 32
                        const half8 b_hi = frag(as_u(qm[0] * f_hi), as_u(qm[1] * f_hi),
                                                as_u(qm[2] * f_hi), as_u(qm[3] * f_hi));
                        const half8 b_lo = frag(as_u(qm[0] * f_lo), as_u(qm[1] * f_lo),
                                                as_u(qm[2] * f_lo), as_u(qm[3] * f_lo));
#pragma unroll
                        for (int g = 0; g < NT; g++) {
                            cm[g] = mfma(a[t][g], b_hi, cm[g]);
                            cm[g] = mfma(a[t][g], b_lo, cm[g]);
                        }
                    }
                }
#pragma unroll
                for (int g = 0; g < NT; g++) {
                    acc[r][g][0] = __builtin_fmaf(dscale, cm[g][0] + cm[g][1], acc[r][g][0]);
                    acc[r][g][1] = __builtin_fmaf(dscale, cm[g][2] + cm[g][3], acc[r][g][1]);
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
                const float sc = yscale[token];
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
        best = wave_max_u64(best);
        if (lane == 0 && best) atomicMax(&argmax->key, (unsigned long long)best);
        if (bad) atomicOr(&argmax->non_finite, 1u);
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

bool qmv_supported(uint32_t type, size_t rows, size_t columns, const void *w, size_t batch) {
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

struct Plan {
    int nt, r, s;
};

Plan choose_plan(uint32_t rows, uint32_t blocks, uint32_t batch, int mode) {
    Plan p;
    p.nt = batch > 8 ? 2 : 1;
    const uint32_t tiles = (rows + 15) / 16;
    p.r = (batch > 2 && mode != 2) ? 2 : 1;
    // Enough waves to fill 256 CUs several times over; otherwise split K.
    const uint32_t waves = (tiles + p.r - 1) / p.r;
    if (waves >= 2048 || blocks < 2) {
        p.s = 1;
    } else if (waves >= 1024 || blocks < 4) {
        p.s = 2;
    } else {
        p.s = 4;
    }
    return p;
}

template <uint32_t TYPE, int NT, int R, int S, int MODE>
hipError_t run(hipStream_t stream, const void *w, const void *w2, uint32_t rows, uint32_t columns,
               uint32_t row_bytes, uint32_t total, const _Float16 *xp, const float *ysc,
               uint32_t batch, float *y, ArgmaxState *am) {
    const uint32_t tiles = (rows + 15) / 16;
    const uint32_t per_wg = (4 / S) * R;
    const uint32_t grid = (tiles + per_wg - 1) / per_wg;
    hipLaunchKernelGGL((qmv_kernel<TYPE, NT, R, S, MODE>), dim3(grid), dim3(256), 0, stream,
                       (const uint8_t *)w, (const uint8_t *)w2, rows, columns, row_bytes, total,
                       xp, ysc, batch, y, am);
    return hipGetLastError();
}

template <uint32_t TYPE, int MODE>
hipError_t dispatch(hipStream_t stream, const Plan &p, const void *w, const void *w2, uint32_t rows,
                    uint32_t columns, uint32_t row_bytes, uint32_t total, const _Float16 *xp,
                    const float *ysc, uint32_t batch, float *y, ArgmaxState *am) {
#define DM_RUN(NT_, R_, S_) \
    return run<TYPE, NT_, R_, S_, MODE>(stream, w, w2, rows, columns, row_bytes, total, xp, ysc, batch, y, am)
    if (p.nt == 1) {
        if (p.r == 1) {
            if (p.s == 1) DM_RUN(1, 1, 1);
            if (p.s == 2) DM_RUN(1, 1, 2);
            DM_RUN(1, 1, 4);
        }
        if (p.s == 1) DM_RUN(1, 2, 1);
        if (p.s == 2) DM_RUN(1, 2, 2);
        DM_RUN(1, 2, 4);
    }
    if (p.r == 1) {
        if (p.s == 1) DM_RUN(2, 1, 1);
        if (p.s == 2) DM_RUN(2, 1, 2);
        DM_RUN(2, 1, 4);
    }
    if (p.s == 1) DM_RUN(2, 2, 1);
    if (p.s == 2) DM_RUN(2, 2, 2);
    DM_RUN(2, 2, 4);
#undef DM_RUN
}

hipError_t prepare(dmhip_ctx *ctx, uint32_t type, uint32_t columns, uint32_t batch, const float *x,
                   int normalize, float eps, _Float16 **xp_out, float **ysc_out) {
    const uint32_t spb = type == kQ4_K ? 9 : 8;
    const size_t frags = (size_t)(columns / 256) * spb * 4;
    const size_t xp_bytes = frags * 2 * batch * 8 * sizeof(_Float16);
    if (ctx->aux.ensure(xp_bytes + 64 * sizeof(float)) != DMHIP_OK) return hipErrorOutOfMemory;
    _Float16 *xp = (_Float16 *)ctx->aux.ptr;
    float *ysc = (float *)((char *)ctx->aux.ptr + ((xp_bytes + 255) & ~(size_t)255));
    uint32_t gx = (uint32_t)((frags + 255) / 256);
    if (gx > 64) gx = 64;
    if (type == kQ4_K)
        hipLaunchKernelGGL(qmv_prepare_kernel<kQ4_K>, dim3(gx, batch), dim3(256), 0, ctx->stream, x,
                           columns, batch, normalize, eps, xp, ysc);
    else
        hipLaunchKernelGGL(qmv_prepare_kernel<kQ6_K>, dim3(gx, batch), dim3(256), 0, ctx->stream, x,
                           columns, batch, normalize, eps, xp, ysc);
    *xp_out = xp;
    *ysc_out = ysc;
    return hipGetLastError();
}

}  // namespace

hipError_t launch_qmv(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns, const void *w,
                      uint32_t batch, const float *x, float *y, ArgmaxState *argmax) {
    _Float16 *xp;
    float *ysc;
    hipError_t e = prepare(ctx, type, columns, batch, x, 0, 0.0f, &xp, &ysc);
    if (e != hipSuccess) return e;
    const uint32_t blocks = columns / 256;
    const uint32_t row_bytes = blocks * (type == kQ4_K ? 144u : 210u);
    const uint32_t total = row_bytes * rows;
    const Plan p = choose_plan(rows, blocks, batch, argmax ? 1 : 0);
    if (type == kQ4_K) {
        if (argmax) return dispatch<kQ4_K, 1>(ctx->stream, p, w, w, rows, columns, row_bytes, total, xp, ysc, batch, y, argmax);
        return dispatch<kQ4_K, 0>(ctx->stream, p, w, w, rows, columns, row_bytes, total, xp, ysc, batch, y, nullptr);
    }
    if (argmax) return dispatch<kQ6_K, 1>(ctx->stream, p, w, w, rows, columns, row_bytes, total, xp, ysc, batch, y, argmax);
    return dispatch<kQ6_K, 0>(ctx->stream, p, w, w, rows, columns, row_bytes, total, xp, ysc, batch, y, nullptr);
}

hipError_t launch_qmv_gate_up(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns,
                              const void *gate, const void *up, uint32_t batch, const float *x,
                              float *act, int normalize, float epsilon) {
    _Float16 *xp;
    float *ysc;
    hipError_t e = prepare(ctx, type, columns, batch, x, normalize, epsilon, &xp, &ysc);
    if (e != hipSuccess) return e;
    const uint32_t blocks = columns / 256;
    const uint32_t row_bytes = blocks * (type == kQ4_K ? 144u : 210u);
    const uint32_t total = row_bytes * rows;
    const Plan p = choose_plan(rows, blocks, batch, 2);
    if (type == kQ4_K)
        return dispatch<kQ4_K, 2>(ctx->stream, p, gate, up, rows, columns, row_bytes, total, xp, ysc, batch, act, nullptr);
    return dispatch<kQ6_K, 2>(ctx->stream, p, gate, up, rows, columns, row_bytes, total, xp, ysc, batch, act, nullptr);
}

}  // namespace dm
