// kernels_gemm.hip -- prefill GEMM C[m][n] = sum_k A[m][k] * W[n][k] for gfx950.
//
// A is bf16 activations [m][k]; W is n encoded rows of k columns.  The
// reference has no batched prefill: it runs one matvec per token
// (src/gemma4/metal.rs:514-536), so the result for token m must match
// cpu::matvec(W, widen(A[m])) (src/cpu.rs:345-399) within fp32 tolerance.
//
// Q4_K weights run on v_mfma_f32_32x32x16_f16 with exact fp16 operands and
// fp32 accumulation:
//  * A: each row is scaled by a power of two 2^-e (max|a| 2^-e in
//    [2^14, 2^15)) and converted to fp16.  bf16 carries 8 significant bits, so
//    the conversion is exact for every value above 2^-17 of the row maximum.
//  * W: each weight enters as the fp16 integer sc*q (0..945), built from the
//    nibble with the "1024 + q" exponent trick and one packed fp16 FMA.  The
//    fp32 partial of every 256-column block is then multiplied by d.
//  * Q4_K's "- dmin * m * sum(a)" term: one extra MFMA per block whose B
//    holds 64 m of the 8 sub-blocks (twice: hi and lo) and whose A holds the
//    sub-block sums of the scaled row times 2^-6 as fp16 hi/lo pairs; the
//    result is multiplied by dmin.
// Other weight types take the decode-GEMV path in chunks of 16 tokens.
//
// Tiling: a workgroup (8 waves) owns a 64 x 128 tile of C; each group of 4
// waves forms a 2 x 2 grid of 32 x 64 sub-tiles (two 32x32 MFMA tiles each)
// and takes every other K-step.  K advances in
// stages of 128 columns (half a Q4_K block): the stage's A rows and
// dequantized W rows go to padded LDS rows (272 B: the 16 lanes of a 128-bit
// read hit 64 distinct banks), double-buffered so that dequantizing the next
// stage overlaps the MFMAs of this one.  Workgroups that work on the same 64
// rows of A run on the same XCD.
#include "dm_device.h"
#include "dm_qmv.h"
#include "runtime.h"

#include <type_traits>

namespace dm {

namespace {

constexpr uint32_t kBM = 64, kBN = 128, kStage = 128;
constexpr uint32_t kLd = kStage + 8;  // halves per LDS row (272 B)

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

__device__ __forceinline__ floatx16 mfma32(half8 a, half8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

}  // namespace

// ---------------------------------------------------------------------------
// A preparation: one workgroup per row of the padded workspace.
//   a16[m][k]      fp16 of A[m][k] * 2^-e_m (zero rows beyond M)
//   sums[m][b][16] sub-block sums of the scaled row * 2^-6 as (hi, lo) fp16
//   rowscale[m]    2^e_m
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) gemm_prep_kernel(const uint16_t *__restrict__ a, uint32_t m_rows,
                                                        uint32_t k, _Float16 *__restrict__ a16,
                                                        _Float16 *__restrict__ sums, float *__restrict__ rowscale) {
    __shared__ float red[4];
    const uint32_t m = blockIdx.x, tid = threadIdx.x;
    const bool live = m < m_rows;
    const uint16_t *row = a + (size_t)m * k;
    // chunk c (8 consecutive values) = tid + 256 r
    float mx = 0.0f;
    for (uint32_t c = tid; c < k / 8; c += 256) {
        if (!live) break;
        const u32x4 v = *(const u32x4 *)(row + 8 * c);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            mx = fmaxf(mx, fabsf(__uint_as_float(v[i] << 16)));
            mx = fmaxf(mx, fabsf(__uint_as_float(v[i] & 0xffff0000u)));
        }
    }
    mx = wave_max(mx);
    if ((tid & 63u) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (mx > 0.0f && __builtin_isfinite(mx)) {
        int ex;
        (void)frexpf(mx, &ex);
        e = ex - 15;
        if (e < -126) e = -126;
        if (e > 127) e = 127;
    }
    const float down = ldexpf(1.0f, -e);
    if (tid == 0) rowscale[m] = live ? ldexpf(1.0f, e) : 0.0f;
    const uint32_t blocks = k / 256;
    for (uint32_t c = tid; c < k / 8; c += 256) {
        float v[8];
        if (live) {
            const u32x4 raw = *(const u32x4 *)(row + 8 * c);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[2 * i] = __uint_as_float(raw[i] << 16) * down;
                v[2 * i + 1] = __uint_as_float(raw[i] & 0xffff0000u) * down;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = 0.0f;
        }
        half8 h;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            h[i] = (_Float16)v[i];
            s += v[i];
        }
        *(half8 *)(a16 + (size_t)m * k + 8 * c) = h;
        // a 32-value sub-block is four consecutive chunks (threads 4j .. 4j+3)
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        if ((tid & 3u) == 0) {
            const uint32_t sb = c / 4, b = sb / 8, j = sb % 8;
            const float scaled = s * 0.015625f;  // 2^-6 keeps |sum| inside fp16
            const _Float16 hi = (_Float16)scaled;
            const _Float16 lo = (_Float16)(scaled - (float)hi);
            _Float16 *dst = sums + ((size_t)m * blocks + b) * 16 + 2 * j;
            dst[0] = hi;
            dst[1] = lo;
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_K GEMM main kernel.  Grid: one workgroup (8 waves) per 64 x 128 tile of
// C.  Waves 0-3 and 4-7 form two groups with the same 2 x 2 layout of 32 x 64
// sub-tiles; group g takes the K-steps of parity g of every stage, and the
// two partial tiles are added at the end (two waves per SIMD, half the
// dequantization per thread).  LDS is double-buffered by stage: while the
// MFMAs of stage s read buffer s & 1, the waves dequantize stage s + 1 from
// registers into the other buffer, and the loads of stage s + 3 are in
// flight.  One barrier per stage.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(512) gemm_q4k_kernel(const _Float16 *__restrict__ a16,
                                                       const _Float16 *__restrict__ sums,
                                                       const float *__restrict__ rowscale,
                                                       const uint8_t *__restrict__ w, uint32_t m_rows,
                                                       uint32_t n_rows, uint32_t k, uint32_t w_bytes,
                                                       uint32_t m_tiles, float *__restrict__ c) {
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][kBM * kLd];
    __shared__ __attribute__((aligned(16))) _Float16 sW[2][kBN * kLd];
    // per block (double-buffered by block parity): sub-block sums (hi, lo),
    // 64 m duplicated for hi and lo, d and dmin
    __shared__ __attribute__((aligned(16))) _Float16 sA2[2][kBM * 16];
    __shared__ __attribute__((aligned(16))) _Float16 sB2[2][kBN * 16];
    __shared__ float sD[2][kBN], sDmin[2][kBN];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t grp = wave >> 2, wm = wave & 1u, wn = (wave >> 1) & 1u;
    // Tile order: the 8 XCDs take workgroups round-robin, so with m-tile =
    // id % m_tiles and 8 m-tiles (M = 512) each XCD keeps one 64-row slice of
    // A (512 KB) in its L2 while W streams past it.
    const uint32_t id = blockIdx.x;
    const uint32_t mt = id % m_tiles, nt = id / m_tiles;
    const uint32_t m0 = mt * kBM, n0 = nt * kBN;
    const uint32_t blocks = k / 256, stages = 2 * blocks;
    const uint32_t row_bytes = blocks * 144;

    const uint32_t records = (w_bytes + 3u) & ~3u;
    const uint32_t nowhere = records + 256;
    const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(w, records);

    // loader roles (per stage of 128 columns)
    const uint32_t a_row = tid >> 3, a_part = tid & 7u;  // 64 rows x 8 parts of 16 halves
    const uint32_t w_row = tid >> 2, w_q = tid & 3u;     // 128 rows x 4 quarters of the stage's qs
    const uint32_t w_base = n0 + w_row < n_rows ? (n0 + w_row) * row_bytes : nowhere;
    const _Float16 *a_src = a16 + (size_t)(m0 + a_row) * k + 16 * a_part;

    struct Regs {
        u32x4 a[2];  // 16 halves of A
        u32x4 q;     // 16 qs bytes: 64 hb + 16 w_q .. + 16
        u32x4 hdr;   // d | dmin | scales
        u32x4 s;     // 8 halves of the block's sub-block sums
    };
    auto fetch = [&](uint32_t s, Regs &r) {
        const uint32_t b = s >> 1, hb = s & 1u;
        const u32x4 *ap = (const u32x4 *)(a_src + b * 256 + hb * 128);
        r.a[0] = ap[0];
        r.a[1] = ap[1];
        const uint32_t off = w_base == nowhere ? nowhere : w_base + b * 144;
        r.hdr = rsrc_load16(rsrc, off);
        r.q = rsrc_load16(rsrc, off == nowhere ? nowhere : off + 16 + 64 * hb + 16 * w_q);
        // every thread loads (threads >= 128 duplicate threads 0..127), so the
        // loop has no divergent branch around a load
        r.s = *(const u32x4 *)(sums + ((size_t)(m0 + ((tid & 127u) >> 1)) * blocks + b) * 16 + 8 * (tid & 1u));
    };

    // Branch-free 6-bit (scale, min) of sub-block sb of a Q4_K block
    // (src/cpu.rs:607-616): for sb < 4 the low 6 bits of scales[sb] and
    // scales[sb+4]; for sb >= 4 nibbles of scales[sb+4] with the top bits of
    // scales[sb-4] and scales[sb].
    auto scale_min = [](const u32x4 &hdr, uint32_t sb, uint32_t &sc, uint32_t &mn) {
        const uint32_t sh = 8 * (sb & 3u);
        const uint32_t b1 = hdr[1] >> sh, b2 = hdr[2] >> sh, b3 = hdr[3] >> sh;
        const uint32_t hi_mask = 0u - (uint32_t)(sb >= 4);
        const uint32_t sc_lo = b1 & 63u, sc_hi = (b3 & 15u) | ((b1 >> 2) & 0x30u);
        const uint32_t mn_lo = b2 & 63u, mn_hi = ((b3 >> 4) & 15u) | ((b2 >> 2) & 0x30u);
        sc = sc_lo ^ ((sc_lo ^ sc_hi) & hi_mask);
        mn = mn_lo ^ ((mn_lo ^ mn_hi) & hi_mask);
    };

    constexpr uint32_t kBias = 0x64646464u;  // source of the 0x64 high bytes ("1024 + q")
    // The thread's 16 qs bytes belong to sub-block pair j = 2 hb + (w_q >> 1):
    // low nibbles are sub-block 2j at stage columns 64 (w_q >> 1) + 16 (w_q & 1)
    // + i, high nibbles sub-block 2j + 1 at the same columns + 32.
    struct Scales {
        half2_t scl[2], bias[2];
    };
    auto scales = [&](auto hb_c, const Regs &r) {
        constexpr uint32_t hb = decltype(hb_c)::value;
        const uint32_t j = 2 * hb + (w_q >> 1);
        Scales out;
#pragma unroll
        for (int t = 0; t < 2; t++) {
            uint32_t sc, mn;
            scale_min(r.hdr, 2 * j + t, sc, mn);
            const _Float16 f = (_Float16)(short)sc;
            out.scl[t] = half2_t{f, f};
            out.bias[t] = out.scl[t] * half2_t{(_Float16)-1024.0f, (_Float16)-1024.0f};
        }
        return out;
    };
    // Piece p (0, 1) dequantizes qs dwords 2p, 2p + 1 (16 weights); piece 1
    // also copies A and, at the first stage of a block, the block data.
    auto store_piece = [&](auto hb_c, auto p_c, uint32_t s, const Regs &r, const Scales &sv) {
        constexpr uint32_t hb = decltype(hb_c)::value;
        constexpr int p = decltype(p_c)::value;
        const uint32_t buf = hb, bb = (s >> 1) & 1u;
        _Float16 *wd = sW[buf] + w_row * kLd + 64 * (w_q >> 1) + 16 * (w_q & 1u) + 8 * p;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const uint32_t d = r.q[2 * p + u];
            const uint32_t l4 = d & 0x0f0f0f0fu, h4 = (d >> 4) & 0x0f0f0f0fu;
            lo[2 * u] = as_u(__builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(l4, kBias, 0x00050004u)), sv.scl[0], sv.bias[0]));
            lo[2 * u + 1] = as_u(__builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(l4, kBias, 0x00070006u)), sv.scl[0], sv.bias[0]));
            hi[2 * u] = as_u(__builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(h4, kBias, 0x00050004u)), sv.scl[1], sv.bias[1]));
            hi[2 * u + 1] = as_u(__builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(h4, kBias, 0x00070006u)), sv.scl[1], sv.bias[1]));
        }
        *(u32x4 *)wd = u32x4{lo[0], lo[1], lo[2], lo[3]};
        *(u32x4 *)(wd + 32) = u32x4{hi[0], hi[1], hi[2], hi[3]};
        if constexpr (p == 1) {
            u32x4 *ad = (u32x4 *)(sA[buf] + a_row * kLd + 16 * a_part);
            ad[0] = r.a[0];
            ad[1] = r.a[1];
            if constexpr (hb == 0) {
                // per block: d, dmin, the 64 m row of the min step, the sums
                sD[bb][w_row] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.hdr[0] & 0xffffu));
                sDmin[bb][w_row] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.hdr[0] >> 16));
                uint32_t mm[2];
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    uint32_t sc, mn;
                    scale_min(r.hdr, 2 * w_q + t, sc, mn);
                    const _Float16 f = (_Float16)(short)(64 * mn);
                    mm[t] = as_u(half2_t{f, f});
                }
                *(u32x2 *)(sB2[bb] + w_row * 16 + 4 * w_q) = u32x2{mm[0], mm[1]};
                // threads >= 128 write the same bytes as thread tid - 128
                *(u32x4 *)(sA2[bb] + ((tid & 127u) >> 1) * 16 + 8 * (tid & 1u)) = r.s;
            }
        }
    };

    floatx16 acc[2], part[2];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int j = 0; j < 16; j++) acc[t][j] = part[t][j] = 0.0f;

    const uint32_t lr = lane & 31u, lk = 8 * (lane >> 5);
    // The group's MFMAs of stage s (parity ODD): K-steps grp, grp + 2, ...,
    // with the store of stage s + 1 spread between them when STORE.
    auto compute_and_store = [&](auto odd_c, auto store_c, uint32_t s, const Regs &next) {
        constexpr uint32_t ODD = decltype(odd_c)::value;
        constexpr bool STORE = decltype(store_c)::value;
        using NextHb = std::integral_constant<uint32_t, ODD ^ 1u>;
        const _Float16 *pa = sA[ODD] + (wm * 32 + lr) * kLd + lk + 16 * grp;
        const _Float16 *pb = sW[ODD] + (wn * 64 + lr) * kLd + lk + 16 * grp;
        Scales sv;
        if constexpr (STORE) sv = scales(NextHb{}, next);
        // fragments of the next K-step are read while this one runs
        half8 av[2], b0[2], b1[2];
        auto frags = [&](uint32_t i, int slot) {
            av[slot] = *(const half8 *)(pa + i * 32);
            b0[slot] = *(const half8 *)(pb + i * 32);
            b1[slot] = *(const half8 *)(pb + 32 * kLd + i * 32);
        };
        frags(0, 0);
#pragma unroll
        for (uint32_t i = 0; i < kStage / 32; i++) {
            if (i + 1 < kStage / 32) frags(i + 1, (int)((i + 1) & 1u));
            part[0] = mfma32(av[i & 1u], b0[i & 1u], part[0]);
            part[1] = mfma32(av[i & 1u], b1[i & 1u], part[1]);
            if constexpr (STORE) {
                if (i == 1) store_piece(NextHb{}, std::integral_constant<int, 0>{}, s + 1, next, sv);
                if (i == 3) store_piece(NextHb{}, std::integral_constant<int, 1>{}, s + 1, next, sv);
            }
        }
        if constexpr (ODD == 1) {
            // end of the block: scale by d; group 0 subtracts dmin * (m . sums)
            const uint32_t bb = (s >> 1) & 1u;
            const half8 av2 = *(const half8 *)(sA2[bb] + (wm * 32 + lr) * 16 + lk);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint32_t col = wn * 64 + t * 32 + lr;
                const float d = sD[bb][col];
#pragma unroll
                for (int j = 0; j < 16; j++) acc[t][j] = __builtin_fmaf(d, part[t][j], acc[t][j]);
                if (grp == 0) {
                    const half8 bv = *(const half8 *)(sB2[bb] + col * 16 + lk);
                    floatx16 zero;
#pragma unroll
                    for (int j = 0; j < 16; j++) zero[j] = 0.0f;
                    const floatx16 mins = mfma32(av2, bv, zero);
                    const float dmin = sDmin[bb][col];
#pragma unroll
                    for (int j = 0; j < 16; j++) acc[t][j] = __builtin_fmaf(-dmin, mins[j], acc[t][j]);
                }
#pragma unroll
                for (int j = 0; j < 16; j++) part[t][j] = 0.0f;
            }
        }
    };
    using Even = std::integral_constant<uint32_t, 0>;
    using Odd = std::integral_constant<uint32_t, 1>;
    using Yes = std::true_type;
    using No = std::false_type;
    auto last = [&](uint32_t t) { return t < stages ? t : stages - 1; };  // clamped prefetch

    // Prologue: stage 0 stored, stages 1 and 2 in flight.
    Regs r0, r1;
    fetch(0, r0);
    fetch(last(1), r1);
    {
        const Scales sv0 = scales(Even{}, r0);
        store_piece(Even{}, std::integral_constant<int, 0>{}, 0, r0, sv0);
        store_piece(Even{}, std::integral_constant<int, 1>{}, 0, r0, sv0);
    }
    fetch(last(2), r0);
    __syncthreads();
    // Iteration pair s, s + 1: compute s (buffer 0) storing s + 1 from r1 and
    // refilling r1 with s + 3; compute s + 1 (buffer 1) storing s + 2 from r0
    // and refilling r0 with s + 4.  The last pair stores nothing beyond the
    // final stage.
    uint32_t s = 0;
    for (; s + 2 < stages; s += 2) {
        compute_and_store(Even{}, Yes{}, s, r1);
        fetch(last(s + 3), r1);
        __syncthreads();
        compute_and_store(Odd{}, Yes{}, s + 1, r0);
        fetch(last(s + 4), r0);
        __syncthreads();
    }
    compute_and_store(Even{}, Yes{}, s, r1);
    __syncthreads();
    compute_and_store(Odd{}, No{}, s + 1, r0);
    __syncthreads();

    // Group 1 hands its partial tile to group 0 through LDS (the A buffers).
    float *red = (float *)&sA[0][0];
    const uint32_t slot = ((wave & 3u) * 64 + lane) * 32;
    if (grp == 1) {
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int j = 0; j < 16; j++) red[slot + 16 * t + j] = acc[t][j];
    }
    __syncthreads();
    if (grp == 1) return;
    // C[m][n] = acc * rowscale[m]; lane holds column lr, rows 8(j/4) + 4(lane/32) + j%4.
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const uint32_t n = n0 + wn * 64 + t * 32 + lr;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const float v = acc[t][j] + red[slot + 16 * t + j];
            const uint32_t m = m0 + wm * 32 + 8 * (j / 4) + 4 * (lane >> 5) + (j % 4);
            if (n < n_rows && m < m_rows) c[(size_t)m * n_rows + n] = v * rowscale[m];
        }
    }
}

__global__ void bf16_to_f32_kernel(const uint16_t *__restrict__ a, size_t count, float *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = __uint_as_float((uint32_t)a[i] << 16);
}

namespace {

size_t padded_rows(size_t m) { return (m + kBM - 1) / kBM * kBM; }

// Workspace of the Q4_K path: a16 | sums | rowscale.
size_t q4k_workspace(size_t m, size_t k) {
    const size_t mp = padded_rows(m);
    return mp * k * 2 + mp * (k / 256) * 16 * 2 + mp * 4 + 3 * 256;
}

}  // namespace

}  // namespace dm

using namespace dm;

extern "C" {

size_t dmhip_gemm_workspace_bytes(size_t m, size_t k) {
    const size_t tokenwise = m * k * sizeof(float) + 256;
    const size_t q4k = q4k_workspace(m, k);
    return tokenwise > q4k ? tokenwise : q4k;
}

int dmhip_gemm_device(dmhip_ctx *ctx, uint32_t type, size_t m, size_t n, size_t k,
                      const uint16_t *a_bf16, const void *weights, float *c, void *workspace) {
    if (!ctx || !a_bf16 || !weights || !c || !workspace)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "gemm arguments must not be null");
    if (!(type == 0 || type == 1 || type == 6 || type == 8 || type == 12 || type == 14))
        return fail(DMHIP_ERR_UNSUPPORTED_TENSOR_TYPE, "HIP GEMM does not support %s", type_name(type));
    uint64_t rb;
    if (!row_byte_len(type, k, &rb))
        return fail(DMHIP_ERR_INVALID_ELEMENT_COUNT, "%s row of %zu values is not whole blocks",
                    type_name(type), k);
    if (m == 0 || n == 0) return DMHIP_OK;
    if (k == 0) return fail(DMHIP_ERR_EMPTY_INPUT, "gemm requires a non-empty input");
    if (m > 0xffffffffull || n > 0xffffffffull || k > 0xffffffffull)
        return fail(DMHIP_ERR_VECTOR_TOO_LARGE, "HIP vector length exceeds the 32-bit kernel limit");
    DM_CHECK_STATUS(set_device(ctx));

    const uint64_t w_bytes = rb * n;
    if (type == kQ4_K && w_bytes + 1024 < 0xffffffffull && ((uintptr_t)weights & 15u) == 0 &&
        ((uintptr_t)a_bf16 & 15u) == 0) {
        const size_t mp = padded_rows(m);
        char *ws = (char *)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
        _Float16 *a16 = (_Float16 *)ws;
        _Float16 *sums = (_Float16 *)(ws + ((mp * k * 2 + 255) & ~(size_t)255));
        float *rowscale =
            (float *)((char *)sums + ((mp * (k / 256) * 32 + 255) & ~(size_t)255));
        hipLaunchKernelGGL(gemm_prep_kernel, dim3((uint32_t)mp), dim3(256), 0, ctx->stream, a_bf16,
                           (uint32_t)m, (uint32_t)k, a16, sums, rowscale);
        DM_HIP(hipGetLastError());
        const uint32_t n_tiles = (uint32_t)((n + kBN - 1) / kBN), m_tiles = (uint32_t)(mp / kBM);
        {
            KernelTimer timer(ctx);
            hipLaunchKernelGGL(gemm_q4k_kernel, dim3(n_tiles * m_tiles), dim3(512), 0, ctx->stream, a16, sums,
                               rowscale, (const uint8_t *)weights, (uint32_t)m, (uint32_t)n, (uint32_t)k,
                               (uint32_t)w_bytes, m_tiles, c);
        }
        DM_HIP(hipGetLastError());
        return DMHIP_OK;
    }

    float *af = (float *)workspace;
    size_t count = m * k;
    size_t blocks = (count + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(bf16_to_f32_kernel, dim3((uint32_t)blocks), dim3(256), 0, ctx->stream, a_bf16,
                       count, af);
    DM_HIP(hipGetLastError());
    for (size_t m0 = 0; m0 < m; m0 += 16) {
        size_t mb = m - m0 < 16 ? m - m0 : 16;
        DM_CHECK_STATUS(enqueue_matvec(ctx, type, n, k, weights, mb, af + m0 * k, c + m0 * n));
    }
    return DMHIP_OK;
}

}  // extern "C"
