// kernels_gemm.hip -- prefill GEMM C[m][n] = sum_k A[m][k] * W[n][k] for gfx950.
//
// A is bf16 activations [m][k]; W is n encoded rows of k columns.  The
// reference has no batched prefill: it runs one matvec per token
// (src/gemma4/metal.rs:514-536), so the result for token m must match
// cpu::matvec(W, widen(A[m])) (src/cpu.rs:345-399) within the GEMM tolerance
// (max |c - r| <= 1e-3 max |r|, cosine >= 0.99999).
//
// Q4_K weights run on v_mfma_f32_32x32x16_f16 with fp32 accumulation after
// an on-the-fly dequantization to fp16:
//  * A: each row is scaled by a power of two 2^-e (max|a| 2^-e in
//    [2^14, 2^15)) and converted to fp16.  bf16 carries 8 significant bits, so
//    the conversion is exact for every value above 2^-17 of the row maximum;
//    the output is multiplied back by 2^e.
//  * W: weight q of sub-block j is fma(q, fp16(d sc_j), fp16(-dmin m_j)) in
//    fp16 (src/cpu.rs:585-605 computes the same value in fp32).  The nibble q
//    is read as an fp8 e4m3 code (codes 0..15 are q * 2^-9 exactly) by
//    v_cvt_scalef32_pk_f16_fp8 with scale 2^9; one packed fp16 FMA then
//    gives two weights.  The roundings of d sc_j, dmin m_j and of the weight
//    to fp16 leave a few 1e-4 of max |r| on seeded Q4_K data.
// The sum over K is order-free, so K is permuted once for both operands: in
// MFMA step s of a block, lane half h holds the low and high nibbles of qs
// bytes 64h + 4s .. 64h + 4s + 3, and A is stored in that order.
// Other weight types take the decode-GEMV path in chunks of 16 tokens.
//
// Tiling: a workgroup of 4 waves (one per SIMD) owns a 128 x 64 tile of C
// (8 waves, two per SIMD, and a 64 x 128 tile for prefills of at most 64
// tokens); wave w computes the 128 x 64 tile (64 x 64 half w / 4) over every
// fourth Q4_K block (w % 4, w % 4 + 4, ...), so every W element is
// dequantized by exactly one wave and feeds 4 (2) MFMA row tiles, and no
// operand is shared through LDS.  A comes from global memory
// already in MFMA fragment order (one 1 KiB load per 32 rows and step); a
// wave stages its W block (64 rows x 144 bytes, contiguous 16-byte loads) in
// its own LDS area and dequantizes from there, with the next block's W in
// flight in registers.  The accumulators stay in AGPRs for the whole K loop;
// the partial tiles are added through LDS at the end.  Workgroups are
// ordered so that each XCD keeps half of A in its L2.
#include "dm_device.h"
#include "dm_qmv.h"
#include "runtime.h"


namespace dm {

namespace {

// Workgroup tilings (BM rows of C x BN columns; wave tile BM x WN):
//  * BM = 64:  BN = 128, 8 waves (4-way K split x 2 column halves), two waves
//    per SIMD, wave tile 64 x 64 (2 x 2 MFMA tiles of 32 x 32);
//  * BM = 128: BN = 64, 4 waves (4-way K split), one wave per SIMD, wave
//    tile 128 x 64 (4 x 2 MFMA tiles): each dequantized weight feeds four
//    MFMA row tiles instead of two.
template <uint32_t BM> struct Tiling {
    static constexpr uint32_t kBM = BM, kBN = BM == 64 ? 128 : 64;
    static constexpr uint32_t kKSplit = 4, kNHalves = BM == 64 ? 2 : 1, kWaves = kKSplit * kNHalves;
    static constexpr uint32_t kWN = kBN / kNHalves;  // columns of a wave's tile
    static constexpr uint32_t kRM = BM / 32;          // MFMA row tiles of a wave
    static constexpr uint32_t kStageBytes = kWN * 144;              // one Q4_K block of a wave's W rows
    static constexpr uint32_t kStageLoads = kStageBytes / 16 / 64;  // 16-byte loads per lane
    static constexpr uint32_t kRedLd = kWN + 4;                     // floats per row of a partial tile in LDS
    static constexpr uint32_t kLdsBytes = kWaves * kBM * kRedLd * 4;  // partial tiles of the final sum
    static_assert(kWaves * kStageBytes <= kLdsBytes, "the W staging areas fit in the reduction area");
    static_assert(kStageBytes % 1024 == 0, "whole staging loads");
    static_assert(kLdsBytes <= 160 * 1024, "one workgroup's LDS");
};
constexpr uint32_t kPadRows = 128;  // workspace rows are padded to a multiple of every tiling's BM
// MFMA steps between the load of an A fragment and its use.  Loads complete
// in order, so this is also the time every W load has to arrive.
constexpr uint32_t kADist = 4;
static_assert(16 % kADist == 0, "the A ring repeats every block");

typedef uint32_t v4u __attribute__((ext_vector_type(4)));  // 16-byte aligned

__device__ __forceinline__ floatx16 mfma32(half8 a, half8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// First column (within its block) of the 8 columns of MFMA step s, lane half
// h: columns base .. base + 3 and base + 32 .. base + 35.
__device__ __forceinline__ uint32_t frag_base(uint32_t s, uint32_t h) { return 64 * (2 * h + s / 8) + 4 * (s % 8); }

// Per sub-block fp16 pairs (d sc, d sc) and (-dmin m, -dmin m).
struct SubScale {
    half2_t mul, add;
};

__device__ __forceinline__ SubScale sub_scale(float d, float dmin, uint32_t sc, uint32_t mn) {
    const _Float16 a = (_Float16)(d * (float)sc), b = (_Float16)(-dmin * (float)mn);
    return SubScale{half2_t{a, a}, half2_t{b, b}};
}

// The 8 weights of one qs dword: low nibbles of its 4 bytes (sub-block
// scale lo), then high nibbles (hi).
template <bool HIGH_WORD>
__device__ __forceinline__ half2_t q_pair(uint32_t v) {
    return __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v, 512.0f, HIGH_WORD));
}

__device__ __forceinline__ half8 dequant8(uint32_t dw, const SubScale &lo, const SubScale &hi) {
    const uint32_t l4 = dw & 0x0f0f0f0fu, h4 = (dw >> 4) & 0x0f0f0f0fu;
    const half2_t a0 = __builtin_elementwise_fma(q_pair<false>(l4), lo.mul, lo.add);
    const half2_t a1 = __builtin_elementwise_fma(q_pair<true>(l4), lo.mul, lo.add);
    const half2_t a2 = __builtin_elementwise_fma(q_pair<false>(h4), hi.mul, hi.add);
    const half2_t a3 = __builtin_elementwise_fma(q_pair<true>(h4), hi.mul, hi.add);
    return half8{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
}

}  // namespace

// ---------------------------------------------------------------------------
// A preparation over the padded workspace (rows beyond M are zero).  For
// the 32-row tile T = m / 32 and lane l = m % 32 + 32 h:
//   a16[((T * blocks + b) * 16 + s) * 64 + l]  half8: A[m][k] * 2^-e_m at
//       the 8 columns of step s, half h of block b (frag_base)
//   rowscale[m]                                2^e_m
// ---------------------------------------------------------------------------
// Workgroup (g, p) takes rows 8 g .. 8 g + 7 and blocks 4 p .. 4 p + 3 (for
// K = 4096 a wave keeps its whole row in registers).  Wave w first finds max|A[m]| of row m = 8 g + w over all of K (every workgroup of
// the row group does; they share an XCD, so the repeats hit its L2) and
// writes rowscale[m] = 2^e_m with max|A[m]| 2^-e_m in [2^14, 2^15) (1 for an
// all-zero or non-finite row, 0 for the padding rows m >= M).  The 8 rows'
// fragments of one (block, step, half) are consecutive in a16, so after a
// pass through LDS the 16-byte stores of 8 neighbouring threads form one
// 128-byte line.
constexpr uint32_t kPackBlocks = 4;
constexpr uint32_t kPackLd = kPackBlocks * 128 + 4;  // dwords per staged row

__global__ void __launch_bounds__(512) gemm_prep_kernel(const uint16_t *__restrict__ a, uint32_t m_rows,
                                                        uint32_t k, half8 *__restrict__ a16,
                                                        float *__restrict__ rowscale) {
    __shared__ uint32_t tile[8][kPackLd];
    __shared__ float sdown[8];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const uint32_t r0 = blockIdx.x * 8, blocks = k / 256, b0 = blockIdx.y * kPackBlocks;
    {
        const uint32_t m = r0 + wave;
        const bool live = m < m_rows;
        float mx[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const uint32_t chunks = k / 8;
        if (live && chunks == 64 * 8) {
            // K = 4096: the whole row in registers, the workgroup's blocks
            // staged from them (chunk lane + 64 j holds columns 8 (lane + 64 j) ..)
            const u32x4 *row = (const u32x4 *)(a + (size_t)m * k);
            u32x4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = row[lane + 64 * j];
#pragma unroll
            for (int j = 0; j < 8; j++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    mx[i] = fmaxf(mx[i], fabsf(__uint_as_float(v[j][i] << 16)));
                    mx[i] = fmaxf(mx[i], fabsf(__uint_as_float(v[j][i] & 0xffff0000u)));
                }
                const uint32_t q = lane + 64 * j - b0 * 32;
                if (q < kPackBlocks * 32) *(u32x4 *)&tile[wave][q * 4] = v[j];
            }
        } else if (live) {
            const u32x4 *row = (const u32x4 *)(a + (size_t)m * k);
            uint32_t c = lane;
            for (; c + 64 * 7 < chunks; c += 64 * 8) {
                u32x4 v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = row[c + 64 * j];
#pragma unroll
                for (int j = 0; j < 8; j++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        mx[i] = fmaxf(mx[i], fabsf(__uint_as_float(v[j][i] << 16)));
                        mx[i] = fmaxf(mx[i], fabsf(__uint_as_float(v[j][i] & 0xffff0000u)));
                    }
            }
            for (; c < chunks; c += 64) {
                const u32x4 v = row[c];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    mx[i] = fmaxf(mx[i], fabsf(__uint_as_float(v[i] << 16)));
                    mx[i] = fmaxf(mx[i], fabsf(__uint_as_float(v[i] & 0xffff0000u)));
                }
            }
        }
        float x = wave_max(fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3])));
        int e = 0;
        if (x > 0.0f && __builtin_isfinite(x)) {
            int ex;
            (void)frexpf(x, &ex);
            e = ex - 15;
            if (e < -126) e = -126;
            if (e > 127) e = 127;
        }
        if (lane == 0) {
            sdown[wave] = live ? ldexpf(1.0f, -e) : 0.0f;
            if (blockIdx.y == 0) rowscale[m] = live ? ldexpf(1.0f, e) : 0.0f;
        }
    }
    if (k / 8 != 64 * 8 || r0 + wave >= m_rows) {
        // the workgroup's blocks: thread (row tid >> 6, 16-byte chunk q) of 128 per row
        const uint32_t rr = tid >> 6;
#pragma unroll
        for (uint32_t j = 0; j < kPackBlocks / 2; j++) {
            const uint32_t q = lane + 64 * j, b = b0 + q / 32;
            u32x4 v = {0, 0, 0, 0};
            if (b < blocks && r0 + rr < m_rows) v = *(const u32x4 *)(a + (size_t)(r0 + rr) * k + b0 * 256 + q * 8);
            *(u32x4 *)&tile[rr][q * 4] = v;
        }
    }
    __syncthreads();
    // thread: row i = tid & 7, fragment f = (tid >> 3) & 31 (half h = f / 16,
    // step s = f % 16) of blocks b0 + (tid >> 8) + 2 j
    const uint32_t i = tid & 7u, f = (tid >> 3) & 31u, h = f >> 4, st = f & 15u;
    const float down = sdown[i];
    const uint32_t fb = frag_base(st, h), tl = r0 / 32, l0 = r0 % 32;
#pragma unroll
    for (uint32_t j = 0; j < kPackBlocks / 2; j++) {
        const uint32_t bq = (tid >> 8) + 2 * j, b = b0 + bq;
        if (b >= blocks) continue;
        const uint32_t *t = &tile[i][bq * 128];
        const uint32_t u[4] = {t[fb / 2], t[fb / 2 + 1], t[(fb + 32) / 2], t[(fb + 32) / 2 + 1]};
        half8 v;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            v[2 * q] = (_Float16)(__uint_as_float(u[q] << 16) * down);
            v[2 * q + 1] = (_Float16)(__uint_as_float(u[q] & 0xffff0000u) * down);
        }
        a16[((size_t)(tl * blocks + b) * 16 + st) * 64 + l0 + i + 32 * h] = v;
    }
}

// ---------------------------------------------------------------------------
// Q4_K GEMM main kernel.  Grid: one workgroup per BM x BN tile of C (see
// Tiling).  Wave w owns the BM x WN part w / 4 of the tile over blocks
// w % 4, w % 4 + 4, ...  With BM = 64 two waves share each SIMD: a lone wave
// issues VALU work at half the SIMD's rate, and the dequantization is VALU
// work, so the second wave supplies the other half while the MFMAs run; with
// BM = 128 each dequantized weight serves twice the MFMAs instead.  Per block
// and wave: 16 MFMA steps of RM x 2 MFMAs (32 x 32 tiles), the A fragments of
// step s + kADist in flight during step s, the W block read from the wave's
// LDS area (the next block's W arrives in registers meanwhile).
// ---------------------------------------------------------------------------
template <uint32_t BM>
__global__ void __launch_bounds__(64 * Tiling<BM>::kWaves)
    __attribute__((amdgpu_waves_per_eu(BM == 64 ? 2 : 1, BM == 64 ? 2 : 1))) gemm_q4k_kernel(const half8 *__restrict__ a16,
                                                               const float *__restrict__ rowscale,
                                                               const uint8_t *__restrict__ w, uint32_t m_rows,
                                                               uint32_t n_rows, uint32_t k, uint32_t w_bytes,
                                                               uint32_t m_tiles, float *__restrict__ c) {
    using T = Tiling<BM>;
    constexpr uint32_t kBN = T::kBN, kKSplit = T::kKSplit, kWaves = T::kWaves, kWN = T::kWN, kRM = T::kRM;
    constexpr uint32_t kStageBytes = T::kStageBytes, kStageLoads = T::kStageLoads, kRedLd = T::kRedLd;
    extern __shared__ v4u gsm[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar offsets
    const uint32_t kpart = wave % kKSplit, nh = wave / kKSplit;
    const uint32_t ln = lane & 31u, h = lane >> 5;
    // Tile order.  The 8 XCDs take workgroups round-robin (XCD = id % 8) and
    // each has its own L2.  When the tiles split evenly, XCD x works on M half
    // x % 2 and N quarter x / 2: its half of A (2 MiB at M = 512) stays in
    // its L2, and the workgroups that share a W tile (the M half's m-tiles)
    // run there back to back, so W crosses from HBM twice rather than once
    // per m-tile.  Otherwise m-tile = id % m_tiles.
    const uint32_t id = blockIdx.x, n_tiles = gridDim.x / m_tiles;
    uint32_t mt, nt;
    if (m_tiles % 2 == 0 && n_tiles % 4 == 0) {
        const uint32_t xcd = id % 8, j = id / 8, mh = m_tiles / 2;
        mt = (xcd & 1u) * mh + j % mh;
        nt = (xcd >> 1) * (n_tiles / 4) + j / mh;
    } else {
        mt = id % m_tiles;
        nt = id / m_tiles;
    }
    const uint32_t m0 = mt * BM, n0 = nt * kBN, wn0 = n0 + nh * kWN;
    const uint32_t blocks = k / 256, row_bytes = blocks * 144;
    const uint32_t mine = kpart < blocks ? (blocks - kpart + kKSplit - 1) / kKSplit : 0;

    // Buffer loads: the per-lane part of every address is computed once; the
    // per-block and per-step parts are wave-uniform offsets.  W rows past
    // n_rows start at kNowhere (>= 2^31 > every W offset): they read zeros.
    constexpr uint32_t kNowhere = 0x80000000u;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(w, w_bytes);
    const __amdgpu_buffer_rsrc_t ars = make_rsrc(a16 + (size_t)kRM * mt * blocks * 1024, kRM * blocks * 1024 * 16);
    v4u *stage = gsm + wave * (kStageBytes / 16);

    // W staging: chunk j * 64 + lane of the block's kWN rows x 9 chunks,
    // which is also its 16-byte slot in the staging area.
    uint32_t wbase[kStageLoads];
#pragma unroll
    for (uint32_t j = 0; j < kStageLoads; j++) {
        const uint32_t chunk = j * 64 + lane, r = chunk / 9, p = chunk % 9;
        wbase[j] = wn0 + r < n_rows ? (wn0 + r) * row_bytes + 16 * p : kNowhere;
    }
    v4u wreg[kStageLoads];
    auto fetch_w = [&](uint32_t b) {
#pragma unroll
        for (uint32_t j = 0; j < kStageLoads; j++)
            wreg[j] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(wrs, wbase[j], b * 144, 0));
    };
    auto put_w = [&]() {
#pragma unroll
        for (uint32_t j = 0; j < kStageLoads; j++) stage[j * 64 + lane] = wreg[j];
    };
    // A fragment of row tile r (32 rows), block b, step s.
    auto a_frag = [&](uint32_t r, uint32_t b, uint32_t s) {
        return __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(
                                             ars, 16 * lane, (r * blocks * 1024 + (b * 16 + s) * 64) * 16, 0));
    };
    // LDS slots of the lane's header (column tile t) and of qs group g.
    const v4u *hdr_slot = stage + ln * 9;
    const v4u *q_slot = stage + ln * 9 + 1 + 4 * h;

    floatx16 acc[kRM][2];
#pragma unroll
    for (uint32_t r = 0; r < kRM; r++)
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int j = 0; j < 16; j++) acc[r][t][j] = 0.0f;

    if (mine > 0) {
        uint32_t b = kpart;
        fetch_w(b);
        put_w();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        fetch_w(mine > 1 ? b + kKSplit : b);
        half8 afr[kRM][kADist];
#pragma unroll
        for (uint32_t s = 0; s < kADist; s++)
#pragma unroll
            for (uint32_t r = 0; r < kRM; r++) afr[r][s] = a_frag(r, b, s);
        for (uint32_t i = 0; i < mine; i++, b += kKSplit) {
            const uint32_t bn = i + 1 < mine ? b + kKSplit : b;  // next block (clamped)
            const uint32_t bnn = i + 2 < mine ? b + 2 * kKSplit : bn;
            // Per column tile t (the lane's column 32 t + ln of the wave's
            // half): the scales of the lane's sub-blocks 4 h .. 4 h + 3
            // (src/cpu.rs:607-616).
            v4u hd[2], q[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                hd[t] = hdr_slot[32 * 9 * t];
                q[t] = q_slot[32 * 9 * t];
            }
            SubScale ss[2][4];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hd[t][0] & 0xffffu));
                const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hd[t][0] >> 16));
                // 6-bit scales and mins of sub-blocks 0-3 and 4-7, as bytes
                const uint32_t sc03 = hd[t][1] & 0x3f3f3f3fu, mn03 = hd[t][2] & 0x3f3f3f3fu;
                const uint32_t sc47 = (hd[t][3] & 0x0f0f0f0fu) | ((hd[t][1] >> 2) & 0x30303030u);
                const uint32_t mn47 = ((hd[t][3] >> 4) & 0x0f0f0f0fu) | ((hd[t][2] >> 2) & 0x30303030u);
                const uint32_t scs = h ? sc47 : sc03, mns = h ? mn47 : mn03;
#pragma unroll
                for (int x = 0; x < 4; x++) ss[t][x] = sub_scale(d, dmin, (scs >> (8 * x)) & 0xffu, (mns >> (8 * x)) & 0xffu);
            }
            // Weights of step 0; then each step issues the A loads of step
            // s + kADist, its 2 RM MFMAs, and the weights of step s + 1.  The
            // scheduling barriers keep every step's loads where they are
            // written, so each A fragment (and every older load) has kADist
            // steps to arrive.
            half8 bv[2];
#pragma unroll
            for (int t = 0; t < 2; t++) bv[t] = dequant8(q[t][0], ss[t][0], ss[t][1]);
            v4u qn[2];
#pragma unroll
            for (uint32_t s = 0; s < 16; s++) {
                __builtin_amdgcn_sched_barrier(0);
                if (s % 4 == 0 && s < 12) {
                    // qs group s / 4 + 1 while group s / 4 is used
#pragma unroll
                    for (int t = 0; t < 2; t++) qn[t] = q_slot[32 * 9 * t + s / 4 + 1];
                }
                // The A fragments of step s + kADist (the next block's first
                // steps at the end) and the weights of step s + 1 are produced
                // before this step's MFMAs consume the current ones, so they
                // live in other registers.
                const uint32_t pb = s + kADist < 16 ? b : bn, ps = (s + kADist) % 16;
                half8 an[kRM];
#pragma unroll
                for (uint32_t r = 0; r < kRM; r++) an[r] = a_frag(r, pb, ps);
                half8 bn_[2];
                if (s + 1 < 16) {
                    const uint32_t s1 = s + 1;
                    if (s1 % 4 == 0) {
#pragma unroll
                        for (int t = 0; t < 2; t++) q[t] = qn[t];
                    }
#pragma unroll
                    for (int t = 0; t < 2; t++) bn_[t] = dequant8(q[t][s1 % 4], ss[t][2 * (s1 / 8)], ss[t][2 * (s1 / 8) + 1]);
                }
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (uint32_t r = 0; r < kRM; r++) acc[r][t] = mfma32(afr[r][s % kADist], bv[t], acc[r][t]);
#pragma unroll
                for (uint32_t r = 0; r < kRM; r++) afr[r][s % kADist] = an[r];
                if (s + 1 < 16) {
#pragma unroll
                    for (int t = 0; t < 2; t++) bv[t] = bn_[t];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            // Other lanes read what a lane stores: every LDS read of this
            // block precedes the stores of the next one, which precede its
            // reads (wavefront-scope fences order them for the compiler; the
            // wave's LDS operations execute in order).
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            put_w();
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            fetch_w(bnn);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // Partial tiles -> LDS as [wave][row][column] (row stride kRedLd), after
    // every wave has left its staging area; then each thread adds the four
    // K-split partials of 16 consecutive columns of one row and stores them.
    __syncthreads();
    float *red = (float *)gsm;
#pragma unroll
    for (uint32_t r = 0; r < kRM; r++)
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const uint32_t row = 32 * r + 8 * (j / 4) + 4 * h + (j % 4), col = 32 * t + ln;
                red[(wave * BM + row) * kRedLd + col] = acc[r][t][j];
            }
    __syncthreads();
    // BM rows x BN / 16 chunks of 16 columns, over the workgroup's threads
    constexpr uint32_t kChunks = BM * (kBN / 16);
    for (uint32_t q = tid; q < kChunks; q += 64 * kWaves) {
        const uint32_t row = q / (kBN / 16), col0 = 16 * (q % (kBN / 16));
        const uint32_t half = col0 / kWN, hcol = col0 % kWN;
        const uint32_t m = m0 + row;
        if (m >= m_rows) continue;
        const float scale = rowscale[m];
        const float *src = red + ((half * kKSplit) * BM + row) * kRedLd + hcol;
        float *dst = c + (size_t)m * n_rows + n0 + col0;
        const bool whole = n0 + col0 + 16 <= n_rows && (n_rows & 3u) == 0 && ((uintptr_t)c & 15u) == 0;
#pragma unroll
        for (uint32_t v = 0; v < 4; v++) {
            floatx4 sum = *(const floatx4 *)(src + 4 * v);
#pragma unroll
            for (uint32_t kp = 1; kp < kKSplit; kp++) sum += *(const floatx4 *)(src + kp * BM * kRedLd + 4 * v);
            sum *= scale;
            if (whole) {
                *(floatx4 *)(dst + 4 * v) = sum;
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (n0 + col0 + 4 * v + e < n_rows) dst[4 * v + e] = sum[e];
            }
        }
    }
}

__global__ void bf16_to_f32_kernel(const uint16_t *__restrict__ a, size_t count, float *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = __uint_as_float((uint32_t)a[i] << 16);
}

namespace {

size_t padded_rows(size_t m) { return (m + kPadRows - 1) / kPadRows * kPadRows; }

template <uint32_t BM>
hipError_t launch_gemm(dmhip_ctx *ctx, const half8 *a16, const float *rowscale, const void *weights, size_t m,
                       size_t n, size_t k, uint64_t w_bytes, float *c) {
    using T = Tiling<BM>;
    const uint32_t n_tiles = (uint32_t)((n + T::kBN - 1) / T::kBN), m_tiles = (uint32_t)((m + BM - 1) / BM);
    static LdsLimit limit;
    hipError_t e = limit.ensure((const void *)gemm_q4k_kernel<BM>, T::kLdsBytes);
    if (e != hipSuccess) return e;
    return launch_kernel(ctx, gemm_q4k_kernel<BM>, dim3(n_tiles * m_tiles), dim3(64 * T::kWaves), T::kLdsBytes, a16,
                         rowscale, (const uint8_t *)weights, (uint32_t)m, (uint32_t)n, (uint32_t)k, (uint32_t)w_bytes,
                         m_tiles, c);
}

// Workspace of the Q4_K path: a16 | rowscale.
size_t q4k_workspace(size_t m, size_t k) {
    const size_t mp = padded_rows(m);
    return mp * k * 2 + mp * 4 + 2 * 256;
}

}  // namespace

// A kernel of this file: resolving it loads the file's code object.
const void *module_anchor_gemm() { return (const void *)bf16_to_f32_kernel; }

}  // namespace dm

using namespace dm;

extern "C" {

size_t dmhip_gemm_workspace_bytes(size_t m, size_t k) {
    const size_t tokenwise = m * k * sizeof(float) + 256;
    const size_t q4k = q4k_workspace(m, k);
    return tokenwise > q4k ? tokenwise : q4k;
}

int dmhip_gemm_device(dmhip_ctx *ctx, uint32_t type, size_t m, size_t n, size_t k,
                      const uint16_t *a_bf16, const void *weights, float *c, void *workspace,
                      size_t workspace_len) {
    if (!ctx || !a_bf16 || !weights || !c || !workspace)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "gemm arguments must not be null");
    if (workspace_len < dmhip_gemm_workspace_bytes(m, k))
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "gemm workspace holds %zu bytes; the shape needs %zu",
                    workspace_len, dmhip_gemm_workspace_bytes(m, k));
    if (!(type == 0 || type == 1 || type == 6 || type == 8 || type == 12 || type == 14))
        return fail_unsupported(type, "HIP GEMM");
    uint64_t rb;
    if (!row_byte_len(type, k, &rb)) return fail_element_count(type, k);
    if (m == 0 || n == 0) return DMHIP_OK;
    if (k == 0) return fail_empty("gemm");
    if (m > 0xffffffffull || n > 0xffffffffull || k > 0xffffffffull)
        return fail(DMHIP_ERR_VECTOR_TOO_LARGE, "HIP vector length exceeds the 32-bit kernel limit");
    DM_CHECK_STATUS(set_device(ctx));

    const uint64_t w_bytes = rb * n;
    if (type == kQ4_K && w_bytes + 1024 < 0xffffffffull && ((uintptr_t)weights & 15u) == 0 &&
        ((uintptr_t)a_bf16 & 15u) == 0) {
        const size_t mp = padded_rows(m);
        char *ws = (char *)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
        half8 *a16 = (half8 *)ws;
        float *rowscale = (float *)(ws + ((mp * k * 2 + 255) & ~(size_t)255));
        // row groups along x: a row group's workgroups are x + (mp / 8) y, one XCD
        hipLaunchKernelGGL(gemm_prep_kernel,
                           dim3((uint32_t)(mp / 8), (uint32_t)((k / 256 + kPackBlocks - 1) / kPackBlocks)), dim3(512),
                           0, ctx->stream, a_bf16, (uint32_t)m, (uint32_t)k, a16, rowscale);
        DM_HIP(hipGetLastError());
        // Tiling: 128 x 64 workgroup tiles (four MFMA row tiles per dequantized
        // weight; 9-11% faster than 64 x 128 at C5), 64 x 128 for prefills of
        // at most 64 tokens.
        const uint32_t bm = m > 64 ? 128u : 64u;
        if (bm == 128) {
            DM_HIP(launch_gemm<128>(ctx, a16, rowscale, weights, m, n, k, w_bytes, c));
        } else {
            DM_HIP(launch_gemm<64>(ctx, a16, rowscale, weights, m, n, k, w_bytes, c));
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
