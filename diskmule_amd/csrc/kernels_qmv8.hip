// kernels_qmv8.hip -- int8-MFMA quantized matvec for gfx950: decode batches
// of one or two tokens over Q4_K / Q6_K rows.
//
// y[b][r] = sum_c W[r][c] * x[b][c] (src/cpu.rs:345-399 semantics; the group
// dots are exact integers, the blocks accumulate in fp32).
//
// v_mfma_i32_16x16x64_i8 with a block-diagonal A operand.  In a wave, lane
// (n, g) (n = lane & 15 the row of a 16-row weight tile, g = lane >> 4) holds
// 16 int8 quant codes of its row as the B operand; A row m carries activation
// bytes only in lane group m / 4, zeros elsewhere.  The accumulator element
// C[m][n] (lane n + 16 (m/4), element m % 4) is then the dot of lane
// (n, m/4)'s 16 codes with A row m: every lane receives the exact int32 dots
// of its own code group with up to four activation rows.
//
//  * Weights enter as their raw codes: Q4_K nibbles 0..15, Q6_K 6-bit codes
//    0..63.  No floating-point conversion and no per-weight scale.
//  * Each token is scaled by a power of two so max|x| 2^-e < 2^22 and rounded
//    to integers X = 65536 hi + 256 mid + lo (balanced bytes); A rows
//    4g + {0, 1, 2} carry hi, mid and lo.  Precision: 22 bits relative to the
//    token's largest element.
//  * A group dot is v = (C0 * 256 + C1) * 256 + C2 in fp32, scaled by the
//    group's 6/8-bit scale and the block's d.  Q6_K's "- 32" offset is the
//    exact accumulator seed -32 * sum(X) of the group; Q4_K's
//    "- dmin * m * x" term uses the sub-block sums of X.
//
// The activation records (A fragments plus seeds or sums) are written once
// per call by qmv8_prepare_kernel and staged in LDS by every workgroup.
#include "dm_device.h"
#include "dm_qmv.h"

#include <stdlib.h>

namespace dm {

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kStep8 = 192;  // A bytes of one MFMA step: 4 groups x 3 terms x 16
constexpr uint32_t kZero8 = 1024;  // zeroed LDS bytes read by lanes whose A row is idle
constexpr uint32_t kMaxWaves8 = 16;

// Bytes of one block's record for one token: A fragments of the four steps
// (768), then Q6_K seeds (4 steps x 4 groups x 4 int32) or Q4_K sub-block
// sums (8 floats).
template <uint32_t TYPE> struct Rec8;
template <> struct Rec8<kQ4_K> { static constexpr uint32_t bytes = 4 * kStep8 + 32; };
template <> struct Rec8<kQ6_K> { static constexpr uint32_t bytes = 4 * kStep8 + 256; };

// Column (0..255) of byte i of lane group g's 16 codes at step t.
template <uint32_t TYPE>
__device__ __forceinline__ uint32_t column8(uint32_t t, uint32_t g, uint32_t i) {
    if (TYPE == kQ4_K) return 64 * g + 16 * t + i;  // qs[32g + 16(t&1) + i], nibble t >> 1
    return 128 * (g >> 1) + 32 * t + 16 * (g & 1u) + i;
}

__device__ __forceinline__ float f16_lo(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
}

__device__ __forceinline__ i32x4 mfma8(i32x4 a, i32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// hi * 65536 + mid * 256 + lo as fp32 (C0 * 256 + C1 stays below 2^31).
__device__ __forceinline__ float combine8(i32x4 c) {
    return __builtin_fmaf((float)(c[0] * 256 + c[1]), 256.0f, (float)c[2]);
}

}  // namespace

// ---------------------------------------------------------------------------
// Activation records.  Grid (workgroups per token, tokens); each workgroup
// reduces max|x| over the whole token row, then quantizes four blocks per
// pass: thread l of a 64-thread slice handles step t = l >> 4, lane group
// g = (l >> 2) & 3 and columns 4q .. 4q+3 (q = l & 3) of that group.
// yscale[token] = 2^e, or NaN when the row holds a non-finite value.
// ---------------------------------------------------------------------------
template <uint32_t TYPE>
__global__ void __launch_bounds__(256) qmv8_prepare_kernel(const float *__restrict__ x, uint32_t columns,
                                                           uint32_t batch, uint8_t *__restrict__ xq,
                                                           float *__restrict__ yscale) {
    constexpr uint32_t REC = Rec8<TYPE>::bytes;
    constexpr uint32_t U = 16;
    __shared__ float red_max[4];
    __shared__ uint32_t red_bad[4];
    const uint32_t token = blockIdx.y;
    const float *xt = x + (size_t)token * columns;
    float mx = 0.0f;
    uint32_t bad = 0;
    for (uint32_t i0 = 0; i0 < columns; i0 += 256 * U) {
        float v[U];
#pragma unroll
        for (uint32_t j = 0; j < U; j++) {
            const uint32_t i = i0 + 256 * j + threadIdx.x;
            v[j] = i < columns ? xt[i] : 0.0f;
        }
#pragma unroll
        for (uint32_t j = 0; j < U; j++) {
            bad |= !__builtin_isfinite(v[j]);
            mx = fmaxf(mx, fabsf(v[j]));
        }
    }
    mx = wave_max(mx);
    bad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;
    if ((threadIdx.x & 63u) == 0) {
        red_max[threadIdx.x >> 6] = mx;
        red_bad[threadIdx.x >> 6] = bad;
    }
    __syncthreads();
    mx = fmaxf(fmaxf(red_max[0], red_max[1]), fmaxf(red_max[2], red_max[3]));
    bad = red_bad[0] | red_bad[1] | red_bad[2] | red_bad[3];
    int e = 0;
    if (!bad && mx > 0.0f) {
        int ex;
        (void)frexpf(mx, &ex);  // mx < 2^ex
        e = ex - 22;
        if (e < -126) e = -126;
        if (e > 127) e = 127;
    }
    const float down = ldexpf(1.0f, -e);
    if (blockIdx.x == 0 && threadIdx.x == 0)
        yscale[token] = bad ? __builtin_nanf("") : ldexpf(1.0f, e);

    const uint32_t blocks = columns / 256;
    const uint32_t l = threadIdx.x & 63u, t = l >> 4, g = (l >> 2) & 3u, q = l & 3u;
    for (uint32_t b = blockIdx.x * 4 + (threadIdx.x >> 6); b < blocks; b += gridDim.x * 4) {
        const float *xb = xt + (size_t)b * 256 + column8<TYPE>(t, g, 4 * q);
        uint32_t term[3] = {0, 0, 0};
        int sum[3] = {0, 0, 0}, sx = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int X = bad ? 0 : (int)rintf(xb[j] * down);  // |X| <= 2^22
            const int lo = (int)(int8_t)(X & 0xff);
            const int x1 = (X - lo) >> 8;
            const int mid = (int)(int8_t)(x1 & 0xff);
            const int hi = (x1 - mid) >> 8;
            term[0] |= (uint32_t)(hi & 0xff) << (8 * j);
            term[1] |= (uint32_t)(mid & 0xff) << (8 * j);
            term[2] |= (uint32_t)(lo & 0xff) << (8 * j);
            sum[0] += hi;
            sum[1] += mid;
            sum[2] += lo;
            sx += X;
        }
        uint8_t *rec = xq + ((size_t)b * batch + token) * REC;
#pragma unroll
        for (int k = 0; k < 3; k++) *(uint32_t *)(rec + t * kStep8 + (g * 3 + k) * 16 + 4 * q) = term[k];
        if (TYPE == kQ6_K) {
            // group (t, g) = the four adjacent threads q = 0..3
#pragma unroll
            for (int k = 0; k < 3; k++) {
                sum[k] += __shfl_xor(sum[k], 1, 64);
                sum[k] += __shfl_xor(sum[k], 2, 64);
            }
            if (q == 0) {
                const i32x4 seed = {-32 * sum[0], -32 * sum[1], -32 * sum[2], 0};
                *(i32x4 *)(rec + 4 * kStep8 + (t * 4 + g) * 16) = seed;
            }
        } else {
            // sub-block 2g + (t >> 1) = threads (t, g, q) and (t ^ 1, g, q)
            sx += __shfl_xor(sx, 1, 64);
            sx += __shfl_xor(sx, 2, 64);
            sx += __shfl_xor(sx, 16, 64);
            if (q == 0 && (t & 1u) == 0) *(float *)(rec + 4 * kStep8 + (2 * g + (t >> 1)) * 4) = (float)sx;
        }
    }
}

namespace {

// Raw bytes of one block of one row as a lane holds them.
template <uint32_t TYPE> struct Raw8;
template <> struct Raw8<kQ4_K> {
    u32x4 hdr, q0, q1;  // d|dmin|scales; qs bytes [32g, 32g+16) and [32g+16, 32g+32)
};
template <> struct Raw8<kQ6_K> {
    u32x4 a1, a2, a3, a4;      // aligned dwords under ql[64h+16c], ql[64h+32+16c], qh[32h+16c], scales
    uint32_t e1, e2, e3, e4;   // the dword after each (e4 also holds d)
    uint32_t s;                // block start mod 4 (0 or 2)
};

// Staging of one 16-row tile's block in LDS.  Row r of the tile occupies
// `chunks` 16-byte chunks: the aligned chunks of global memory that cover
// its block (Q4_K blocks start 16-aligned; a Q6_K block starts s16 = 0..14
// bytes into its first chunk).  Consecutive lanes load consecutive chunks of
// a row, so each quad of lanes reads one contiguous 64-byte span; the lanes
// then read their own pieces of their own row from LDS.
template <uint32_t TYPE> struct Stage8;
template <> struct Stage8<kQ4_K> { static constexpr uint32_t chunks = 9; };
template <> struct Stage8<kQ6_K> { static constexpr uint32_t chunks = 15; };
template <uint32_t TYPE> constexpr uint32_t stage_loads8() { return (16 * Stage8<TYPE>::chunks + 63) / 64; }
// One wave's staging area (every lane of every load writes one chunk).
template <uint32_t TYPE> constexpr uint32_t stage_bytes8() { return stage_loads8<TYPE>() * 64 * 16; }

typedef uint32_t v4u __attribute__((ext_vector_type(4)));  // 16-byte aligned (LDS)

__device__ __forceinline__ u32x4 as_u32x4(v4u v) { return __builtin_bit_cast(u32x4, v); }

// Lane (n, g)'s pieces of row n's block from the staging area.  `start` is
// the block's global byte offset (its low four bits locate it in the chunk).
template <uint32_t TYPE>
__device__ __forceinline__ void take8(const v4u *stage, uint32_t n, uint32_t g, uint32_t start, Raw8<TYPE> &raw);

template <>
__device__ __forceinline__ void take8<kQ4_K>(const v4u *stage, uint32_t n, uint32_t g, uint32_t,
                                             Raw8<kQ4_K> &raw) {
    const v4u *sr = stage + n * Stage8<kQ4_K>::chunks;
    raw.hdr = as_u32x4(sr[0]);
    raw.q0 = as_u32x4(sr[1 + 2 * g]);
    raw.q1 = as_u32x4(sr[2 + 2 * g]);
}

template <>
__device__ __forceinline__ void take8<kQ6_K>(const v4u *stage, uint32_t n, uint32_t g, uint32_t start,
                                             Raw8<kQ6_K> &raw) {
    const uint32_t s16 = start & 15u;
    // dwords of row n from the one holding the block's first byte
    const uint32_t *sw = (const uint32_t *)(stage + n * Stage8<kQ6_K>::chunks) + (s16 >> 2);
    const uint32_t h = g >> 1, c = g & 1u;
    const uint32_t o1 = 16 * h + 4 * c, o2 = o1 + 8, o3 = 32 + 8 * h + 4 * c;
    raw.s = s16 & 3u;
    raw.a1 = u32x4{sw[o1], sw[o1 + 1], sw[o1 + 2], sw[o1 + 3]};
    raw.a2 = u32x4{sw[o2], sw[o2 + 1], sw[o2 + 2], sw[o2 + 3]};
    raw.a3 = u32x4{sw[o3], sw[o3 + 1], sw[o3 + 2], sw[o3 + 3]};
    raw.a4 = u32x4{sw[48], sw[49], sw[50], sw[51]};
    raw.e1 = sw[o1 + 4];
    raw.e2 = sw[o2 + 4];
    raw.e3 = sw[o3 + 4];
    raw.e4 = sw[52];
}

// The block's contribution to acc[token].  `lds` is the staged record area;
// a_off / a_stride address this lane's A fragment of token 0 at step 0 (the
// zeroed region, stride 0, for idle lanes); rec is the block's first record.
template <int TOK>
__device__ __forceinline__ void block_dot8(const Raw8<kQ4_K> &raw, const i32x4 *lds, uint32_t a_off,
                                           uint32_t a_stride, uint32_t rec, uint32_t g, float (&acc)[TOK]) {
    constexpr uint32_t REC = Rec8<kQ4_K>::bytes;
    const u32x4 hdr = raw.hdr;
    const float d = f16_lo(hdr[0]);
    const float dmin = f16_lo(hdr[0] >> 16);
    // (scale, min) of sub-blocks 2g and 2g+1 (src/cpu.rs:607-616): for
    // sub-block j < 4 the low 6 bits of scales[j], scales[j+4]; for j >= 4
    // nibbles of scales[j+4] with the top bits of scales[j-4], scales[j].
    const bool high_half = g >= 2;
    float sc[2], mn[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t sh = 8 * ((2 * g + j) & 3u);
        const uint32_t b1 = hdr[1] >> sh, b2 = hdr[2] >> sh, b3 = hdr[3] >> sh;
        const uint32_t sc_lo = b1 & 63u, mn_lo = b2 & 63u;
        const uint32_t sc_hi = (b3 & 15u) | ((b1 >> 2) & 0x30u);
        const uint32_t mn_hi = ((b3 >> 4) & 15u) | ((b2 >> 2) & 0x30u);
        sc[j] = (float)(high_half ? sc_hi : sc_lo);
        mn[j] = (float)(high_half ? mn_hi : mn_lo);
    }
    constexpr uint32_t M4 = 0x0f0f0f0fu;
    const i32x4 b0 = __builtin_bit_cast(i32x4, raw.q0 & M4);
    const i32x4 b1 = __builtin_bit_cast(i32x4, raw.q1 & M4);
    const i32x4 b2 = __builtin_bit_cast(i32x4, (raw.q0 >> 4) & M4);
    const i32x4 b3 = __builtin_bit_cast(i32x4, (raw.q1 >> 4) & M4);
    const i32x4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int tok = 0; tok < TOK; tok++) {
        const uint32_t a = (a_off + tok * a_stride) / 16;
        i32x4 c_lo = mfma8(lds[a], b0, zero);
        c_lo = mfma8(lds[a + kStep8 / 16], b1, c_lo);
        i32x4 c_hi = mfma8(lds[a + 2 * kStep8 / 16], b2, zero);
        c_hi = mfma8(lds[a + 3 * kStep8 / 16], b3, c_hi);
        const float *sums = (const float *)lds + (rec + tok * REC + 4 * kStep8) / 4 + 2 * g;
        const float part = __builtin_fmaf(sc[1], combine8(c_hi), sc[0] * combine8(c_lo));
        const float mins = __builtin_fmaf(mn[1], sums[1], mn[0] * sums[0]);
        acc[tok] = __builtin_fmaf(d, part, acc[tok]);
        acc[tok] = __builtin_fmaf(-dmin, mins, acc[tok]);
    }
}

template <int TOK>
__device__ __forceinline__ void block_dot8(const Raw8<kQ6_K> &raw, const i32x4 *lds, uint32_t a_off,
                                           uint32_t a_stride, uint32_t rec, uint32_t g, float (&acc)[TOK]) {
    constexpr uint32_t REC = Rec8<kQ6_K>::bytes;
    const uint32_t s = raw.s;
    uint32_t L0[4], L1[4], H[4], W[4];
    if (__builtin_amdgcn_ballot_w64(s != 0) == 0) {
        // every row of the tile starts this block on a dword boundary
#pragma unroll
        for (int i = 0; i < 4; i++) {
            L0[i] = raw.a1[i];
            L1[i] = raw.a2[i];
            H[i] = raw.a3[i];
            W[i] = raw.a4[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            L0[i] = funnel(raw.a1[i], i < 3 ? raw.a1[i + 1] : raw.e1, s);
            L1[i] = funnel(raw.a2[i], i < 3 ? raw.a2[i + 1] : raw.e2, s);
            H[i] = funnel(raw.a3[i], i < 3 ? raw.a3[i + 1] : raw.e3, s);
            W[i] = funnel(raw.a4[i], i < 3 ? raw.a4[i + 1] : raw.e4, s);
        }
    }
    // d sits at block offset 208: bytes 0-1 of e4, or 2-3 when s == 2.
    const float d = f16_lo(s ? raw.e4 >> 16 : raw.e4);
    // int8 scales sc[8h + 2t + c]: byte 2(t&1) + c of scale word 2h + (t>>1).
    const uint32_t h = g >> 1, c = g & 1u;
    const uint32_t sw0 = h ? W[2] : W[0], sw1 = h ? W[3] : W[1];
    float sc[4];
#pragma unroll
    for (int t = 0; t < 4; t++) sc[t] = (float)(int)(int8_t)((t < 2 ? sw0 : sw1) >> (16 * (t & 1) + 8 * c));
    // 6-bit codes of step t (elements 128h + 32t + 16c + i): low nibble of
    // ql (t = 0, 1) or its high nibble (t = 2, 3), with qh bits 2t..2t+1 as
    // bits 4-5.
    constexpr uint32_t M4 = 0x0f0f0f0fu, M2 = 0x30303030u;
    i32x4 b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        b[0][i] = (int)((L0[i] & M4) | ((H[i] << 4) & M2));
        b[1][i] = (int)((L1[i] & M4) | ((H[i] << 2) & M2));
        b[2][i] = (int)(((L0[i] >> 4) & M4) | (H[i] & M2));
        b[3][i] = (int)(((L1[i] >> 4) & M4) | ((H[i] >> 2) & M2));
    }
#pragma unroll
    for (int tok = 0; tok < TOK; tok++) {
        const uint32_t a = (a_off + tok * a_stride) / 16;
        const uint32_t seeds = (rec + tok * REC + 4 * kStep8) / 16 + g;
        float part = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const i32x4 cc = mfma8(lds[a + t * (kStep8 / 16)], b[t], lds[seeds + 4 * t]);
            part = __builtin_fmaf(sc[t], combine8(cc), part);
        }
        acc[tok] = __builtin_fmaf(d, part, acc[tok]);
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Main kernel.  WAVES = max(8, S) waves per workgroup; S waves split the
// blocks of one 16-row tile, so a workgroup covers WAVES / S tiles.
// Dynamic LDS: activation records | zeroed region | per-wave staging.
// MODE 0: y = W x.  MODE 1 (one token): also one ArgmaxPartial per tile.
// ---------------------------------------------------------------------------
template <uint32_t TYPE, int S, int MODE, int TOK>
__global__ void __launch_bounds__(64 * (S > 8 ? S : 8)) qmv8_kernel(
    const uint8_t *__restrict__ w, uint32_t rows, uint32_t columns, uint32_t row_bytes,
    uint32_t total_bytes, const uint8_t *__restrict__ xq, const float *__restrict__ yscale,
    float *__restrict__ y, ArgmaxPartial *__restrict__ partials) {
    constexpr uint32_t WAVES = S > 8 ? S : 8;
    constexpr uint32_t REC = Rec8<TYPE>::bytes;
    constexpr uint32_t BB = TYPE == kQ4_K ? 144u : 210u;
    constexpr uint32_t CH = Stage8<TYPE>::chunks, NL = stage_loads8<TYPE>();
    extern __shared__ i32x4 lds8[];
    __shared__ float red[S > 1 ? WAVES * 64 * TOK : 1];
    __shared__ float tscale[TOK];

    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t group = wave / S, kpart = wave % S;
    const uint32_t tile = blockIdx.x * (WAVES / S) + group;
    const uint32_t blocks = columns / 256;
    const uint32_t rec_bytes = blocks * TOK * REC;
    v4u *stage = (v4u *)((uint8_t *)lds8 + rec_bytes + kZero8) + wave * (NL * 64);

    // Whole dwords: the last dword of the matrix may extend up to 3 bytes past
    // its end (inside the allocation's granularity); loads beyond it read 0.
    const uint32_t records = (total_bytes + 3u) & ~3u;
    const uint32_t nowhere = records + 256;  // every load from here reads 0
    const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(w, records);
    const uint32_t row = tile * 16 + n;
    const uint32_t row_base = row < rows ? row * row_bytes : nowhere;

    // Chunk j*64 + lane of the staging area: row r, chunk c of the tile.
    uint32_t src_row[NL], src_chunk[NL];
#pragma unroll
    for (uint32_t j = 0; j < NL; j++) {
        const uint32_t item = j * 64 + lane, r = item / CH, c = item % CH;
        const uint32_t rr = tile * 16 + r;
        src_row[j] = (item < 16 * CH && rr < rows) ? rr * row_bytes : nowhere;
        src_chunk[j] = 16 * c;
    }
    v4u st[NL];
    auto fetch = [&](uint32_t blk) {
#pragma unroll
        for (uint32_t j = 0; j < NL; j++) {
            const uint32_t off = src_row[j] == nowhere ? nowhere : ((src_row[j] + blk * BB) & ~15u) + src_chunk[j];
            st[j] = __builtin_bit_cast(v4u, rsrc_load16(rsrc, off));
        }
    };

    // Wave kpart takes blocks kpart, kpart + S, ...: the S waves of a tile
    // read S consecutive blocks of each row at a time.  The first block is
    // requested before the activation records are staged.
    const uint32_t b_begin = kpart;
    if (b_begin < blocks) fetch(b_begin);

    {
        const i32x4 *src = (const i32x4 *)xq;
        for (uint32_t i = threadIdx.x; i < rec_bytes / 16; i += 64 * WAVES) lds8[i] = src[i];
        for (uint32_t i = threadIdx.x; i < kZero8 / 16; i += 64 * WAVES) lds8[rec_bytes / 16 + i] = i32x4{0, 0, 0, 0};
        if (threadIdx.x < (uint32_t)TOK) tscale[threadIdx.x] = yscale[threadIdx.x];
        __syncthreads();
    }
    // A row n of the MFMA: live when it is term n % 4 (< 3) of lane group n / 4.
    const uint32_t term = n & 3u;
    const bool a_live = (n >> 2) == g && term < 3;
    const uint32_t a_base = a_live ? (g * 3 + term) * 16 : rec_bytes;
    const uint32_t a_stride = a_live ? REC : 0;

    float acc[TOK];
#pragma unroll
    for (int tok = 0; tok < TOK; tok++) acc[tok] = 0.0f;

    // The chunks of block blk go to the wave's staging area; the loads of
    // the next block are in flight while this one is read back and computed.
    // A wave only reads its own staging area, and its LDS operations run in
    // order, so no barrier is needed.
    for (uint32_t blk = b_begin; blk < blocks; blk += S) {
#pragma unroll
        for (uint32_t j = 0; j < NL; j++) stage[j * 64 + lane] = st[j];
        if (blk + S < blocks) fetch(blk + S);
        Raw8<TYPE> raw;
        take8<TYPE>(stage, n, g, row_base == nowhere ? 0u : row_base + blk * BB, raw);
        block_dot8<TOK>(raw, lds8, a_base + blk * TOK * a_stride, a_stride, blk * TOK * REC, g, acc);
    }

    // The four lane groups of row n hold disjoint parts of its dot.
#pragma unroll
    for (int tok = 0; tok < TOK; tok++) {
        acc[tok] += __shfl_xor(acc[tok], 16, 64);
        acc[tok] += __shfl_xor(acc[tok], 32, 64);
    }
    if constexpr (S > 1) {
#pragma unroll
        for (int tok = 0; tok < TOK; tok++) red[(wave * 64 + lane) * TOK + tok] = acc[tok];
        __syncthreads();
        if (kpart != 0) return;
#pragma unroll
        for (int tok = 0; tok < TOK; tok++) {
            float v = 0.0f;
            for (int p = 0; p < S; p++) v += red[((wave + p) * 64 + lane) * TOK + tok];
            acc[tok] = v;
        }
    }

    uint64_t best = 0;
    uint32_t bad = 0;
    if (g < (uint32_t)TOK && row < rows) {
        const float v = (TOK == 1 || g == 0 ? acc[0] : acc[TOK - 1]) * tscale[g];
        y[(size_t)g * rows + row] = v;
        if constexpr (MODE == 1) {
            bad = !__builtin_isfinite(v);
            best = argmax_key(v, row);
        }
    }
    if constexpr (MODE == 1) {
        best = wave_max_u64(best);
        bad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;
        if (lane == 0) {
            ArgmaxPartial p;
            p.key = best;
            p.non_finite = bad;
            p.pad = 0;
            partials[tile] = p;
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

namespace {

constexpr size_t kMaxLds8 = 64 * 1024;

// Dynamic LDS of one workgroup: records, zeroed region, staging per wave.
size_t lds8_bytes(uint32_t type, uint32_t blocks, uint32_t batch, uint32_t waves) {
    const size_t rec = type == kQ4_K ? Rec8<kQ4_K>::bytes : Rec8<kQ6_K>::bytes;
    const size_t stage = type == kQ4_K ? stage_bytes8<kQ4_K>() : stage_bytes8<kQ6_K>();
    return (size_t)blocks * batch * rec + kZero8 + (size_t)waves * stage;
}

// Split of each tile's blocks over S waves: enough waves to keep every SIMD
// busy, at least two blocks per wave, and the workgroup's LDS (dynamic plus
// the split-K scratch) within 64 KiB.  DMHIP_QMV8_SPLIT (1..16, a power of
// two) overrides the wave-count rule for tuning.  Returns 0 when no split
// fits.
uint32_t plan_split8(uint32_t type, uint32_t rows, uint32_t columns, uint32_t batch) {
    static const int forced = [] {
        const char *v = getenv("DMHIP_QMV8_SPLIT");
        return v ? atoi(v) : 0;
    }();
    const uint32_t tiles = (rows + 15) / 16, blocks = columns / 256;
    uint32_t s = 1;
    if (forced == 1 || forced == 2 || forced == 4 || forced == 8 || forced == 16) {
        s = (uint32_t)forced;
    } else {
        while (s < kMaxWaves8 && (size_t)tiles * s < 4096 && blocks >= 4 * s) s *= 2;
    }
    for (; s >= 1; s /= 2) {
        const uint32_t waves = s > 8 ? s : 8;
        const size_t stat = (s > 1 ? (size_t)waves * 64 * batch * sizeof(float) : 4) + 64;
        if (lds8_bytes(type, blocks, batch, waves) + stat <= kMaxLds8) return s;
    }
    return 0;
}

template <uint32_t TYPE, int S, int MODE, int TOK>
hipError_t run8(dmhip_ctx *ctx, uint32_t rows, uint32_t columns, const void *w, const uint8_t *xq,
                const float *ysc, float *y, ArgmaxPartial *partials, uint32_t *count) {
    constexpr uint32_t WAVES = S > 8 ? S : 8;
    const uint32_t tiles = (rows + 15) / 16, per = WAVES / S;
    const uint32_t grid = (tiles + per - 1) / per;
    const uint32_t blocks = columns / 256;
    const uint32_t row_bytes = blocks * (TYPE == kQ4_K ? 144u : 210u);
    if (count) *count = grid * per;
    KernelTimer timer(ctx);
    hipLaunchKernelGGL((qmv8_kernel<TYPE, S, MODE, TOK>), dim3(grid), dim3(64 * WAVES),
                       lds8_bytes(TYPE, blocks, TOK, WAVES), ctx->stream, (const uint8_t *)w, rows, columns,
                       row_bytes, row_bytes * rows, xq, ysc, y, partials);
    return hipGetLastError();
}

template <uint32_t TYPE, int MODE, int TOK>
hipError_t run8_s(dmhip_ctx *ctx, uint32_t s, uint32_t rows, uint32_t columns, const void *w,
                  const uint8_t *xq, const float *ysc, float *y, ArgmaxPartial *partials, uint32_t *count) {
    switch (s) {
    case 1: return run8<TYPE, 1, MODE, TOK>(ctx, rows, columns, w, xq, ysc, y, partials, count);
    case 2: return run8<TYPE, 2, MODE, TOK>(ctx, rows, columns, w, xq, ysc, y, partials, count);
    case 4: return run8<TYPE, 4, MODE, TOK>(ctx, rows, columns, w, xq, ysc, y, partials, count);
    case 8: return run8<TYPE, 8, MODE, TOK>(ctx, rows, columns, w, xq, ysc, y, partials, count);
    default: return run8<TYPE, 16, MODE, TOK>(ctx, rows, columns, w, xq, ysc, y, partials, count);
    }
}

template <uint32_t TYPE>
hipError_t launch8(dmhip_ctx *ctx, uint32_t rows, uint32_t columns, const void *w, uint32_t batch,
                   const float *x, float *y, ArgmaxPartial *partials, uint32_t *count) {
    const uint32_t blocks = columns / 256;
    const size_t rec_bytes = (size_t)blocks * batch * Rec8<TYPE>::bytes;
    const size_t xq_bytes = (rec_bytes + 255) & ~(size_t)255;
    if (ctx->aux.ensure(xq_bytes + 64 * sizeof(float)) != DMHIP_OK) return hipErrorOutOfMemory;
    uint8_t *xq = (uint8_t *)ctx->aux.ptr;
    float *ysc = (float *)((char *)ctx->aux.ptr + xq_bytes);
    uint32_t gx = (blocks + 3) / 4;
    if (gx > 16) gx = 16;
    hipLaunchKernelGGL(qmv8_prepare_kernel<TYPE>, dim3(gx, batch), dim3(256), 0, ctx->stream, x, columns,
                       batch, xq, ysc);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t s = plan_split8(TYPE, rows, columns, batch);
    if (s == 0) return hipErrorInvalidValue;
    if (partials) return run8_s<TYPE, 1, 1>(ctx, s, rows, columns, w, xq, ysc, y, partials, count);
    if (batch == 1) return run8_s<TYPE, 0, 1>(ctx, s, rows, columns, w, xq, ysc, y, nullptr, nullptr);
    return run8_s<TYPE, 0, 2>(ctx, s, rows, columns, w, xq, ysc, y, nullptr, nullptr);
}

}  // namespace

bool qmv8_supported(uint32_t type, size_t rows, size_t columns, size_t batch) {
    if (type != kQ4_K && type != kQ6_K) return false;
    if (batch < 1 || batch > 2 || columns % 256 || columns == 0) return false;
    return plan_split8(type, (uint32_t)rows, (uint32_t)columns, (uint32_t)batch) != 0;
}

hipError_t launch_qmv8(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns, const void *w,
                       uint32_t batch, const float *x, float *y, ArgmaxPartial *partials, uint32_t *count) {
    if (type == kQ4_K) return launch8<kQ4_K>(ctx, rows, columns, w, batch, x, y, partials, count);
    return launch8<kQ6_K>(ctx, rows, columns, w, batch, x, y, partials, count);
}

}  // namespace dm
