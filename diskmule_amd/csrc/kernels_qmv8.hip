// kernels_qmv8.hip -- int8-MFMA quantized matvec for gfx950: decode batches
// of one to four tokens over Q4_K / Q6_K / Q8_0 rows.
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
//    0..63, Q8_0 signed bytes.  No floating-point conversion and no
//    per-weight scale.  A Q8_0 row is handled in 256-value super-blocks of 8
//    blocks (272 bytes); lane group g holds blocks 2g and 2g + 1, each step
//    within one block, whose d scales that step's dot.
//  * Each 256-value block of a token is scaled by its own power of two so
//    max|x| 2^-e < 2^22 over the block and rounded to integers
//    X = 65536 hi + 256 mid + lo (balanced bytes); A rows 4g + {0, 1, 2} carry
//    hi, mid and lo.  Precision: 22 bits relative to the block's largest
//    element; 2^e multiplies the block's result.
//  * A group dot is v = (C0 * 256 + C1) * 256 + C2 in fp32, scaled by the
//    group's 6/8-bit scale and the block's d.  Q6_K's "- 32" offset is the
//    exact accumulator seed -32 * sum(X) of the group; Q4_K's
//    "- dmin * m * x" term uses the sub-block sums of X.
//
// Every workgroup quantizes the tokens into activation records (A fragments
// plus seeds or sums) in its own LDS, then streams weight tiles.  Weight bytes
// go through a per-wave LDS staging area so that the global loads are fully
// coalesced.
#include "dm_device.h"
#include "dm_qmv.h"


namespace dm {

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kStep8 = 192;  // A bytes of one MFMA step: 4 groups x 3 terms x 16
constexpr uint32_t kZero8 = 1024;  // zeroed LDS bytes read by lanes whose A row is idle
constexpr int kNonTemporal = 2;     // buffer load cache policy: NT (no reuse expected)
constexpr uint32_t kMaxWaves8 = 16;
// Tokens per launch: lane group g writes token g.  A batch's records must
// fit the workgroup's LDS with the staging areas (plan8), which bounds the
// row length: 4 tokens of Q4_K rows up to about 8192 columns.
constexpr uint32_t kMaxTokens8 = 4;

// Bytes of one block's record for one token: A fragments of the four steps
// (768), then Q6_K seeds (4 steps x 4 groups x 4 int32) or Q4_K sub-block
// sums (8 floats), then the block's activation scale 2^e (a float, padded to
// 16 bytes).
template <uint32_t TYPE> struct Rec8;
template <> struct Rec8<kQ4_K> { static constexpr uint32_t bytes = 4 * kStep8 + 32 + 16; };
template <> struct Rec8<kQ6_K> { static constexpr uint32_t bytes = 4 * kStep8 + 256 + 16; };
template <> struct Rec8<kQ8_0> { static constexpr uint32_t bytes = 4 * kStep8 + 16; };

// Bytes of one 256-value block (Q8_0: 8 blocks of 34).
template <uint32_t TYPE> constexpr uint32_t kBlock8 = TYPE == kQ4_K ? 144u : TYPE == kQ6_K ? 210u : 272u;

// Column (0..255) of byte i of lane group g's 16 codes at step t.
template <uint32_t TYPE>
__device__ __forceinline__ uint32_t column8(uint32_t t, uint32_t g, uint32_t i) {
    if (TYPE == kQ4_K) return 64 * g + 16 * t + i;  // qs[32g + 16(t&1) + i], nibble t >> 1
    if (TYPE == kQ8_0) return 64 * g + 16 * t + i;  // block 2g + t/2, codes 16(t&1) + i
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

namespace {

// Activation records of TOK tokens (token t at x + t * x_stride) written by
// the workgroup into LDS at `rec` (record of block b, token t at
// (b * TOK + t) * REC).  Wave k handles
// blocks k, k + WAVES, ...: lane l takes the four values of step t = l >> 4,
// lane group g = (l >> 2) & 3, columns 4q .. 4q+3 (q = l & 3) of the block,
// and the block gets its own power-of-two scale 2^e (max|x| 2^-e < 2^22 over
// the block; a wave-wide maximum, no barrier).  The scale is stored after the
// record; it is NaN when the block holds a non-finite value, which makes
// every output of that token NaN.  With NORM each wave also leaves its part
// of sum(x^2) per token in red_ss[tok * WAVES + wave].
//
// The values of a wave's first XP blocks are loaded by preload_x8 before the
// kernel requests its weights: a wave's loads complete in the order they were
// issued, so activations requested after the weights could only be used
// once the weights had arrived.
template <int TOK, int XP> struct XPre8 {
    floatx4 v[TOK][XP > 0 ? XP : 1];
};

template <uint32_t TYPE, int TOK, uint32_t WAVES, int XP>
__device__ __forceinline__ void preload_x8(const float *__restrict__ x, int x_stride, uint32_t columns,
                                           XPre8<TOK, XP> &pre) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t blocks = columns / 256;
    const uint32_t t = lane >> 4, g = (lane >> 2) & 3u, q = lane & 3u;
#pragma unroll
    for (int tok = 0; tok < TOK; tok++)
#pragma unroll
        for (int i = 0; i < XP; i++) {
            // No branch around the loads: a branch that may skip a load makes
            // every later wait on the wave's loads wait for all of them.
            const uint32_t b = wave + (uint32_t)i * WAVES;
            const uint32_t bc = b < blocks ? b : 0u;
            // Written as the instruction: the compiler sinks a plain load to
            // its first use, behind the weight loads.  wait_x8 waits for it.
            const float *xb = x + (ptrdiff_t)tok * x_stride + (size_t)bc * 256 + column8<TYPE>(t, g, 4 * q);
            asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(pre.v[tok][i]) : "v"(xb) : "memory");
        }
}

// Waits until at most `later` vector-memory loads issued after the preload
// are outstanding (loads complete in order, so the preload has landed).  The
// values are operands of the wait, so no use of them can move above it, and
// the memory clobbers of the loads and the wait keep every other memory
// operation out of the span between them: exactly the `later` weight loads
// of the first fetch lie in it.
template <uint32_t later, int TOK, int XP>
__device__ __forceinline__ void wait_x8(XPre8<TOK, XP> &pre) {
    static_assert(later < 64, "vmcnt is 6 bits");
    constexpr int N = TOK * XP;
    static_assert(N >= 0 && N <= 4, "0 to 4 preloaded blocks");
    // preloaded block i is pre.v[i / XP][i % XP]
    constexpr int D = XP > 0 ? XP : 1;
    floatx4 &a = pre.v[0][0];
    floatx4 &b = pre.v[(N > 1 ? 1 : 0) / D][(N > 1 ? 1 : 0) % D];
    floatx4 &c = pre.v[(N > 2 ? 2 : 0) / D][(N > 2 ? 2 : 0) % D];
    floatx4 &d = pre.v[(N > 3 ? 3 : 0) / D][(N > 3 ? 3 : 0) % D];
    if constexpr (N == 0) {
        // nothing preloaded
    } else if constexpr (N == 1) {
        asm volatile("s_waitcnt vmcnt(%1)" : "+v"(a) : "n"(later) : "memory");
    } else if constexpr (N == 2) {
        asm volatile("s_waitcnt vmcnt(%2)" : "+v"(a), "+v"(b) : "n"(later) : "memory");
    } else if constexpr (N == 3) {
        asm volatile("s_waitcnt vmcnt(%3)" : "+v"(a), "+v"(b), "+v"(c) : "n"(later) : "memory");
    } else {
        asm volatile("s_waitcnt vmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(later) : "memory");
    }
}

template <uint32_t TYPE, int TOK, uint32_t WAVES, bool NORM, int XP>
__device__ __forceinline__ void build_records8(const float *__restrict__ x, int x_stride, uint32_t columns,
                                               uint8_t *rec, float *red_ss, const XPre8<TOK, XP> &pre) {
    constexpr uint32_t REC = Rec8<TYPE>::bytes;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t blocks = columns / 256;
    const uint32_t t = lane >> 4, g = (lane >> 2) & 3u, q = lane & 3u;
#pragma unroll
    for (int tok = 0; tok < TOK; tok++) {
        float ss = 0.0f;
        // `store` false: computed for a block past the end (a clamped
        // preload), nothing written.
        auto record = [&](uint32_t b, const floatx4 vin, bool store) {
            float v[4];
            float mx = 0.0f;
            uint32_t bad = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[j] = vin[j];
                bad |= !__builtin_isfinite(v[j]);
                mx = fmaxf(mx, fabsf(v[j]));
                if (NORM && store) ss = __builtin_fmaf(v[j], v[j], ss);
            }
            mx = wave_max(mx);
            bad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;
            int e = 0;
            if (!bad && mx > 0.0f) {
                int ex;
                (void)frexpf(mx, &ex);  // mx < 2^ex
                e = ex - 22;
                if (e < -126) e = -126;
                if (e > 127) e = 127;
            }
            const float down = ldexpf(1.0f, -e);
            uint32_t term[3] = {0, 0, 0};
            int sum[3] = {0, 0, 0}, sx = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int X = bad ? 0 : (int)rintf(v[j] * down);  // |X| <= 2^22
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
            uint8_t *r = rec + ((size_t)b * TOK + tok) * REC;
#pragma unroll
            for (int k = 0; k < 3; k++)
                if (store) *(uint32_t *)(r + t * kStep8 + (g * 3 + k) * 16 + 4 * q) = term[k];
            if constexpr (TYPE == kQ8_0) {
                // signed codes, no offset: nothing besides the A fragments
            } else if (TYPE == kQ6_K) {
                // group (t, g) = the four adjacent lanes q = 0..3
#pragma unroll
                for (int k = 0; k < 3; k++) {
                    sum[k] += __shfl_xor(sum[k], 1, 64);
                    sum[k] += __shfl_xor(sum[k], 2, 64);
                }
                if (store && q == 0) *(i32x4 *)(r + 4 * kStep8 + (t * 4 + g) * 16) = i32x4{-32 * sum[0], -32 * sum[1], -32 * sum[2], 0};
            } else {
                // sub-block 2g + (t >> 1) = lanes (t, g, q) and (t ^ 1, g, q)
                sx += __shfl_xor(sx, 1, 64);
                sx += __shfl_xor(sx, 2, 64);
                sx += __shfl_xor(sx, 16, 64);
                if (store && q == 0 && (t & 1u) == 0) *(float *)(r + 4 * kStep8 + (2 * g + (t >> 1)) * 4) = (float)sx;
            }
            if (store && lane == 0) *(float *)(r + REC - 16) = bad ? __builtin_nanf("") : ldexpf(1.0f, e);
        };
        // The preloaded blocks are computed whether or not they exist, so no
        // branch separates their loads from this use (the compiler would
        // otherwise move the loads into the branch, behind the weights).
#pragma unroll
        for (int i = 0; i < XP; i++) {
            const uint32_t b = wave + (uint32_t)i * WAVES;
            record(b < blocks ? b : 0u, pre.v[tok][i], b < blocks);
        }
        for (uint32_t b = wave + XP * WAVES; b < blocks; b += WAVES) {
            const float *xb = x + (ptrdiff_t)tok * x_stride + (size_t)b * 256 + column8<TYPE>(t, g, 4 * q);
            record(b, floatx4{xb[0], xb[1], xb[2], xb[3]}, true);
        }
        if (NORM) {
            ss = wave_sum(ss);
            if (lane == 0) red_ss[tok * WAVES + wave] = ss;
        }
    }
}

}  // namespace

namespace {

// Raw bytes of one block of one row as a lane holds them.
template <uint32_t TYPE> struct Raw8;
template <> struct Raw8<kQ4_K> {
    u32x4 hdr, q0, q1;  // d|dmin|scales; qs bytes [32g, 32g+16) and [32g+16, 32g+32)
};
template <> struct Raw8<kQ8_0> {
    // bytes [68g, 68g + 68) of the super-block: blocks 2g (d, 32 codes from
    // byte 2) and 2g + 1 (d at 34, codes from 36, dword-aligned)
    u32x4 w0, w1;  // dwords 0..7
    uint32_t w8;   // dword 8: last two codes of block 2g, d of block 2g + 1
    u32x4 c2, c3;  // dwords 9..16: codes of block 2g + 1
};
template <> struct Raw8<kQ6_K> {
    u32x4 a1, a2, a3, a4;      // aligned dwords under ql[64h+16c], ql[64h+32+16c], qh[32h+16c], scales
    uint32_t e1, e2, e3, e4;   // the dword after each (e4 also holds d)
    uint32_t s;                // block start mod 4 (0 or 2)
};

// Staging of G consecutive blocks of a 16-row tile in LDS.  Row r of the
// tile occupies `chunks` 16-byte chunks loaded from the dword-aligned address
// at or below its first block (Q4_K rows start 16-aligned: 9 chunks per
// block; a Q6_K run of 210 G bytes starts 0 or 2 bytes into its first dword).
// Consecutive lanes load consecutive chunks of a row, so each quad of lanes
// reads one contiguous 64-byte span and each fetch of a row requests whole
// runs of cache lines; the lanes then read their own pieces of their own row
// from LDS.
template <uint32_t TYPE, uint32_t G> struct Stage8 {
    static constexpr uint32_t chunks = TYPE == kQ4_K ? 9 * G : TYPE == kQ8_0 ? 17 * G : (210 * G + 2 + 15) / 16;
    static constexpr uint32_t items = 16 * chunks;        // chunks of one tile
    static constexpr uint32_t loads = (items + 63) / 64;  // 16-byte loads per lane
    static constexpr uint32_t bytes = items * 16;         // one wave's staging area
};

typedef uint32_t v4u __attribute__((ext_vector_type(4)));  // 16-byte aligned (LDS)

__device__ __forceinline__ u32x4 as_u32x4(v4u v) { return __builtin_bit_cast(u32x4, v); }

// Lane (n, g)'s pieces of one block of row n from a staging area of CH
// chunks per row; `off` is the block's byte offset inside the row's run.
template <uint32_t CH>
__device__ __forceinline__ void take8(const v4u *stage, uint32_t n, uint32_t g, uint32_t off, Raw8<kQ4_K> &raw) {
    const v4u *sr = stage + n * CH + off / 16;  // Q4_K blocks stay 16-aligned
    raw.hdr = as_u32x4(sr[0]);
    raw.q0 = as_u32x4(sr[1 + 2 * g]);
    raw.q1 = as_u32x4(sr[2 + 2 * g]);
}

template <uint32_t CH>
__device__ __forceinline__ void take8(const v4u *stage, uint32_t n, uint32_t g, uint32_t off, Raw8<kQ8_0> &raw) {
    const uint32_t *sw = (const uint32_t *)(stage + n * CH) + off / 4 + 17 * g;  // super-blocks stay 16-aligned
    raw.w0 = u32x4{sw[0], sw[1], sw[2], sw[3]};
    raw.w1 = u32x4{sw[4], sw[5], sw[6], sw[7]};
    raw.w8 = sw[8];
    raw.c2 = u32x4{sw[9], sw[10], sw[11], sw[12]};
    raw.c3 = u32x4{sw[13], sw[14], sw[15], sw[16]};
}

template <uint32_t CH>
__device__ __forceinline__ void take8(const v4u *stage, uint32_t n, uint32_t g, uint32_t off, Raw8<kQ6_K> &raw) {
    // dwords of row n from the one holding the block's first byte
    const uint32_t *sw = (const uint32_t *)(stage + n * CH) + (off >> 2);
    const uint32_t h = g >> 1, c = g & 1u;
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
        const float bs = ((const float *)lds)[(rec + tok * REC + REC - 16) / 4];  // block scale 2^e
        const float part = __builtin_fmaf(sc[1], combine8(c_hi), sc[0] * combine8(c_lo));
        const float mins = __builtin_fmaf(mn[1], sums[1], mn[0] * sums[0]);
        acc[tok] = __builtin_fmaf(d * bs, part, acc[tok]);
        acc[tok] = __builtin_fmaf(-dmin * bs, mins, acc[tok]);
    }
}

// Q8_0 (src/cpu.rs:576-583, value = d * q): the codes of block 2g start two
// bytes into dword 0, so steps 0 and 1 take dwords shifted by two bytes;
// block 2g + 1's codes are dword-aligned.
template <int TOK>
__device__ __forceinline__ void block_dot8(const Raw8<kQ8_0> &raw, const i32x4 *lds, uint32_t a_off,
                                           uint32_t a_stride, uint32_t rec, uint32_t g, float (&acc)[TOK]) {
    constexpr uint32_t REC = Rec8<kQ8_0>::bytes;
    const uint32_t w[9] = {raw.w0[0], raw.w0[1], raw.w0[2], raw.w0[3], raw.w1[0],
                           raw.w1[1], raw.w1[2], raw.w1[3], raw.w8};
    i32x4 b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        b[0][i] = (int)funnel(w[i], w[i + 1], 2);
        b[1][i] = (int)funnel(w[i + 4], w[i + 5], 2);
    }
    b[2] = __builtin_bit_cast(i32x4, raw.c2);
    b[3] = __builtin_bit_cast(i32x4, raw.c3);
    const float d0 = f16_lo(raw.w0[0]), d1 = f16_lo(raw.w8 >> 16);
    const i32x4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int tok = 0; tok < TOK; tok++) {
        const uint32_t a = (a_off + tok * a_stride) / 16;
        const float p0 = combine8(mfma8(lds[a], b[0], zero)) + combine8(mfma8(lds[a + kStep8 / 16], b[1], zero));
        const float p1 =
            combine8(mfma8(lds[a + 2 * kStep8 / 16], b[2], zero)) + combine8(mfma8(lds[a + 3 * kStep8 / 16], b[3], zero));
        const float bs = ((const float *)lds)[(rec + tok * REC + REC - 16) / 4];  // block scale 2^e
        acc[tok] = __builtin_fmaf(bs, __builtin_fmaf(d1, p1, d0 * p0), acc[tok]);
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
        const float bs = ((const float *)lds)[(rec + tok * REC + REC - 16) / 4];  // block scale 2^e
        acc[tok] = __builtin_fmaf(d * bs, part, acc[tok]);
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Main kernel.  W waves per workgroup (a multiple of S).
//  * S == 1 (tall matrices): persistent.  Workgroup b owns an even share
//    [t0, t1) of the 16-row tiles; each wave takes the next tile from an LDS
//    counter when it starts the last block group of its current one, so the
//    first group of the next tile is in flight across the switch.
//  * S > 1 (short matrices): S waves split the block groups (G consecutive
//    blocks) of one tile and reduce through LDS; a workgroup covers WAVES / S
//    tiles once.
// Dynamic LDS: activation records | zeroed region | per-wave staging.
// MODE 0: y = W x.  MODE 1 (one token): also one ArgmaxPartial per
// workgroup in partials[blockIdx.x].  MODE 2: W (gate) and W2 (up) of the same
// shape on RMSNorm(x) (unit weight, when `normalize`), y = silu(gate) * up
// with the stable sigmoid, or with `glm` the routed-expert form
// gate / (1 + exp(-gate)) * up.
// Token t reads x + t * x_stride and writes y + t * y_stride.
// Register budget: 4 waves per SIMD (G <= 2) or 2 (G = 4), about what the
// workgroup's LDS allows on a C2-sized row; a tighter budget makes the
// compiler wait for each prefetch right after issuing it.
// ---------------------------------------------------------------------------
template <uint32_t TYPE, int S, int MODE, int TOK, uint32_t G, uint32_t W, bool PC = false, bool PUB = false>
__device__ __forceinline__ void qmv8_body(const uint8_t *__restrict__ w, const uint8_t *__restrict__ w2,
                                          uint32_t rows, uint32_t columns, uint32_t row_bytes,
                                          uint32_t total_bytes, const float *__restrict__ x, int x_stride,
                                          int normalize, float epsilon, int glm, float *__restrict__ y,
                                          int y_stride, ArgmaxPartial *__restrict__ partials,
                                          const ArgmaxFinish finish) {
    constexpr uint32_t WAVES = W;
    static_assert(W % S == 0, "a workgroup holds whole tiles");
    static_assert(!PC || (S == (int)W && S > 1), "a cooperative workgroup splits each tile over all its waves");
    constexpr int NM = MODE == 2 ? 2 : 1;  // weight matrices streamed
    // Activation blocks of each wave loaded ahead of the weights: what a
    // wave's share of a 4096-column row is (16 blocks over W waves), so that
    // no record is computed for a block past the end; wider rows load the
    // rest after the weights.  None on the persistent one-tile-per-wave
    // schedule of single matrices (S = 1, tall matrices), which requests its
    // first weights behind a branch and builds the records after them:
    // measured on MI355X at C2 (Q6_K 151936 x 4096 with the argmax,
    // interleaved runs on one box) 94.0-94.2 us against 97.3-97.8 us with
    // the preloading, branch-free prologue the split schedules use, which
    // also read 4.7% more bytes per launch.
    constexpr int XP = (S == 1 && !PC && MODE != 2) ? 0 : (TOK >= 2 ? 1 : (W >= 16 ? 1 : 2));
    constexpr uint32_t REC = Rec8<TYPE>::bytes;
    constexpr uint32_t BB = kBlock8<TYPE>;
    using ST = Stage8<TYPE, G>;
    constexpr uint32_t CH = ST::chunks, NL = ST::loads, ITEMS = ST::items;
    extern __shared__ i32x4 lds8[];
    __shared__ float red[S > 1 ? WAVES * 64 * TOK * NM : 1];
    __shared__ float red_ss[TOK * WAVES];
    __shared__ uint32_t next_tile;
    __shared__ unsigned long long wg_key[WAVES];
    __shared__ uint32_t wg_bad[WAVES];

    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t kpart = wave % S;
    const uint32_t blocks = columns / 256, groups = (blocks + G - 1) / G;
    const uint32_t tiles = (rows + 15) / 16;
    const uint32_t rec_bytes = blocks * TOK * REC;
    v4u *stage = (v4u *)((uint8_t *)lds8 + rec_bytes + kZero8) + wave * ITEMS * NM;
    v4u *stage2 = stage + (NM - 1) * ITEMS;

    // Whole dwords: the last dword of the matrix may extend up to 3 bytes past
    // its end (inside the allocation's granularity); loads beyond it read 0.
    const uint32_t records = (total_bytes + 3u) & ~3u;
    const uint32_t nowhere = records + 256;  // every load from here reads 0
    const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(w, records);
    const __amdgpu_buffer_rsrc_t rsrc2 = make_rsrc(MODE == 2 ? w2 : w, records);

    // Tile schedule.
    uint32_t tile, t_end;
    if constexpr (S == 1) {
        const uint32_t t0 = (uint32_t)((uint64_t)blockIdx.x * tiles / gridDim.x);
        t_end = (uint32_t)((uint64_t)(blockIdx.x + 1) * tiles / gridDim.x);
        tile = t0 + wave;
        if (threadIdx.x == 0) next_tile = t0 + WAVES;
    } else if constexpr (PC) {
        // persistent: the workgroup takes tiles blockIdx.x, + gridDim.x, ...
        tile = blockIdx.x;
        t_end = tiles;
    } else {
        tile = blockIdx.x * (WAVES / S) + wave / S;
        t_end = tile + 1 < tiles ? tile + 1 : tiles;
    }

    // Staging chunk j*64 + lane: row r, chunk c of the tile.
    uint32_t src_row[NL], src_chunk[NL];
    uint32_t next_row_base = nowhere;
    auto setup = [&](uint32_t tl, bool live) {
#pragma unroll
        for (uint32_t j = 0; j < NL; j++) {
            const uint32_t item = j * 64 + lane, r = item / CH, c = item % CH;
            const uint32_t rr = tl * 16 + r;
            src_row[j] = (live && item < ITEMS && rr < rows) ? rr * row_bytes : nowhere;
            src_chunk[j] = 16 * c;
        }
        const uint32_t rw = tl * 16 + n;
        next_row_base = (live && rw < rows) ? rw * row_bytes : nowhere;
    };
    v4u st[NL], st2[MODE == 2 ? NL : 1];
    // Consecutive fetches of a row share the 128-byte line at their
    // boundary, and a wave's next fetch of the row comes microseconds later:
    // the rest of a fetch is loaded non-temporal (evicted first from the
    // L2), the chunks in the line where the row's next fetch starts are
    // loaded normally, so that line is still there for it (C2: 1.11 ->
    // 1.06 times the algorithmic bytes, 95 -> 92 us).  Lines are 128-byte
    // aligned in the address space, hence the base's low bits (the gate/up
    // pairs' matrices share them: separate allocations, or the up rows at a
    // multiple of 128 bytes; otherwise only the cache hint is off).
    const uint32_t lo = (uint32_t)(uintptr_t)w & 127u;
    constexpr bool kHint = S == 1 && !PC && TOK == 1;
    auto fetch = [&](uint32_t grp, bool live) {
#pragma unroll
        for (uint32_t j = 0; j < NL; j++) {
            const uint32_t cur = (src_row[j] + grp * G * BB) & ~3u;
            const uint32_t off = (!live || src_row[j] == nowhere) ? nowhere : cur + src_chunk[j];
            // the line where the next fetch starts (within 3 bytes: a hint);
            // only where one wave reads a tile's groups one after another
            // (the persistent one-tile-per-wave schedule, one token): where
            // neighbouring waves read adjacent groups at the same time, the
            // hint made C1, C3 and the Q8_0 head 10-14% slower
            const bool keep = !kHint || off + 16 > ((lo + cur + G * BB) & ~127u) - lo;
            if (keep) {
                st[j] = __builtin_bit_cast(v4u, rsrc_load16(rsrc, off));
                if constexpr (MODE == 2) st2[j] = __builtin_bit_cast(v4u, rsrc_load16(rsrc2, off));
            } else {
                st[j] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, kNonTemporal));
                if constexpr (MODE == 2)
                    st2[j] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rsrc2, off, 0, kNonTemporal));
            }
        }
    };

    // The wave's first activation values, then its first weights, are
    // requested before the records are built.
    XPre8<TOK, XP> xpre;
    preload_x8<TYPE, TOK, WAVES, XP>(x, x_stride, columns, xpre);
    bool active = tile < t_end;
    if constexpr (XP == 0) {
        if (active) {
            setup(tile, true);
            if (kpart < groups) fetch(kpart, true);
        }
    } else {
        // Issued without a branch (an idle wave's loads all read past the end).
        setup(active ? tile : 0u, active);
        fetch(kpart, active && kpart < groups);
    }
    wait_x8<NL * NM>(xpre);
    uint32_t row_base = next_row_base;

    const bool norm = MODE == 2 && normalize;
    if (norm)
        build_records8<TYPE, TOK, WAVES, true, XP>(x, x_stride, columns, (uint8_t *)lds8, red_ss, xpre);
    else
        build_records8<TYPE, TOK, WAVES, false, XP>(x, x_stride, columns, (uint8_t *)lds8, red_ss, xpre);
    for (uint32_t i = threadIdx.x; i < kZero8 / 16; i += 64 * WAVES) lds8[rec_bytes / 16 + i] = i32x4{0, 0, 0, 0};
    __syncthreads();
    // Output scale per token: 1, or the RMSNorm factor (unit weight)
    // inv = (ss/n + eps).sqrt().recip() (src/cpu.rs:98-142) folded in.
    float tscale[TOK];
#pragma unroll
    for (int tok = 0; tok < TOK; tok++) {
        tscale[tok] = 1.0f;
        if (norm) {
            float q = 0.0f;
            for (uint32_t k2 = 0; k2 < WAVES; k2++) q += red_ss[tok * WAVES + k2];
            tscale[tok] = 1.0f / __builtin_sqrtf(q / (float)columns + epsilon);
        }
    }

    // A row n of the MFMA: live when it is term n % 4 (< 3) of lane group n / 4.
    const uint32_t term = n & 3u;
    const bool a_live = (n >> 2) == g && term < 3;
    const uint32_t a_base = a_live ? (g * 3 + term) * 16 : rec_bytes;
    const uint32_t a_stride = a_live ? REC : 0;

    // The chunks of a block group go to the wave's staging area; the loads of
    // the next group are in flight while this one is read back and computed.
    // A wave only reads its own staging area, and its LDS operations run in
    // order, so no barrier is needed; the wavefront-scope fences keep the
    // compiler from moving another lane's reads across these writes.
    auto put_stage = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (uint32_t j = 0; j < NL; j++)
            if (j + 1 < NL || j * 64 + lane < ITEMS) {
                stage[j * 64 + lane] = st[j];
                if constexpr (MODE == 2) stage2[j * 64 + lane] = st2[j];
            }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    };
    // acc[m][tok]: matrix m (gate, up) of token tok
    auto compute_group = [&](uint32_t grp, uint32_t rb, float (&acc)[NM][TOK]) {
        // the run of row n starts 0 or 2 bytes into its first dword (Q6_K)
        const uint32_t s0 = rb == nowhere ? 0u : ((rb + grp * G * BB) & 3u);
#pragma unroll
        for (uint32_t b = 0; b < G; b++) {
            const uint32_t blk = grp * G + b;
            if (blk >= blocks) break;
#pragma unroll
            for (int mtx = 0; mtx < NM; mtx++) {
                Raw8<TYPE> raw;
                take8<CH>(mtx == 0 ? stage : stage2, n, g, s0 + b * BB, raw);
                block_dot8<TOK>(raw, lds8, a_base + blk * TOK * a_stride, a_stride, blk * TOK * REC, g, acc[mtx]);
            }
        }
    };

    uint64_t best = 0;
    uint32_t bad = 0;
    auto finish_row = [&](float (&acc)[NM][TOK], uint32_t rb, uint32_t tl) {
        const uint32_t row = tl * 16 + n;
        if (g < (uint32_t)TOK && rb != nowhere) {
            // after the cross-group sums every lane group holds every token:
            // lane group g writes token g.  The candidates pass through an
            // empty asm as plain values, so the selection cannot become an
            // index into the arrays (which would put them in scratch).
            float ts = tscale[0], gate = acc[0][0], up = acc[NM - 1][0];
#pragma unroll
            for (int tok = 1; tok < TOK; tok++) {
                float t_ts = tscale[tok], t_gate = acc[0][tok], t_up = acc[NM - 1][tok];
                asm volatile("" : "+v"(t_ts), "+v"(t_gate), "+v"(t_up));
                if (g == (uint32_t)tok) {
                    ts = t_ts;
                    gate = t_gate;
                    up = t_up;
                }
            }
            float v = gate * ts;
            if constexpr (MODE == 2) {
                const float u = up * ts;
                if (glm) {
                    // routed-expert activation (src/glm52/expert.rs:260-267)
                    v = (v / (1.0f + expf(-v))) * u;
                } else {
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
            }
            if constexpr (PUB) {
                // published for another workgroup: performed at the memory
                // side before this wave goes on (the fence-free pattern)
                const float old = __hip_atomic_exchange(&y[(ptrdiff_t)g * y_stride + row], v, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
                asm volatile("" ::"v"(old) : "memory");
            } else {
                y[(ptrdiff_t)g * y_stride + row] = v;
            }
            if constexpr (MODE == 1) {
                bad |= !__builtin_isfinite(v);
                const uint64_t key = argmax_key(v, row);
                best = key > best ? key : best;
            }
        }
    };

    if constexpr (S == 1) {
        while (active) {
            float acc[NM][TOK];
#pragma unroll
            for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
                for (int tok = 0; tok < TOK; tok++) acc[mtx][tok] = 0.0f;
            uint32_t next = t_end;
            const uint32_t rb = row_base;
            for (uint32_t grp = 0; grp < groups; grp++) {
                put_stage();
                if (grp + 1 < groups) {
                    fetch(grp + 1, true);
                } else {
                    uint32_t claimed = 0;
                    if (lane == 0) claimed = atomicAdd(&next_tile, 1u);
                    next = __builtin_amdgcn_readfirstlane(claimed);
                    if (next < t_end) {
                        setup(next, true);
                        fetch(0, true);
                    }
                }
                compute_group(grp, rb, acc);
            }
#pragma unroll
            for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
                for (int tok = 0; tok < TOK; tok++) {
                    acc[mtx][tok] += __shfl_xor(acc[mtx][tok], 16, 64);
                    acc[mtx][tok] += __shfl_xor(acc[mtx][tok], 32, 64);
                }
            finish_row(acc, rb, tile);
            tile = next;
            row_base = next_row_base;
            active = tile < t_end;
        }
    } else if constexpr (PC) {
        // Every wave takes block groups kpart, kpart + S, ... of the
        // workgroup's current tile, so the workgroup requests the tile's 16
        // rows together (whole rows: one contiguous span of the matrix); the
        // next tile's first groups are requested before the reduction.
        // `active` is the same in every wave of the workgroup.
        while (active) {
            float acc[NM][TOK];
#pragma unroll
            for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
                for (int tok = 0; tok < TOK; tok++) acc[mtx][tok] = 0.0f;
            const uint32_t next = tile + gridDim.x;
            const uint32_t rb = row_base;
            for (uint32_t grp = kpart; grp < groups; grp += S) {
                put_stage();
                if (grp + S < groups) {
                    fetch(grp + S, true);
                } else if (next < t_end) {
                    setup(next, true);
                    fetch(kpart, true);
                }
                compute_group(grp, rb, acc);
            }
#pragma unroll
            for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
                for (int tok = 0; tok < TOK; tok++) {
                    acc[mtx][tok] += __shfl_xor(acc[mtx][tok], 16, 64);
                    acc[mtx][tok] += __shfl_xor(acc[mtx][tok], 32, 64);
                    red[((wave * 64 + lane) * TOK + tok) * NM + mtx] = acc[mtx][tok];
                }
            __syncthreads();
            if (kpart == 0) {
#pragma unroll
                for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
                    for (int tok = 0; tok < TOK; tok++) {
                        float v = 0.0f;
                        for (int p = 0; p < S; p++) v += red[(((wave + p) * 64 + lane) * TOK + tok) * NM + mtx];
                        acc[mtx][tok] = v;
                    }
                finish_row(acc, rb, tile);
            }
            __syncthreads();  // red is written again for the next tile
            tile = next;
            row_base = next_row_base;
            active = tile < t_end;
        }
    } else {
        float acc[NM][TOK];
#pragma unroll
        for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
            for (int tok = 0; tok < TOK; tok++) acc[mtx][tok] = 0.0f;
        if (active) {
            for (uint32_t grp = kpart; grp < groups; grp += S) {
                put_stage();
                if (grp + S < groups) fetch(grp + S, true);
                compute_group(grp, row_base, acc);
            }
        }
#pragma unroll
        for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
            for (int tok = 0; tok < TOK; tok++) {
                acc[mtx][tok] += __shfl_xor(acc[mtx][tok], 16, 64);
                acc[mtx][tok] += __shfl_xor(acc[mtx][tok], 32, 64);
                red[((wave * 64 + lane) * TOK + tok) * NM + mtx] = acc[mtx][tok];
            }
        __syncthreads();
        if (kpart == 0 && active) {
#pragma unroll
            for (int mtx = 0; mtx < NM; mtx++)
#pragma unroll
                for (int tok = 0; tok < TOK; tok++) {
                    float v = 0.0f;
                    for (int p = 0; p < S; p++) v += red[(((wave + p) * 64 + lane) * TOK + tok) * NM + mtx];
                    acc[mtx][tok] = v;
                }
            finish_row(acc, row_base, tile);
        }
    }

    if constexpr (MODE == 1) {
        best = wave_max_u64(best);
        bad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;
        if (lane == 0) {
            wg_key[wave] = best;
            wg_bad[wave] = bad;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t k = wg_key[0];
            uint32_t f = wg_bad[0];
            for (uint32_t i = 1; i < WAVES; i++) {
                k = wg_key[i] > k ? wg_key[i] : k;
                f |= wg_bad[i];
            }
            if (finish.ticket) {
                // Fold the candidate into the device-wide maximum (a
                // non-finite row contributes the all-ones key, above every
                // finite key), wait for the atomic to complete, then take a
                // ticket: the workgroup that draws the last one reads the
                // final maximum.  No cache-wide release fence is needed.
                const unsigned long long packed = f ? ~0ull : k;
                const unsigned long long prev = atomicMax(finish.best, packed);
                asm volatile("" ::"v"(prev) : "memory");
                if (atomicAdd(finish.ticket, 1u) == gridDim.x - 1) {
                    const uint64_t kb = __hip_atomic_load(finish.best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    const uint32_t nf = kb == ~0ull ? 1u : 0u;
                    finish.state->key = nf ? 0ull : kb;
                    finish.state->non_finite = nf;
                    finish.state->done = gridDim.x;
                    *finish.index = argmax_key_index(kb);
                    __hip_atomic_store(finish.best, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(finish.ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            } else {
                ArgmaxPartial p;
                p.key = k;
                p.non_finite = f;
                p.pad = 0;
                partials[blockIdx.x] = p;
            }
        }
    }
}

// Register budget: four waves per SIMD (128 VGPRs), or two (256) for
// four-block fetches and for the gate/up kernels that need more (Q6_K pairs,
// two-token two-block fetches); with less they spill to scratch.
template <uint32_t TYPE, int MODE, int TOK, uint32_t G, bool PC = false>
constexpr int waves_per_eu8() {
    // cooperative: the Q8_0 form gets 256 registers (one 8-wave workgroup
    // per CU); the Q4_K form fits 128 (two per CU)
    return ((PC && TYPE == kQ8_0) || G > 2 || TOK > 2 || (MODE == 2 && (TYPE == kQ6_K || (TOK == 2 && G == 2)))) ? 2
                                                                                                            : 4;
}

template <uint32_t TYPE, int S, int MODE, int TOK, uint32_t G, uint32_t W, bool PC = false>
__global__ void __launch_bounds__(64 * W)
    __attribute__((amdgpu_waves_per_eu(waves_per_eu8<TYPE, MODE, TOK, G, PC>()))) qmv8_kernel(
    const uint8_t *__restrict__ w, const uint8_t *__restrict__ w2, uint32_t rows, uint32_t columns,
    uint32_t row_bytes, uint32_t total_bytes, const float *__restrict__ x, int normalize, float epsilon,
    float *__restrict__ y, ArgmaxPartial *__restrict__ partials, ArgmaxFinish finish) {
    qmv8_body<TYPE, S, MODE, TOK, G, W, PC>(w, w2, rows, columns, row_bytes, total_bytes, x, (int)columns,
                                            normalize, epsilon, 0, y, (int)rows, partials, finish);
}

// Grouped launch over the routed-expert jobs of a MoE layer: job
// blockIdx.y applies the matrix at jobs.job[j].w (and, in MODE 2, the up
// matrix w2_offset bytes further) to TOK tokens at x + x_off, x_stride apart,
// writing y + y_off, y_stride apart.  Every job has the same shape.
struct Job8 {
    uint64_t w;
    uint32_t x_off, y_off;
    int32_t x_stride, y_stride;
};
constexpr uint32_t kMaxJobs8 = kMaxGroupedJobs;
struct JobTable8 {
    Job8 job[kMaxJobs8];
};

// The ordered combine of each token's routed experts fused into their down
// launch: y[r] = fma(out_k-1[r], p[k-1], ... fma(out_0[r], p[0], 0)) in
// selection order, as the separate combine computes it
// (src/gemma4/cpu.rs:608-611).  Job j is selection j % k of token j / k.
// Every workgroup publishes its expert's rows (PUB), then takes the ticket
// of its token's row tiles; the one that draws the last (of k) adds the k
// rows of those tiles and resets the ticket.
struct Combine8 {
    uint32_t *tickets;  // one per (token, blockIdx.x), zero between launches
    const float *p;     // k probabilities per token
    float *y;           // token t's output at y + t * y_stride
    uint32_t k, y_stride;
};

template <uint32_t TYPE, int S, int MODE, int TOK, uint32_t G, bool PUB = false>
__global__ void __launch_bounds__(64 * (S > 8 ? S : 8))
    __attribute__((amdgpu_waves_per_eu(waves_per_eu8<TYPE, MODE, TOK, G>()))) qmv8_grouped_kernel(JobTable8 jobs, uint32_t rows, uint32_t columns, uint32_t row_bytes,
                        uint32_t total_bytes, uint64_t w2_offset, const float *__restrict__ x,
                        float *__restrict__ y, int glm, const uint64_t *__restrict__ dev_w,
                        const uint32_t *__restrict__ go, uint32_t go_count, Combine8 cb) {
    // Jobs whose matrices a kernel earlier on the stream looked up: their
    // addresses come from dev_w, and the launch does nothing unless each of
    // the go_count tokens' go words is 1.
    if (go)
        for (uint32_t t = 0; t < go_count; t++)
            if (go[t] == 0) return;
    const Job8 j = jobs.job[blockIdx.y];
    const uint8_t *w = (const uint8_t *)(dev_w ? dev_w[blockIdx.y] : j.w);
    constexpr uint32_t WAVES = S > 8 ? S : 8;
    qmv8_body<TYPE, S, MODE, TOK, G, WAVES, false, PUB>(w, w + w2_offset, rows, columns, row_bytes, total_bytes,
                                                        x + j.x_off, j.x_stride, 0, 0.0f, glm, y + j.y_off,
                                                        j.y_stride, nullptr,
                                                        ArgmaxFinish{nullptr, nullptr, nullptr, nullptr});
    if constexpr (PUB) {
        static_assert(MODE == 0 && TOK == 1 && S > 1, "the combine follows one-token split launches");
        __shared__ uint32_t s_last;
        const uint32_t token = blockIdx.y / cb.k;
        uint32_t *ticket = &cb.tickets[(size_t)token * gridDim.x + blockIdx.x];
        __syncthreads();  // every wave's rows are published
        if (threadIdx.x == 0) s_last = atomicAdd(ticket, 1u) == cb.k - 1 ? 1u : 0u;
        __syncthreads();
        if (!s_last) return;
        // the rows of this workgroup's tiles (y_off of job p is p * rows)
        const uint32_t r0 = blockIdx.x * (WAVES / S) * 16, r1 = min(r0 + (WAVES / S) * 16, rows);
        const uint32_t j0 = token * cb.k;
        for (uint32_t r = r0 + threadIdx.x; r < r1; r += blockDim.x) {
            float acc = 0.0f;
            for (uint32_t p = j0; p < j0 + cb.k; p++)
                acc = __builtin_fmaf(__hip_atomic_load(&y[(size_t)p * rows + r], __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT),
                                     cb.p[p], acc);
            cb.y[(size_t)token * cb.y_stride + r] = acc;
        }
        if (threadIdx.x == 0) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

namespace {

constexpr size_t kMaxLds8 = 160 * 1024;  // gfx950 LDS per workgroup

size_t stage_bytes8(uint32_t type, uint32_t g) {
    if (type == kQ4_K) return g == 1 ? Stage8<kQ4_K, 1>::bytes : g == 2 ? Stage8<kQ4_K, 2>::bytes : Stage8<kQ4_K, 4>::bytes;
    if (type == kQ8_0) return g == 1 ? Stage8<kQ8_0, 1>::bytes : g == 2 ? Stage8<kQ8_0, 2>::bytes : Stage8<kQ8_0, 4>::bytes;
    return g == 1 ? Stage8<kQ6_K, 1>::bytes : g == 2 ? Stage8<kQ6_K, 2>::bytes : Stage8<kQ6_K, 4>::bytes;
}

// Dynamic LDS of one workgroup: records, zeroed region, staging per wave
// (one area per streamed matrix).
size_t lds8_bytes(uint32_t type, uint32_t blocks, uint32_t batch, uint32_t waves, uint32_t g, uint32_t mats) {
    const size_t rec = type == kQ4_K ? Rec8<kQ4_K>::bytes : type == kQ8_0 ? Rec8<kQ8_0>::bytes : Rec8<kQ6_K>::bytes;
    return (size_t)blocks * batch * rec + kZero8 + (size_t)waves * mats * stage_bytes8(type, g);
}

struct Plan8 {
    uint32_t s = 0, g = 1;
    bool pc = false;  // persistent workgroups whose S = 8 waves share each tile
};

// Very tall Q4_K and Q8_0 matrices (output heads): persistent 8-wave
// workgroups that read each 16-row tile together (every wave one group of
// the tile's rows, so the workgroup requests one contiguous span), rather
// than waves that each stream their own tile.  Measured on MI355X at
// 151936 x 4096, batch 1: Q4_K 61.5 against 65.5 us (with the argmax 63.2
// against 69.0), Q8_0 111.2 against 116.5 us.  Below about 8192 tiles it
// loses (Q4_K 65536 x 2048: 17.1 against 16.3 us), and Q6_K gains nothing
// (a 16-wave form: 95.9 against 95.6 us at C2, slower below), so those keep
// per-wave tiles.
constexpr bool kCooperativeTall = true;
constexpr uint32_t kCooperativeTiles = 8192;

// Waves per workgroup of a plan with split S: eight up to S = 8 (several
// tiles per workgroup below that), S above.
constexpr uint32_t waves8(uint32_t s) { return s <= 8 ? 8u : s; }

bool fits8(uint32_t type, uint32_t blocks, uint32_t batch, uint32_t mats, uint32_t s, uint32_t g) {
    const uint32_t waves = waves8(s);
    // static: split-K scratch, token maxima, argmax candidates, counters
    const size_t stat = (s > 1 ? (size_t)waves * 64 * batch * mats * sizeof(float) : 4) + 768;
    return lds8_bytes(type, blocks, batch, waves, g, mats) + stat <= kMaxLds8;
}

// Blocks per fetch (G) and split of each tile's block groups over S waves:
// enough waves to keep every SIMD busy, at least one group per wave, and the
// workgroup's LDS (dynamic plus split-K scratch) within the 160 KiB of a
// gfx950 workgroup.  Two blocks per fetch on tall matrices halve the cache
// lines requested twice (a block's last line is the next block's first);
// short ones need the parallelism of single-block groups more.  Measured on
// MI355X (kernel trace medians): a 4096 x 4096 Q4_K matrix runs 5.7 us with
// 16 waves of one block per tile against 6.2 us with one 4-wave workgroup of
// four-block fetches per tile, and 4096 x 2048 runs 4.2 us with 8 waves
// against 5.2 us with four of two-block fetches.
// s == 0: no plan.
Plan8 plan8(uint32_t type, uint32_t rows, uint32_t columns, uint32_t batch, uint32_t mats) {
    Plan8 p;
    const uint32_t tiles = (rows + 15) / 16, blocks = columns / 256;
    p.g = tiles >= 2048 ? 2u : 1u;
    while (p.g > 1 && blocks < 2 * p.g) p.g /= 2;
    const uint32_t groups = (blocks + p.g - 1) / p.g;
    if (kCooperativeTall && type != kQ6_K && tiles >= kCooperativeTiles && p.g == 2 && groups >= 8 && mats == 1 &&
        batch <= 2 && fits8(type, blocks, batch, mats, 8, p.g)) {
        p.s = 8;
        p.pc = true;
        return p;
    }
    const uint32_t s_max = mats == 2 ? 8u : kMaxWaves8;  // gate/up: see run8_s
    // A gate/up wave streams both matrices, so half the wave-tiles carry the
    // same bytes in flight: C3's 12288 x 4096 pair ran its layer in 25.3 us
    // with S = 4 against 26.6 us with S = 8.
    uint32_t s = 1;
    while (s < s_max && (size_t)tiles * s * mats < 4096 && groups >= 2 * s) s *= 2;
    for (; s >= 1; s /= 2)
        if (fits8(type, blocks, batch, mats, s, p.g)) {
            p.s = s;
            return p;
        }
    p.s = 0;
    return p;
}

// Launch arguments shared by every instantiation.
struct Args8 {
    uint32_t rows, columns;
    const void *w, *w2;
    const float *x;
    int normalize;
    float epsilon;
    float *y;
    ArgmaxPartial *partials;
    uint32_t *count;
    ArgmaxFinish finish;
};

template <uint32_t TYPE, int S, int MODE, int TOK, uint32_t G, bool PC = false>
hipError_t run8(dmhip_ctx *ctx, const Args8 &a) {
    constexpr uint32_t WAVES = waves8(S);
    const uint32_t rows = a.rows, columns = a.columns;
    const uint32_t tiles = (rows + 15) / 16;
    const uint32_t blocks = columns / 256;
    const uint32_t row_bytes = blocks * kBlock8<TYPE>;
    const size_t lds = lds8_bytes(TYPE, blocks, TOK, WAVES, G, MODE == 2 ? 2u : 1u);
    uint32_t grid;
    if (S == 1 || PC) {
        // persistent: as many workgroups as fit on the device at once (the
        // register budget allows waves_per_eu8 waves per SIMD)
        const uint32_t by_regs = 4 * waves_per_eu8<TYPE, MODE, TOK, G, PC>() / WAVES;
        uint32_t by_lds = (uint32_t)(kMaxLds8 / (lds + 4096));
        uint32_t per_cu = by_regs < by_lds ? by_regs : by_lds;
        if (per_cu == 0) per_cu = 1;
        const uint32_t cus = ctx->compute_units > 0 ? (uint32_t)ctx->compute_units : 256u;
        const uint32_t need = PC ? tiles : (tiles + WAVES - 1) / WAVES;
        grid = cus * per_cu < need ? cus * per_cu : need;
    } else {
        const uint32_t per = WAVES / S;
        grid = (tiles + per - 1) / per;
    }
    if (a.count) *a.count = grid;
    auto kernel = qmv8_kernel<TYPE, S, MODE, TOK, G, WAVES, PC>;
    if (lds > 64 * 1024) {
        static LdsLimit limit;
        hipError_t e = limit.ensure((const void *)kernel, lds);
        if (e != hipSuccess) return e;
    }
    return launch_kernel(ctx, kernel, dim3(grid), dim3(64 * WAVES), lds, (const uint8_t *)a.w,
                         (const uint8_t *)a.w2, rows, columns, row_bytes, row_bytes * rows, a.x, a.normalize,
                         a.epsilon, a.y, a.partials, a.finish);
}

template <uint32_t TYPE, int MODE, int TOK, uint32_t G>
hipError_t run8_s(dmhip_ctx *ctx, uint32_t s, const Args8 &a) {
    switch (s) {
    case 1: return run8<TYPE, 1, MODE, TOK, G>(ctx, a);
    case 2: return run8<TYPE, 2, MODE, TOK, G>(ctx, a);
    case 4: return run8<TYPE, 4, MODE, TOK, G>(ctx, a);
    case 8: return run8<TYPE, 8, MODE, TOK, G>(ctx, a);
    default:
        // gate/up plans and four-block fetches stop at 8 waves (plan8): their
        // registers do not fit the 16-wave workgroup's budget
        if constexpr (MODE == 2 || G == 4) return hipErrorInvalidValue;
        else return run8<TYPE, 16, MODE, TOK, G>(ctx, a);
    }
}

template <uint32_t TYPE, int MODE, int TOK>
hipError_t run8_g(dmhip_ctx *ctx, const Plan8 &p, const Args8 &a) {
    if constexpr (TYPE != kQ6_K && MODE != 2 && TOK <= 2) {
        if (p.pc) return p.g == 2 && p.s == 8 ? run8<TYPE, 8, MODE, TOK, 2, true>(ctx, a) : hipErrorInvalidValue;
    } else {
        if (p.pc) return hipErrorInvalidValue;  // plan8 plans no cooperative Q6_K or gate/up launch
    }
    if constexpr (MODE != 2 && TOK <= 2) {
        if (p.g == 4) return run8_s<TYPE, MODE, TOK, 4>(ctx, p.s, a);
    } else {
        if (p.g == 4) return hipErrorInvalidValue;  // not instantiated: plan8 picks G <= 2
    }
    if (p.g == 2) return run8_s<TYPE, MODE, TOK, 2>(ctx, p.s, a);
    return run8_s<TYPE, MODE, TOK, 1>(ctx, p.s, a);
}

// Grouped jobs: blocks per fetch (G = 2 for rows of 8 or more blocks, whose
// runs of 2 blocks stream about 60% faster than single blocks; G = 1
// otherwise), and a split of each tile's
// block groups that gives the whole launch about 4096 wave-tiles with at
// least one group per wave.
Plan8 plan8_grouped(uint32_t type, uint32_t rows, uint32_t columns, uint32_t batch, uint32_t mats,
                    uint32_t jobs) {
    Plan8 p;
    const uint32_t tiles = (rows + 15) / 16, blocks = columns / 256;
    // Small launches (C4's routed experts: 384 and 1024 job tiles) measured
    // 4-5% faster with single-block groups over 4 waves per tile.
    const bool small = (size_t)tiles * jobs < 1536 && blocks >= 2;
    uint32_t g = blocks >= 8 && !small ? 2u : 1u;
    if (blocks < 2) g = 1;
    for (; g >= 1; g /= 2) {
        const uint32_t groups = (blocks + g - 1) / g;
        uint32_t s = 1;
        if (small) {
            s = 4;
        } else {
            while (s < 8 && (size_t)tiles * jobs * s < 4096 && groups >= 2 * s) s *= 2;
        }
        for (; s >= 1; s /= 2) {
            const size_t stat = (s > 1 ? (size_t)8 * 64 * batch * mats * sizeof(float) : 4) + 768;
            if (lds8_bytes(type, blocks, batch, 8, g, mats) + stat <= kMaxLds8) {
                p.s = s;
                p.g = g;
                return p;
            }
        }
    }
    p.s = 0;
    return p;
}

struct DeviceJobs {
    const uint64_t *w;
    const uint32_t *go;
    uint32_t go_count;  // go words (tokens) a launch checks
    Combine8 cb;        // cb.tickets set: the fused combine (one-token down jobs)
};

template <uint32_t TYPE, int S, int MODE, int TOK, uint32_t G>
hipError_t run8_grouped(dmhip_ctx *ctx, uint32_t rows, uint32_t columns, uint64_t up_offset,
                        const JobTable8 &table, uint32_t count, const float *x, float *y, DeviceJobs dj) {
    constexpr uint32_t WAVES = 8;
    const uint32_t tiles = (rows + 15) / 16;
    const uint32_t blocks = columns / 256;
    const uint32_t row_bytes = blocks * kBlock8<TYPE>;
    const size_t lds = lds8_bytes(TYPE, blocks, TOK, WAVES, G, MODE == 2 ? 2u : 1u);
    // S == 1: one tile per wave; S > 1: WAVES / S tiles per workgroup.
    const uint32_t per = S == 1 ? WAVES : WAVES / S;
    const uint32_t grid = (tiles + per - 1) / per;
    auto kernel = qmv8_grouped_kernel<TYPE, S, MODE, TOK, G>;
    if constexpr (MODE == 0 && TOK == 1 && S > 1) {
        if (dj.cb.tickets) kernel = qmv8_grouped_kernel<TYPE, S, MODE, TOK, G, true>;
    }
    if (lds > 64 * 1024) {
        static LdsLimit limit, limit_pub;
        hipError_t e = (dj.cb.tickets ? limit_pub : limit).ensure((const void *)kernel, lds);
        if (e != hipSuccess) return e;
    }
    return launch_kernel(ctx, kernel, dim3(grid, count), dim3(64 * WAVES), lds, table, rows, columns, row_bytes,
                         row_bytes * rows, up_offset, x, y, MODE == 2 ? 1 : 0, dj.w, dj.go, dj.go_count, dj.cb);
}

template <uint32_t TYPE, int MODE, int TOK, uint32_t G>
hipError_t run8_grouped_sg(dmhip_ctx *ctx, uint32_t s, uint32_t rows, uint32_t columns, uint64_t up_offset,
                           const JobTable8 &table, uint32_t count, const float *x, float *y, DeviceJobs dj) {
    switch (s) {
    case 1: return run8_grouped<TYPE, 1, MODE, TOK, G>(ctx, rows, columns, up_offset, table, count, x, y, dj);
    case 2: return run8_grouped<TYPE, 2, MODE, TOK, G>(ctx, rows, columns, up_offset, table, count, x, y, dj);
    case 4: return run8_grouped<TYPE, 4, MODE, TOK, G>(ctx, rows, columns, up_offset, table, count, x, y, dj);
    default: return run8_grouped<TYPE, 8, MODE, TOK, G>(ctx, rows, columns, up_offset, table, count, x, y, dj);
    }
}

template <uint32_t TYPE, int MODE, int TOK>
hipError_t run8_grouped_s(dmhip_ctx *ctx, const Plan8 &p, uint32_t rows, uint32_t columns, uint64_t up_offset,
                          const JobTable8 &table, uint32_t count, const float *x, float *y, DeviceJobs dj) {
    if (p.g == 2)
        return run8_grouped_sg<TYPE, MODE, TOK, 2>(ctx, p.s, rows, columns, up_offset, table, count, x, y, dj);
    return run8_grouped_sg<TYPE, MODE, TOK, 1>(ctx, p.s, rows, columns, up_offset, table, count, x, y, dj);
}

template <uint32_t TYPE>
hipError_t launch8(dmhip_ctx *ctx, uint32_t batch, int mode, const Args8 &a) {
    const Plan8 p = plan8(TYPE, a.rows, a.columns, batch, mode == 2 ? 2u : 1u);
    if (p.s == 0) return hipErrorInvalidValue;
    if (mode == 1) return run8_g<TYPE, 1, 1>(ctx, p, a);
    if (mode == 2) {
        if constexpr (TYPE == kQ8_0) {
            return hipErrorInvalidValue;  // gate/up pairs are Q4_K or Q6_K
        } else {
            // 1-2 tokens (qmv8_gate_up_supported)
            if (batch > 2) return hipErrorInvalidValue;
            return batch == 1 ? run8_g<TYPE, 2, 1>(ctx, p, a) : run8_g<TYPE, 2, 2>(ctx, p, a);
        }
    }
    switch (batch) {
    case 1: return run8_g<TYPE, 0, 1>(ctx, p, a);
    case 2: return run8_g<TYPE, 0, 2>(ctx, p, a);
    case 3: return run8_g<TYPE, 0, 3>(ctx, p, a);
    default: return run8_g<TYPE, 0, 4>(ctx, p, a);
    }
}

}  // namespace

bool qmv8_supported(uint32_t type, size_t rows, size_t columns, size_t batch) {
    if (type != kQ4_K && type != kQ6_K && type != kQ8_0) return false;
    if (batch < 1 || batch > kMaxTokens8 || columns % 256 || columns == 0) return false;
    // 3-4 tokens of Q4_K / Q6_K: the int8 kernel against the fp16 one and its
    // preparation launch, measured per launch on MI355X: 4096 x 4096 Q4_K
    // 7.4 / 8.5 us against 11.0 us, Q6_K 9.4 / 10.8 against 12.3 us, but
    // 12288 x 4096 Q4_K 17.4 / 21.1 against 17.7 / 17.8 us (the records of
    // every token make each block's work longer than its bytes take to
    // arrive).  Q8_0 has only this kernel.
    if (batch > 2 && type != kQ8_0 && (uint64_t)rows * columns > (20ull << 20)) return false;
    return plan8(type, (uint32_t)rows, (uint32_t)columns, (uint32_t)batch, 1).s != 0;
}

bool qmv8_gate_up_supported(uint32_t type, size_t rows, size_t columns, size_t batch) {
    if (type != kQ4_K && type != kQ6_K) return false;
    // Gate/up pairs of 3-4 tokens measured slower here than on the fp16
    // kernels with their preparation launch (C3, Q4_K 12288 x 4096, 4
    // tokens: 37.5 us against 19.4 + 4.6 us): the records of both matrices'
    // token blocks leave one 8-wave workgroup per CU.
    if (batch < 1 || batch > 2 || columns % 256 || columns == 0) return false;
    return plan8(type, (uint32_t)rows, (uint32_t)columns, (uint32_t)batch, 2).s != 0;
}

hipError_t launch_qmv8(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns, const void *w,
                       uint32_t batch, const float *x, float *y, ArgmaxPartial *partials, uint32_t *count,
                       ArgmaxFinish finish) {
    const Args8 a{rows, columns, w, w, x, 0, 0.0f, y, partials, count, finish};
    const int mode = partials ? 1 : 0;
    if (type == kQ4_K) return launch8<kQ4_K>(ctx, batch, mode, a);
    if (type == kQ8_0) return launch8<kQ8_0>(ctx, batch, mode, a);
    return launch8<kQ6_K>(ctx, batch, mode, a);
}

hipError_t launch_qmv8_gate_up(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns,
                               const void *gate, const void *up, uint32_t batch, const float *x, float *act,
                               int normalize, float epsilon) {
    const Args8 a{rows, columns, gate, up, x, normalize, epsilon, act, nullptr, nullptr,
                  ArgmaxFinish{nullptr, nullptr, nullptr, nullptr}};
    if (type == kQ4_K) return launch8<kQ4_K>(ctx, batch, 2, a);
    return launch8<kQ6_K>(ctx, batch, 2, a);
}

bool qmv8_grouped_supported(uint32_t type, size_t rows, size_t columns, uint32_t mats) {
    if (type != kQ4_K && type != kQ6_K) return false;
    if (columns % 256 || columns == 0 || rows == 0 || columns > 0xffffffffull || rows > 0xffffffffull)
        return false;
    const uint64_t bytes = (uint64_t)rows * (columns / 256) * (type == kQ4_K ? 144u : 210u);
    if (bytes * mats >= (1ull << 32)) return false;
    return plan8_grouped(type, (uint32_t)rows, (uint32_t)columns, 2, mats, 1).s != 0;
}

hipError_t launch_qmv8_grouped(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns, int gate_up,
                               uint64_t up_offset, const QmvJob *jobs, size_t count, const float *x, float *y,
                               const uint64_t *dev_w, const uint32_t *go, const QmvCombine *combine,
                               uint32_t go_count) {
    const uint32_t mats = gate_up ? 2u : 1u;
    // device-side addresses (and the fused combine): one launch of one-token
    // jobs, in order
    if (dev_w || combine) {
        if (count > kMaxJobs8) return hipErrorInvalidValue;
        for (size_t i = 0; i < count; i++)
            if (jobs[i].tokens != 1) return hipErrorInvalidValue;
    }
    DeviceJobs dj{dev_w, go, go_count, Combine8{nullptr, nullptr, nullptr, 1u, 0u}};
    if (combine) {
        // the combine reads job p's rows at y + p * rows, and needs a split
        // launch (one workgroup holds whole tiles of every job) with a ticket
        // per token and row-tile workgroup
        for (size_t i = 0; i < count; i++)
            if (jobs[i].y_off != i * rows) return hipErrorInvalidValue;
        if (combine->k == 0 || count % combine->k != 0) return hipErrorInvalidValue;
        const Plan8 p = plan8_grouped(type, rows, columns, 1, mats, (uint32_t)count);
        if (gate_up || p.s < 2) return hipErrorInvalidValue;
        const size_t groups = ((size_t)(rows + 15) / 16 + 8 / p.s - 1) / (8 / p.s);
        if (groups * (count / combine->k) > combine->tickets_count) return hipErrorInvalidValue;
        dj.cb = Combine8{combine->tickets, combine->p, combine->y, combine->k, combine->y_stride};
    }
    // Jobs of one and of two tokens go to separate launches, kMaxJobs8 each.
    for (uint32_t tok = 1; tok <= 2; tok++) {
        size_t i = 0;
        while (i < count) {
            JobTable8 table;
            uint32_t n = 0;
            for (; i < count && n < kMaxJobs8; i++) {
                const QmvJob &j = jobs[i];
                if (j.tokens != tok) continue;
                table.job[n++] = Job8{(uint64_t)(uintptr_t)j.w, j.x_off, j.y_off, j.x_stride, j.y_stride};
            }
            if (n == 0) continue;
            // the split is planned for the jobs of this launch
            const Plan8 p = plan8_grouped(type, rows, columns, tok, mats, n);
            if (p.s == 0) return hipErrorInvalidValue;
            hipError_t e;
            if (type == kQ4_K) {
                e = gate_up ? (tok == 1 ? run8_grouped_s<kQ4_K, 2, 1>(ctx, p, rows, columns, up_offset, table, n, x, y, dj)
                                        : run8_grouped_s<kQ4_K, 2, 2>(ctx, p, rows, columns, up_offset, table, n, x, y, dj))
                            : (tok == 1 ? run8_grouped_s<kQ4_K, 0, 1>(ctx, p, rows, columns, 0, table, n, x, y, dj)
                                        : run8_grouped_s<kQ4_K, 0, 2>(ctx, p, rows, columns, 0, table, n, x, y, dj));
            } else {
                e = gate_up ? (tok == 1 ? run8_grouped_s<kQ6_K, 2, 1>(ctx, p, rows, columns, up_offset, table, n, x, y, dj)
                                        : run8_grouped_s<kQ6_K, 2, 2>(ctx, p, rows, columns, up_offset, table, n, x, y, dj))
                            : (tok == 1 ? run8_grouped_s<kQ6_K, 0, 1>(ctx, p, rows, columns, 0, table, n, x, y, dj)
                                        : run8_grouped_s<kQ6_K, 0, 2>(ctx, p, rows, columns, 0, table, n, x, y, dj));
            }
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

// A kernel of this file: resolving it loads the file's code object.
const void *module_anchor_qmv8() { return (const void *)qmv8_kernel<kQ4_K, 16, 0, 1, 1, 16>; }

}  // namespace dm
