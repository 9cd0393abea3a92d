// kernels_gemm.hip -- prefill GEMM C[m][n] = sum_k A[m][k] * W[n][k] for gfx950.
//
// A is bf16 activations [m][k]; W is n encoded rows of k columns.  The
// reference has no batched prefill: it runs one matvec per token
// (src/gemma4/metal.rs:514-536), so the result for token m must match
// cpu::matvec(W, widen(A[m])) (src/cpu.rs:345-399) within the GEMM tolerance
// (max |c - r| <= 1e-3 max |r|, cosine >= 0.99999).
//
// Q4_K, Q6_K and Q8_0 weights run on v_mfma_f32_32x32x16_f16 with fp32
// accumulation after an on-the-fly dequantization to fp16:
//  * A: the columns a wave sums over (one quarter of K, below) are scaled per
//    row by a power of two 2^-e (their max |a| 2^-e in [2^14, 2^15)) and
//    converted to fp16.  bf16 carries 8 significant bits, so the conversion is
//    exact for every value above 2^-17 of that maximum; the wave multiplies
//    its partial sums back by 2^e before the quarters are added.
//  * W, one rounding per factor, fp16 in place of the reference's fp32
//    (src/cpu.rs:576-645):
//      Q4_K  fma(q, fp16(d sc_j), fp16(-dmin m_j)); the nibble q is read as an
//            fp8 e4m3 code (codes 0..15 are q 2^-9 exactly) by
//            v_cvt_scalef32_pk_f16_fp8 with scale 2^9;
//      Q6_K  (q - 32) fp16(d sc_j): the 6-bit q becomes the fp16 1024 + q by
//            placing it under the exponent of 1024 (v_perm_b32), 1056 is
//            subtracted exactly, one product rounds;
//      Q8_0  q d: the byte q + 128 becomes 1024 + q + 128 the same way, 1152
//            is subtracted exactly, one product rounds.
//    These roundings leave a few 1e-4 of max |r| on seeded data.
// The sum over K is order-free, so the columns of each 256-column block are
// permuted once for both operands: MFMA step s of a block, lane half h,
// element e of the lane's 8 holds column base(s, h) + e % 4 + run (e / 4)
// (per format below), chosen so that a lane's 8 weights come from one or two
// aligned dwords of the block.  The A preparation stores A in that order.
//
// Tiling: a workgroup of 4 waves (one per SIMD) owns a 128 x 64 tile of C;
// wave w sums over the w-th quarter of the K blocks (no operand is shared
// between waves), with 4 x 2 MFMA tiles of 32 x 32 in AGPRs, so every
// dequantized weight feeds four MFMAs.  A arrives from global memory already
// in fragment order (one 1 KiB load per 32 rows and step, kADist steps ahead
// of its use); W for the wave's 64 rows is staged one block at a time in the
// wave's own LDS area, fetched into registers one block ahead and written to
// LDS two thirds through the current block, so the next block's scales are
// decoded while the current block's MFMAs run.  Workgroups are persistent
// (one per CU): a wave walks its tiles' blocks as one sequence, so the next
// tile's first loads are in flight during a tile's final sum.  The quarters'
// partial tiles are added through LDS (two regions, column-major, 16-byte
// accesses).  Tiles are ordered so that each XCD keeps half of A in its L2.
#include "dm_device.h"
#include "dm_qmv.h"
#include "runtime.h"


namespace dm {

namespace {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));  // 16-byte aligned

constexpr uint32_t kBN = 64, kWaves = 4;
constexpr uint32_t kPadRows = 128;  // workspace rows are padded to every tile height
// MFMA steps between the load of an A fragment and its use.  Loads complete
// in order, so this is also the time every W load has to arrive.
constexpr uint32_t kADist = 4;
static_assert(16 % kADist == 0, "the A ring repeats every block");

// Tile shape: RM = 4 MFMA row tiles per wave, a 128 x 64 tile per workgroup,
// one persistent workgroup per CU (one wave per SIMD).  (64 x 64 tiles with
// two workgroups per CU measured no faster: the loop's MFMA share is the
// same, and each weight then feeds two MFMAs instead of four.)  W of a
// tile's next block is staged during the current tile's last block, so the
// partial tiles have LDS of their own: [W staging][2 partial tiles][row
// scales].
template <uint32_t RM>
struct Tile {
    static constexpr uint32_t kRM = RM, kBM = 32 * RM;
    static constexpr uint32_t kRedLd = kBM / 2 + 4;  // floats per column of an exchange region (64 rows)
    static constexpr uint32_t kRedBytes = kWaves * kBN * kRedLd * 4;
    template <class F>
    static constexpr uint32_t stage_bytes() { return kWaves * 64 * F::kChunks * 16; }
    template <class F>
    static constexpr uint32_t red_offset() { return stage_bytes<F>(); }
    template <class F>
    static constexpr uint32_t rsl_offset() { return stage_bytes<F>() + kRedBytes; }
    template <class F>
    static constexpr uint32_t lds_bytes() { return rsl_offset<F>() + kWaves * kBM * 4; }
};
constexpr uint32_t kRowTiles = 4;

__device__ __forceinline__ floatx16 mfma32(half8 a, half8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half2_t splat(float v) {
    const _Float16 x = (_Float16)v;
    return half2_t{x, x};
}

// The byte pairs (b0, b1) / (b2, b3) of v as the fp16 pair (1024 + b0, 1024 + b1)
// / (1024 + b2, 1024 + b3): each byte under the exponent byte 0x64.
__device__ __forceinline__ half2_t magic_lo(uint32_t v) {
    return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u));
}
__device__ __forceinline__ half2_t magic_hi(uint32_t v) {
    return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u));
}

// Workgroup barrier ordering LDS only: the wave's global loads in flight
// (the next tile's W and A) are not waited for, as __syncthreads() would.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Dword x of a span that starts o bytes (0..3) into the aligned dwords d.
__device__ __forceinline__ uint32_t span_dword(const uint32_t *d, uint32_t x, uint32_t o) {
    return funnel(d[x], d[x + 1], o);
}

// ---------------------------------------------------------------------------
// Weight formats.  Per 256-column block of a row: kSpan encoded bytes, staged
// as kChunks 16-byte pieces starting at the span's 4-byte-aligned start
// (the span itself when kAligned), the span beginning span_shift bytes into
// the staged row.
// From its staged row (dwords `row`), a lane reads the block's header (Head,
// turned into per-block Scales for its column and half) and, one MFMA step at
// a time, the few dwords of that step (Step); weights() gives the step's 8
// fp16 weights.
// ---------------------------------------------------------------------------

// Q4_K (src/cpu.rs:585-616): d, dmin, 12 scale bytes, 128 qs bytes.  Lane
// half h takes sub-blocks 4h .. 4h + 3; step s reads qs dword 16h + s: low
// nibbles are columns base .. base + 3, high nibbles base + 32 .. base + 35.
struct FormatQ4K {
    static constexpr uint32_t kType = kQ4_K, kSpan = 144, kChunks = 9, kRun = 32;
    __host__ __device__ static constexpr uint32_t base(uint32_t s, uint32_t h) { return 64 * (2 * h + s / 8) + 4 * (s % 8); }
    static constexpr bool kAligned = true;  // spans start 4-byte aligned when rows do
    __device__ static uint32_t span_shift(uint32_t, uint32_t) { return 0; }
    struct Head {
        v4u v;
    };
    struct Sub {
        half2_t mul, add;  // (d sc, d sc), (-dmin m, -dmin m)
    };
    struct Scales {
        Sub sub[4];
    };
    struct Step {
        uint32_t q;
    };
    __device__ static Head head(const uint32_t *row, uint32_t, uint32_t) { return Head{*(const v4u *)row}; }
    __device__ static Scales scales(const Head &hd_, uint32_t h) {
        const v4u hd = hd_.v;
        const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hd[0] & 0xffffu));
        const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hd[0] >> 16));
        // 6-bit scales and mins of sub-blocks 0-3 and 4-7, as bytes
        // (src/cpu.rs:607-616)
        const uint32_t sc03 = hd[1] & 0x3f3f3f3fu, mn03 = hd[2] & 0x3f3f3f3fu;
        const uint32_t sc47 = (hd[3] & 0x0f0f0f0fu) | ((hd[1] >> 2) & 0x30303030u);
        const uint32_t mn47 = ((hd[3] >> 4) & 0x0f0f0f0fu) | ((hd[2] >> 2) & 0x30303030u);
        const uint32_t scs = h ? sc47 : sc03, mns = h ? mn47 : mn03;
        Scales r;
#pragma unroll
        for (int x = 0; x < 4; x++) {
            r.sub[x].mul = splat(d * (float)((scs >> (8 * x)) & 0xffu));
            r.sub[x].add = splat(-dmin * (float)((mns >> (8 * x)) & 0xffu));
        }
        return r;
    }
    __device__ static Step step(const uint32_t *row, uint32_t h, uint32_t s, uint32_t) { return Step{row[4 + 16 * h + s]}; }
    __device__ static half8 weights(const Scales &sc, const Step &st, uint32_t s) {
        const Sub &lo = sc.sub[2 * (s / 8)], &hi = sc.sub[2 * (s / 8) + 1];
        const uint32_t l4 = st.q & 0x0f0f0f0fu, h4 = (st.q >> 4) & 0x0f0f0f0fu;
        const half2_t a0 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l4, 512.0f, false)), lo.mul, lo.add);
        const half2_t a1 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l4, 512.0f, true)), lo.mul, lo.add);
        const half2_t a2 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(h4, 512.0f, false)), hi.mul, hi.add);
        const half2_t a3 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(h4, 512.0f, true)), hi.mul, hi.add);
        return half8{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
    }
};

// Q6_K (src/cpu.rs:618-645): ql[128], qh[64], 16 int8 scales, d.  Lane half
// h takes the block half h (ql 64h.., qh 32h.., scales 8h..); step s reads ql
// dword 16h + s and qh dword 32 + 8h + s % 8 (bit pair s / 8): low nibbles
// are columns 128h + 4s .. + 3 (scale 8h + s / 4), high nibbles those + 64
// (scale 8h + s / 4 + 4).  Spans are 2-byte aligned: the staged row starts
// at the span's aligned-down dword.
struct FormatQ6K {
    static constexpr uint32_t kType = kQ6_K, kSpan = 210, kChunks = 14, kRun = 64;
    __host__ __device__ static constexpr uint32_t base(uint32_t s, uint32_t h) { return 128 * h + 4 * s; }
    static constexpr bool kAligned = false;
    __device__ static uint32_t span_shift(uint32_t row_offset, uint32_t b) { return (row_offset + kSpan * b) & 3u; }
    struct Head {
        uint32_t s0, s1, d;  // scales 8h .. 8h + 3, 8h + 4 .. 8h + 7; d in the low half
    };
    struct Scales {
        half2_t lo[4], hi[4];  // (d sc, d sc) of scales 8h + x and 8h + x + 4
    };
    struct Step {
        uint32_t ql, qh;
    };
    __device__ static Head head(const uint32_t *row, uint32_t h, uint32_t o) {
        return Head{span_dword(row, 48 + 2 * h, o), span_dword(row, 49 + 2 * h, o), span_dword(row, 52, o)};
    }
    __device__ static Scales scales(const Head &hd, uint32_t) {
        const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hd.d & 0xffffu));
        Scales r;
#pragma unroll
        for (int x = 0; x < 4; x++) {
            r.lo[x] = splat(d * (float)(int8_t)(hd.s0 >> (8 * x)));
            r.hi[x] = splat(d * (float)(int8_t)(hd.s1 >> (8 * x)));
        }
        return r;
    }
    __device__ static Step step(const uint32_t *row, uint32_t h, uint32_t s, uint32_t o) {
        return Step{span_dword(row, 16 * h + s, o), span_dword(row, 32 + 8 * h + s % 8, o)};
    }
    __device__ static half8 weights(const Scales &sc, const Step &st, uint32_t s) {
        const uint32_t l = st.ql, q = st.qh >> (2 * (s / 8));
        const uint32_t lo6 = (l & 0x0f0f0f0fu) | ((q << 4) & 0x30303030u);
        const uint32_t hi6 = ((l >> 4) & 0x0f0f0f0fu) | (q & 0x30303030u);
        const half2_t off = half2_t{(_Float16)-1056.0f, (_Float16)-1056.0f};
        const half2_t a0 = (magic_lo(lo6) + off) * sc.lo[s / 4];
        const half2_t a1 = (magic_hi(lo6) + off) * sc.lo[s / 4];
        const half2_t a2 = (magic_lo(hi6) + off) * sc.hi[s / 4];
        const half2_t a3 = (magic_hi(hi6) + off) * sc.hi[s / 4];
        return half8{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
    }
};

// Q8_0 (src/cpu.rs:576-583): eight 34-byte blocks (d, 32 int8) per 256
// columns.  Lane half h takes blocks 4h .. 4h + 3; step s reads bytes
// 8 (s % 4) .. + 7 of block 4h + s / 4's quants: columns 128h + 8s .. + 7.
// Block 4h + g starts at byte 136h + 34g: the quants of even g start 2 bytes
// past a dword boundary (d in the low half of that dword), those of odd g on
// one (d in the high half of the dword before).
struct FormatQ80 {
    static constexpr uint32_t kType = kQ8_0, kSpan = 272, kChunks = 17, kRun = 4;
    __host__ __device__ static constexpr uint32_t base(uint32_t s, uint32_t h) { return 128 * h + 8 * s; }
    static constexpr bool kAligned = true;
    __device__ static uint32_t span_shift(uint32_t, uint32_t) { return 0; }
    struct Head {};
    struct Scales {};
    struct Step {
        uint32_t q0, q1;
        half2_t d;
    };
    __device__ static Head head(const uint32_t *, uint32_t, uint32_t) { return Head{}; }
    __device__ static Scales scales(const Head &, uint32_t) { return Scales{}; }
    __device__ static Step step(const uint32_t *row, uint32_t h, uint32_t s, uint32_t) {
        const uint32_t g = s / 4, i = 2 * (s % 4);
        Step r;
        if (g % 2 == 0) {
            const uint32_t *p = row + 34 * h + 17 * (g / 2);
            r.d = __builtin_bit_cast(half2_t, (p[0] & 0xffffu) * 0x00010001u);
            const uint32_t v0 = p[i], v1 = p[i + 1], v2 = p[i + 2];
            r.q0 = funnel(v0, v1, 2);
            r.q1 = funnel(v1, v2, 2);
        } else {
            const uint32_t *p = row + 34 * h + (17 * g - 1) / 2;
            r.d = __builtin_bit_cast(half2_t, (p[0] >> 16) * 0x00010001u);
            r.q0 = p[1 + i];
            r.q1 = p[2 + i];
        }
        return r;
    }
    __device__ static half8 weights(const Scales &, const Step &st, uint32_t) {
        const uint32_t x0 = st.q0 ^ 0x80808080u, x1 = st.q1 ^ 0x80808080u;
        const half2_t off = half2_t{(_Float16)-1152.0f, (_Float16)-1152.0f};
        const half2_t a0 = (magic_lo(x0) + off) * st.d;
        const half2_t a1 = (magic_hi(x0) + off) * st.d;
        const half2_t a2 = (magic_lo(x1) + off) * st.d;
        const half2_t a3 = (magic_hi(x1) + off) * st.d;
        return half8{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
    }
};

// The K blocks [begin, end) wave (or quarter) w of 4 sums over.
__host__ __device__ inline uint32_t quarter_begin(uint32_t blocks, uint32_t w) { return blocks * w / kWaves; }

}  // namespace

// ---------------------------------------------------------------------------
// A preparation over the padded workspace (rows beyond M are zero).  For the
// 32-row tile T = m / 32 and lane l = m % 32 + 32 h:
//   a16[((T * blocks + b) * 16 + s) * 64 + l]  half8: A[m][k] * 2^-e at the
//       8 columns of step s, half h of block b (F::base, F::kRun)
//   rowscale[q * mp + m]                       2^e of quarter q of row m
// Workgroup (g, q) takes rows 8 g .. 8 g + 7 and the K blocks of quarter q:
// 32 threads per row load the quarter's columns into LDS and find their max,
// then each thread converts fragments of one row; the 8 rows' fragments of
// one (block, step, half) are consecutive in a16, so 8 neighbouring threads
// store one 128-byte line.  rowscale is 2^e with max 2^-e in [2^14, 2^15)
// (1 for an all-zero or non-finite quarter, 0 for the padding rows).  (One
// wave per row and quarter, with the fragments formed in registers, measured
// slower: its 16-byte stores land on 64 different lines each.)
// ---------------------------------------------------------------------------
template <class F>
__global__ void __launch_bounds__(256) gemm_prep_kernel(const uint16_t *__restrict__ a, uint32_t m_rows, uint32_t k,
                                                        uint32_t mp, half8 *__restrict__ a16,
                                                        float *__restrict__ rowscale) {
    extern __shared__ uint32_t prep_tile[];
    __shared__ float sdown[8];
    const uint32_t tid = threadIdx.x, blocks = k / 256, q = blockIdx.y;
    const uint32_t b0 = quarter_begin(blocks, q), nb = quarter_begin(blocks, q + 1) - b0;
    const uint32_t ld = nb * 128 + 4;  // dwords per staged row
    const uint32_t r0 = blockIdx.x * 8;
    {
        const uint32_t i = tid >> 5, lc = tid & 31u, m = r0 + i;
        const bool live = m < m_rows;
        const u32x4 *row = (const u32x4 *)(a + (size_t)m * k + (size_t)b0 * 256);
        float mx = 0.0f;
        const uint32_t chunks = nb * 32;
        uint32_t c = lc;
        for (; c + 32 * 3 < chunks; c += 32 * 4) {
            u32x4 v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = live ? row[c + 32 * j] : u32x4{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 4; j++) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    mx = fmaxf(mx, fabsf(__uint_as_float(v[j][e] << 16)));
                    mx = fmaxf(mx, fabsf(__uint_as_float(v[j][e] & 0xffff0000u)));
                }
                *(u32x4 *)&prep_tile[i * ld + (c + 32 * j) * 4] = v[j];
            }
        }
        for (; c < chunks; c += 32) {
            const u32x4 v = live ? row[c] : u32x4{0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                mx = fmaxf(mx, fabsf(__uint_as_float(v[e] << 16)));
                mx = fmaxf(mx, fabsf(__uint_as_float(v[e] & 0xffff0000u)));
            }
            *(u32x4 *)&prep_tile[i * ld + c * 4] = v;
        }
#pragma unroll
        for (int s = 16; s >= 1; s >>= 1) mx = fmaxf(mx, __shfl_xor(mx, s, 64));
        int e = 0;
        if (mx > 0.0f && __builtin_isfinite(mx)) {
            int ex;
            (void)frexpf(mx, &ex);
            e = ex - 15;
            if (e < -126) e = -126;
            if (e > 127) e = 127;
        }
        if (lc == 0) {
            sdown[i] = live ? ldexpf(1.0f, -e) : 0.0f;
            rowscale[(size_t)q * mp + m] = live ? ldexpf(1.0f, e) : 0.0f;
        }
    }
    __syncthreads();
    // thread: row i = tid & 7, fragment f = tid >> 3 (half f / 16, step f % 16)
    const uint32_t i = tid & 7u, f = tid >> 3, h = f >> 4, st = f & 15u;
    const float down = sdown[i];
    const uint32_t fb = F::base(st, h), tl = r0 / 32, l0 = r0 % 32;
    for (uint32_t bq = 0; bq < nb; bq++) {
        const uint32_t *t = &prep_tile[i * ld + bq * 128];
        // columns fb .. fb + 3 and fb + kRun .. + 3: bf16 pairs (dwords) fb / 2 ..
        const u32x2 p0 = *(const u32x2 *)&t[fb / 2], p1 = *(const u32x2 *)&t[(fb + F::kRun) / 2];
        const uint32_t u[4] = {p0[0], p0[1], p1[0], p1[1]};
        half8 v;
#pragma unroll
        for (int x = 0; x < 4; x++) {
            v[2 * x] = (_Float16)(__uint_as_float(u[x] << 16) * down);
            v[2 * x + 1] = (_Float16)(__uint_as_float(u[x] & 0xffff0000u) * down);
        }
        a16[((size_t)(tl * blocks + b0 + bq) * 16 + st) * 64 + l0 + i + 32 * h] = v;
    }
}

// ---------------------------------------------------------------------------
// GEMM main kernel.  Grid: one persistent workgroup per CU (at most one per
// tile); workgroup g takes tiles g, g + grid, ...  Wave w sums over the K
// blocks of quarter w of each tile; its (tile, block) pairs form one sequence
// whose loads run ahead across tile boundaries.  Per block: 16 MFMA steps of
// 4 x 2 MFMAs; step s issues the A loads of step s + kADist, the LDS reads of
// step s + 2 and the dequantization of step s + 1.  At step 14 (after the
// last read of the block, made at step 13) the next block's W, fetched into
// registers a block earlier, is written to the wave's LDS area and the W of
// the block after it is fetched; the next block's header and first steps
// are read at steps 14 and 15.
// ---------------------------------------------------------------------------
template <class F, uint32_t RM>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_kernel(const half8 *__restrict__ a16, uint32_t a_bytes, const float *__restrict__ rowscale, uint32_t mp,
            const uint8_t *__restrict__ w, uint32_t w_bytes, uint32_t m_rows, uint32_t n_rows, uint32_t k,
            uint32_t m_tiles, uint32_t n_tiles, float *__restrict__ c) {
    using T = Tile<RM>;
    constexpr uint32_t kChunks = F::kChunks, kStageDwords = 64 * kChunks * 4, kRM = RM, kBM = T::kBM;
    constexpr uint32_t kRedLd = T::kRedLd;
    extern __shared__ v4u gsm[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar offsets
    const uint32_t ln = lane & 31u, h = lane >> 5;
    const uint32_t blocks = k / 256, row_bytes = blocks * F::kSpan, tiles = m_tiles * n_tiles;
    const uint32_t kb0 = quarter_begin(blocks, wave), kb1 = quarter_begin(blocks, wave + 1);
    uint32_t *stage = (uint32_t *)gsm + wave * kStageDwords;
    float *red = (float *)((char *)gsm + T::template red_offset<F>());
    float *rsl = (float *)((char *)gsm + T::template rsl_offset<F>()) + wave * kBM;  // the wave's row scales of the tile
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(w, w_bytes), ars = make_rsrc(a16, a_bytes);
    const __amdgpu_buffer_rsrc_t crs = make_rsrc(c, m_rows * n_rows * 4);

    // Position in the wave's (tile, block) sequence; t >= tiles past the end.
    // The 8 XCDs take workgroups round-robin (XCD = id % 8, and the grid is a
    // multiple of 8 or the tile count), each with its own L2: when the tiles
    // split evenly, XCD x works on M half x % 2 and N quarter x / 2, so its
    // half of A stays in its L2 and the tiles sharing a W tile run there.
    struct Pos {
        uint32_t t, b, mt, nt;
    };
    auto at = [&](uint32_t t, uint32_t b) {
        Pos p{t, b, 0, 0};
        if (m_tiles % 2 == 0 && n_tiles % 4 == 0) {
            const uint32_t xcd = t % 8, j = t / 8, mh = m_tiles / 2;
            p.mt = (xcd & 1u) * mh + j % mh;
            p.nt = (xcd >> 1) * (n_tiles / 4) + j / mh;
        } else {
            p.mt = t % m_tiles;
            p.nt = t / m_tiles;
        }
        return p;
    };
    auto next = [&](const Pos &p) { return p.b + 1 < kb1 ? Pos{p.t, p.b + 1, p.mt, p.nt} : at(p.t + gridDim.x, kb0); };

    // W staging: chunk j * 64 + lane of the block's 64 rows x kChunks pieces,
    // which is also its 16-byte slot in the wave's LDS area.  wlane[j] is the
    // chunk's offset from the first row's span; rows past n start at or past
    // w_bytes, where buffer loads read zeros (the range check covers the
    // lane offset, so every row-dependent term goes there).
    uint32_t wlane[kChunks];
#pragma unroll
    for (uint32_t j = 0; j < kChunks; j++) {
        const uint32_t chunk = j * 64 + lane;
        wlane[j] = chunk / kChunks * row_bytes + chunk % kChunks * 16;
    }
    v4u wreg[kChunks];
    auto fetch_w = [&](const Pos &p) {
        const uint32_t u = p.nt * kBN * row_bytes;
#pragma unroll
        for (uint32_t j = 0; j < kChunks; j++) {
            uint32_t off, soff;
            if constexpr (F::kAligned) {
                off = wlane[j] + u;
                soff = F::kSpan * p.b;
            } else {
                off = (wlane[j] + u + F::kSpan * p.b) & ~3u;  // the span's aligned-down start
                soff = 0;
            }
            wreg[j] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(wrs, off, soff, 0));
        }
    };
    auto put_w = [&]() {
#pragma unroll
        for (uint32_t j = 0; j < kChunks; j++) ((v4u *)stage)[j * 64 + lane] = wreg[j];
    };
    // A fragment of row tile r (32 rows), step s of p's block.
    // (The step within its group of 4 goes to the instruction's offset field.)
    auto a_frag = [&](const Pos &p, uint32_t r, uint32_t s) {
        const uint32_t off = (((kRM * p.mt + r) * blocks + p.b) * 16 + (s & ~3u)) * 1024;
        return __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(ars, 16 * lane + 1024 * (s % 4), off, 0));
    };
    // The lane's staged rows (column tile t: row 32 t + ln of the block) and
    // the span offsets of p's block in them.
    const uint32_t *rows[2] = {stage + ln * kChunks * 4, stage + (32 + ln) * kChunks * 4};
    auto shift = [&](const Pos &p, int t) { return F::span_shift((p.nt * kBN + 32 * t + ln) * row_bytes, p.b); };

    if (blockIdx.x >= tiles) return;
    floatx16 acc[kRM][2];
    Pos cur = at(blockIdx.x, kb0);
    const bool any = kb0 < kb1;  // waves of a K shorter than 4 blocks may have none
    typename F::Scales sc[2];
    typename F::Step sa[2];  // the LDS data of the step after the current one
    half8 afr[kRM][kADist], bv[2];
    uint32_t sh[2] = {0, 0};
    if (any) {
        fetch_w(cur);
        put_w();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        const Pos n1 = next(cur);
        if (n1.t < tiles) fetch_w(n1);
#pragma unroll
        for (uint32_t s = 0; s < kADist; s++)
#pragma unroll
            for (uint32_t r = 0; r < kRM; r++) afr[r][s] = a_frag(cur, r, s);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            sh[t] = shift(cur, t);
            sc[t] = F::scales(F::head(rows[t], h, sh[t]), h);
            bv[t] = F::weights(sc[t], F::step(rows[t], h, 0, sh[t]), 0);
            sa[t] = F::step(rows[t], h, 1, sh[t]);
        }
    }
    float2 rsv = {0.0f, 0.0f};
    for (;;) {
        const uint32_t m0 = cur.mt * kBM, n0 = cur.nt * kBN, tile = cur.t;
#pragma unroll
        for (uint32_t r = 0; r < kRM; r++)
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int j = 0; j < 16; j++) acc[r][t][j] = 0.0f;
        for (uint32_t b = kb0; b < kb1; b++) {
            const Pos n1 = next(cur);
            const bool have1 = n1.t < tiles;
            const Pos &pa = have1 ? n1 : cur;  // the A ring's next block (clamped at the end)
            if (b + 1 == kb1) {
                // this quarter's row scales for the final sum, kBM / 64 per lane
                if constexpr (kBM == 128) {
                    rsv = *(const float2 *)&rowscale[(size_t)wave * mp + m0 + 2 * lane];
                } else {
                    rsv.x = rowscale[(size_t)wave * mp + m0 + lane];
                }
            }
            typename F::Head hn[2];
            uint32_t shn[2] = {0, 0};
#pragma unroll
            for (uint32_t s = 0; s < 16; s++) {
                __builtin_amdgcn_sched_barrier(0);
                if (s == 14 && have1) {
                    // Every LDS read of this block is done (the last, of step
                    // 15, at step 13); other lanes read what a lane stores, and
                    // the wave's LDS operations run in order.
                    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                    put_w();
                    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                    const Pos n2 = next(n1);
                    if (n2.t < tiles) fetch_w(n2);
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        shn[t] = shift(n1, t);
                        hn[t] = F::head(rows[t], h, shn[t]);
                    }
                }
                // LDS data of step s + 2 (the next block's first steps at the end)
                typename F::Step sb[2];
                if (s + 2 < 16) {
#pragma unroll
                    for (int t = 0; t < 2; t++) sb[t] = F::step(rows[t], h, s + 2, sh[t]);
                } else if (have1) {
#pragma unroll
                    for (int t = 0; t < 2; t++) sb[t] = F::step(rows[t], h, s + 2 - 16, shn[t]);
                }
                // The A fragments of step s + kADist and the weights of step
                // s + 1 are produced before this step's MFMAs consume the
                // current ones, so they live in other registers.
                half8 an[kRM];
#pragma unroll
                for (uint32_t r = 0; r < kRM; r++)
                    an[r] = s + kADist < 16 ? a_frag(cur, r, s + kADist) : a_frag(pa, r, s + kADist - 16);
                half8 bn[2];
                if (s + 1 < 16) {
#pragma unroll
                    for (int t = 0; t < 2; t++) bn[t] = F::weights(sc[t], sa[t], s + 1);
                } else if (have1) {
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        sc[t] = F::scales(hn[t], h);
                        bn[t] = F::weights(sc[t], sa[t], 0);
                    }
                }
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (uint32_t r = 0; r < kRM; r++) acc[r][t] = mfma32(afr[r][s % kADist], bv[t], acc[r][t]);
#pragma unroll
                for (uint32_t r = 0; r < kRM; r++) afr[r][s % kADist] = an[r];
                if (s + 1 < 16 || have1) {
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        bv[t] = bn[t];
                        sa[t] = sb[t];
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            sh[0] = shn[0];
            sh[1] = shn[1];
            cur = n1;
        }
        if (!any) cur = at(tile + gridDim.x, kb0);

        // Final sum of the tile.  Each wave multiplies its quarter's partial
        // tile by the quarter's row scales, then partners exchange halves
        // through LDS in two rounds (every wave busy in both): with waves
        // 0/2 and 1/3 as partners, wave w keeps rows 64 (w / 2) .. + 63 and
        // hands the other 64 rows to its partner; then with waves 0/1 and 2/3
        // as partners it keeps rows 32 w .. 32 w + 31 and hands over the
        // other 32.  Wave w then holds the sum of all four quarters for rows
        // 32 w .. + 31 and stores them.  Regions are laid out [column][row]
        // (a lane's 4 consecutive rows of one column are one 16-byte
        // access); the second round writes into the region the wave itself
        // read in the first, which no other wave reads.
        if constexpr (kBM == 128) {
            *(float2 *)&rsl[2 * lane] = rsv;
        } else {
            rsl[lane] = rsv.x;
        }
        lds_barrier();  // every wave is done with its K blocks and with the previous tile's final sum
        constexpr uint32_t kRegion = kBN * kRedLd;  // floats of one exchange region
        auto slot = [&](uint32_t region, uint32_t row, int t) {
            return (floatx4 *)&red[region * kRegion + (32 * t + ln) * kRedLd + row];
        };
        const uint32_t keep_half = wave >> 1, keep_quarter = wave & 1u;
#pragma unroll
        for (uint32_t r = 0; r < kRM; r++) {
            floatx4 rs[4];
#pragma unroll
            for (int g = 0; g < 4; g++) rs[g] = *(const floatx4 *)&rsl[32 * r + 8 * g + 4 * h];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int g = 0; g < 4; g++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[r][t][4 * g + e] *= rs[g][e];
        }
        // first exchange: rows of the other half to region `wave`
#pragma unroll
        for (uint32_t r = 0; r < kRM; r++) {
            if (r / 2 == keep_half) continue;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    *slot(wave, 32 * (r % 2) + 8 * g + 4 * h, t) =
                        floatx4{acc[r][t][4 * g], acc[r][t][4 * g + 1], acc[r][t][4 * g + 2], acc[r][t][4 * g + 3]};
        }
        lds_barrier();
#pragma unroll
        for (uint32_t r = 0; r < kRM; r++) {
            if (r / 2 != keep_half) continue;
            floatx4 o[2][4];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int g = 0; g < 4; g++) o[t][g] = *slot(wave ^ 2u, 32 * (r % 2) + 8 * g + 4 * h, t);
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int g = 0; g < 4; g++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[r][t][4 * g + e] += o[t][g][e];
        }
        // second exchange: the other 32 rows of the kept half to region wave ^ 2
#pragma unroll
        for (uint32_t r = 0; r < kRM; r++) {
            if (r / 2 != keep_half || r % 2 == keep_quarter) continue;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    *slot(wave ^ 2u, 8 * g + 4 * h, t) =
                        floatx4{acc[r][t][4 * g], acc[r][t][4 * g + 1], acc[r][t][4 * g + 2], acc[r][t][4 * g + 3]};
        }
        lds_barrier();
        // rows 32 wave + 8 g + 4 h + e, column n0 + 32 t + ln; rows past m
        // lie past the end of C, where buffer stores are dropped (the range
        // check covers the lane offset, which holds the row).  The stores are
        // non-temporal: C is not read again here, and keeping it out of the
        // L2 left the N = 4096 kernels 0.5-0.6 us faster (all three types).
        const bool whole_n = n0 + kBN <= n_rows;
#pragma unroll
        for (uint32_t r = 0; r < kRM; r++) {
            if (r != wave) continue;
            floatx4 o[2][4];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int g = 0; g < 4; g++) o[t][g] = *slot(wave ^ 3u, 8 * g + 4 * h, t);
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int g = 0; g < 4; g++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float v = acc[r][t][4 * g + e] + o[t][g][e];
                        const uint32_t m = m0 + 32 * r + 8 * g + 4 * h + e, n = n0 + 32 * t + ln;
                        if (whole_n || n < n_rows)
                            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), crs,
                                                                  (m * n_rows + n) * 4, 0, 2);
                    }
        }
        if (cur.t >= tiles) break;
    }
}

__global__ void bf16_to_f32_kernel(const uint16_t *__restrict__ a, size_t count, float *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = __uint_as_float((uint32_t)a[i] << 16);
}

namespace {

size_t padded_rows(size_t m) { return (m + kPadRows - 1) / kPadRows * kPadRows; }

// Workspace of the MFMA path: a16 | rowscale (4 quarters).
size_t mfma_workspace(size_t m, size_t k) {
    const size_t mp = padded_rows(m);
    return mp * k * 2 + 4 * mp * 4 + 2 * 256;
}

static_assert(Tile<kRowTiles>::lds_bytes<FormatQ80>() <= 160 * 1024, "one workgroup's LDS");

template <class F, uint32_t RM>
int launch_gemm(dmhip_ctx *ctx, size_t mp, size_t m, size_t n, size_t k, const half8 *a16, const float *rowscale,
                const void *weights, uint64_t w_bytes, float *c) {
    using T = Tile<RM>;
    const uint32_t m_tiles = (uint32_t)(mp / T::kBM), n_tiles = (uint32_t)((n + kBN - 1) / kBN);
    const uint32_t tiles = m_tiles * n_tiles;
    // one workgroup per CU, a multiple of the 8 XCDs
    uint32_t grid = ctx->compute_units > 0 ? (uint32_t)ctx->compute_units / 8 * 8 : 256u;
    if (grid == 0) grid = 8;
    if (tiles < grid) grid = tiles;
    constexpr uint32_t lds = T::template lds_bytes<F>();
    static LdsLimit limit;
    DM_HIP(limit.ensure((const void *)gemm_kernel<F, RM>, lds));
    DM_HIP(launch_kernel(ctx, gemm_kernel<F, RM>, dim3(grid), dim3(64 * kWaves), lds, a16, (uint32_t)(mp * k * 2),
                         rowscale, (uint32_t)mp, (const uint8_t *)weights, (uint32_t)w_bytes, (uint32_t)m, (uint32_t)n,
                         (uint32_t)k, m_tiles, n_tiles, c));
    return DMHIP_OK;
}

template <class F>
int run_gemm(dmhip_ctx *ctx, size_t m, size_t n, size_t k, const uint16_t *a_bf16, const void *weights,
             uint64_t w_bytes, float *c, void *workspace) {
    const size_t mp = padded_rows(m);
    char *ws = (char *)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
    half8 *a16 = (half8 *)ws;
    float *rowscale = (float *)(ws + ((mp * k * 2 + 255) & ~(size_t)255));
    const uint32_t blocks = (uint32_t)(k / 256);
    // the largest quarter's columns staged per row (bf16 pairs), 8 rows
    const uint32_t qmax = (blocks + kWaves - 1) / kWaves;
    const uint32_t prep_lds = 8 * (qmax * 128 + 4) * 4;
    static LdsLimit prep_limit;
    DM_HIP(prep_limit.ensure((const void *)gemm_prep_kernel<F>, prep_lds));
    hipLaunchKernelGGL(gemm_prep_kernel<F>, dim3((uint32_t)(mp / 8), kWaves), dim3(256), prep_lds, ctx->stream,
                       a_bf16, (uint32_t)m, (uint32_t)k, (uint32_t)mp, a16, rowscale);
    DM_HIP(hipGetLastError());
    return launch_gemm<F, kRowTiles>(ctx, mp, m, n, k, a16, rowscale, weights, w_bytes, c);
}

}  // namespace

// A kernel of this file: resolving it loads the file's code object.
const void *module_anchor_gemm() { return (const void *)bf16_to_f32_kernel; }

}  // namespace dm

using namespace dm;

extern "C" {

size_t dmhip_gemm_workspace_bytes(size_t m, size_t k) {
    const size_t tokenwise = m * k * sizeof(float) + 256;
    const size_t mfma = mfma_workspace(m, k);
    return tokenwise > mfma ? tokenwise : mfma;
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

    // The MFMA path: more than 16 tokens (fewer stream W faster through the
    // decode GEMV), whole 256-column blocks, offsets that fit the 31-bit
    // buffer range, 16-byte aligned operands.
    const uint64_t w_bytes = rb * n;
    const size_t mp = padded_rows(m);
    const bool mfma = m > 16 && k % 256 == 0 && (type == kQ4_K || type == kQ6_K || type == kQ8_0) &&
                      w_bytes + 1024 < 0x7fffffffull && (uint64_t)mp * k * 2 < 0x7fffffffull &&
                      (uint64_t)m * n * 4 < 0x7fffffffull &&
                      ((uintptr_t)weights & 15u) == 0 && ((uintptr_t)a_bf16 & 15u) == 0 && ((uintptr_t)c & 15u) == 0;
    if (mfma) {
        if (type == kQ4_K) return run_gemm<FormatQ4K>(ctx, m, n, k, a_bf16, weights, w_bytes, c, workspace);
        if (type == kQ6_K) return run_gemm<FormatQ6K>(ctx, m, n, k, a_bf16, weights, w_bytes, c, workspace);
        return run_gemm<FormatQ80>(ctx, m, n, k, a_bf16, weights, w_bytes, c, workspace);
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
