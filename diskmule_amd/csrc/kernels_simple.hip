// kernels_simple.hip -- exact per-element kernels for gfx950.
//
// These kernels reproduce the reference arithmetic element by element:
//  * dequantize_kernel: bit-exact cpu::dequantize (src/cpu.rs:546-645);
//  * gemv_exact_kernel: any supported type and any column count; each weight
//    is dequantized exactly and folded with fma (one wave per row).  It
//    serves shapes the MFMA kernels do not take (unaligned rows, columns
//    that are not whole 256-blocks, F32/F16/BF16 rows);
//  * reductions for argmax / top-k / RMSNorm, SiLU products, the exact bf16
//    router fold and the ordered expert combine.
#include "dm_device.h"

#include <utility>
#include "dm_kernels.h"

namespace dm {

// Exact value of element t (0 <= t < block elements) of one encoded block.
// Operation order and rounding follow src/cpu.rs:576-645; compiled without
// contraction, so each product and difference rounds separately.
__device__ __forceinline__ float dequant_element(uint32_t type, const uint8_t *block, uint32_t t) {
    switch (type) {
    case kF32:
        return __uint_as_float((uint32_t)block[0] | ((uint32_t)block[1] << 8) |
                               ((uint32_t)block[2] << 16) | ((uint32_t)block[3] << 24));
    case kF16:
        return f16_bits_to_f32((uint32_t)block[0] | ((uint32_t)block[1] << 8));
    case kBF16:
        return __uint_as_float(((uint32_t)block[0] | ((uint32_t)block[1] << 8)) << 16);
    case kQ8_0: {
        float delta = f16_bits_to_f32((uint32_t)block[0] | ((uint32_t)block[1] << 8));
        return delta * (float)(int8_t)block[2 + t];
    }
    case kQ5_0: {
        // src/cpu.rs:560-574
        float delta = f16_bits_to_f32((uint32_t)block[0] | ((uint32_t)block[1] << 8));
        uint32_t high_bits = (uint32_t)block[2] | ((uint32_t)block[3] << 8) |
                             ((uint32_t)block[4] << 16) | ((uint32_t)block[5] << 24);
        uint32_t index = t & 15u;
        uint32_t packed = block[6 + index];
        int32_t q;
        if (t < 16)
            q = (int32_t)((packed & 0x0fu) | (((high_bits >> index) << 4) & 0x10u)) - 16;
        else
            q = (int32_t)((packed >> 4) | ((high_bits >> (index + 12)) & 0x10u)) - 16;
        return delta * (float)q;
    }
    case kQ4_K: {
        float delta = f16_bits_to_f32((uint32_t)block[0] | ((uint32_t)block[1] << 8));
        float minimum = f16_bits_to_f32((uint32_t)block[2] | ((uint32_t)block[3] << 8));
        uint32_t group_pair = t >> 6, within = t & 63u, high = within >> 5, i = within & 31u;
        uint32_t packed = block[16 + 32 * group_pair + i];
        uint32_t sc, m;
        scale_min_q4_k((int)(2 * group_pair + high), block + 4, sc, m);
        uint32_t q = high ? (packed >> 4) : (packed & 0x0fu);
        return delta * (float)sc * (float)q - minimum * (float)m;
    }
    case kQ6_K: {
        float delta = f16_bits_to_f32((uint32_t)block[208] | ((uint32_t)block[209] << 8));
        uint32_t half = t >> 7, r = t & 127u, k = r >> 5, i = r & 31u;
        const uint8_t *low = block + 64 * half;
        const uint8_t *high = block + 128 + 32 * half;
        const int8_t *scales = (const int8_t *)(block + 192 + 8 * half);
        uint32_t scale_pair = i >> 4;
        uint32_t lo = (k & 1u) ? low[i + 32] : low[i];
        uint32_t nib = (k & 2u) ? (lo >> 4) : (lo & 0x0fu);
        uint32_t q = nib | (((high[i] >> (2 * k)) & 3u) << 4);
        return delta * (float)scales[scale_pair + 2 * k] * ((float)q - 32.0f);
    }
    default:
        return 0.0f;
    }
}

__global__ void dequantize_kernel(uint32_t type, const uint8_t *__restrict__ encoded,
                                  uint32_t block_elements, uint32_t block_bytes, size_t elements,
                                  float *__restrict__ out) {
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < elements; e += stride) {
        size_t b = e / block_elements;
        uint32_t t = (uint32_t)(e - b * block_elements);
        out[e] = dequant_element(type, encoded + b * block_bytes, t);
    }
}

// One wave per (row); lanes stride over columns, each weight dequantized
// exactly, fma into per-lane sums, then a wave sum.  256 threads = 4 rows.
__global__ void __launch_bounds__(256) gemv_exact_kernel(
    uint32_t type, uint32_t block_elements, uint32_t block_bytes, uint32_t rows,
    uint32_t columns, size_t row_bytes, const uint8_t *__restrict__ weights, uint32_t batch,
    const float *__restrict__ x, float *__restrict__ y) {
    uint32_t lane = threadIdx.x & 63u;
    uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint8_t *w = weights + (size_t)row * row_bytes;
    for (uint32_t b = 0; b < batch; b++) {
        const float *xb = x + (size_t)b * columns;
        float acc = 0.0f;
        for (uint32_t c = lane; c < columns; c += 64) {
            uint32_t blk = c / block_elements;
            float v = dequant_element(type, w + (size_t)blk * block_bytes, c - blk * block_elements);
            acc = __builtin_fmaf(v, xb[c], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) y[(size_t)b * rows + row] = acc;
    }
}

// ---- argmax over a device vector (src/cpu.rs:275-293) -------------------
__global__ void argmax_init_kernel(ArgmaxState *state) {
    state->key = 0;
    state->non_finite = 0;
    state->done = 0;
}

__global__ void __launch_bounds__(256) argmax_kernel(const float *__restrict__ v, size_t n,
                                                     ArgmaxState *state) {
    uint64_t best = 0;
    uint32_t bad = 0;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        float value = v[i];
        if (!__builtin_isfinite(value)) bad = 1;
        uint64_t key = argmax_key(value, (uint32_t)i);
        best = key > best ? key : best;
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63u) == 0) {
        atomicMax((unsigned long long *)&state->key, (unsigned long long)best);
    }
    if (bad) atomicOr(&state->non_finite, 1u);
}

__global__ void argmax_finish_kernel(const ArgmaxState *state, uint32_t *index) {
    *index = argmax_key_index(state->key);
}

// ---- top-k softmax (src/cpu.rs:232-260) -------------------------------
// One workgroup per row of `count` logits.  Selection i is the largest key
// strictly below selection i-1 (keys are unique: value, then index).  A
// non-finite logit stores non_finite.mark into *non_finite.word; the return
// value (the same in every thread) says whether the row held one.
__device__ bool block_top_k(const float *logits, uint32_t count, uint32_t k, uint32_t *ids,
                            float *probabilities, BadFlag non_finite) {
    __shared__ uint64_t partial[16];
    __shared__ uint64_t chosen[kMaxTopK];
    __shared__ float values[kMaxTopK];
    uint32_t tid = threadIdx.x, nthreads = blockDim.x;
    uint32_t bad = 0;
    for (size_t i = tid; i < count; i += nthreads)
        if (!__builtin_isfinite(logits[i])) bad = 1;
    if (bad) *non_finite.word = non_finite.mark;  // every writer stores the same value
    const bool row_bad = __syncthreads_or((int)bad) != 0;
    uint64_t previous = ~0ull;
    for (uint32_t s = 0; s < k; s++) {
        uint64_t best = 0;
        for (size_t i = tid; i < count; i += nthreads) {
            uint64_t key = argmax_key(logits[i], (uint32_t)i);
            if (key < previous && key > best) best = key;
        }
        best = wave_max_u64(best);
        if ((tid & 63u) == 0) partial[tid >> 6] = best;
        __syncthreads();
        if (tid == 0) {
            uint64_t b = partial[0];
            for (uint32_t w = 1; w < (nthreads + 63) / 64; w++) b = partial[w] > b ? partial[w] : b;
            chosen[s] = b;
        }
        __syncthreads();
        previous = chosen[s];
    }
    if (tid == 0) {
        // softmax_in_place over the selected logits (src/cpu.rs:195-230):
        // maximum, exp(v - max), sequential sum, divide.
        float maximum = -__builtin_inff();
        for (uint32_t s = 0; s < k; s++) {
            uint32_t index = argmax_key_index(chosen[s]);
            ids[s] = index;
            values[s] = logits[index];
            maximum = fmaxf(maximum, values[s]);
        }
        float sum = 0.0f;
        for (uint32_t s = 0; s < k; s++) {
            values[s] = expf(values[s] - maximum);
            sum += values[s];
        }
        for (uint32_t s = 0; s < k; s++) probabilities[s] = values[s] / sum;
    }
    return row_bad;
}

__global__ void __launch_bounds__(256) top_k_kernel(const float *__restrict__ logits,
                                                    uint32_t count, uint32_t k, uint32_t *ids,
                                                    float *probabilities, BadFlag non_finite) {
    uint32_t row = blockIdx.x;
    block_top_k(logits + (size_t)row * count, count, k, ids + (size_t)row * k,
                probabilities + (size_t)row * k, non_finite);
}

// Exact bf16 router + top-k, one workgroup per token.  Thread r folds row r
// sequentially from column 0 with fma (src/cpu.rs:391-394 order), so the
// logits equal the CPU's bit for bit and the selected ids cannot differ.
__global__ void __launch_bounds__(256) router_top_k_kernel(
    const uint16_t *__restrict__ router, uint32_t hidden, uint32_t experts, uint32_t k,
    const float *__restrict__ x, float *__restrict__ logits, uint32_t *ids,
    float *probabilities, BadFlag non_finite) {
    uint32_t token = blockIdx.x;
    extern __shared__ float s_logits[];
    const float *xt = x + (size_t)token * hidden;
    float *lt = logits + (size_t)token * experts;
    for (uint32_t r = threadIdx.x; r < experts; r += blockDim.x) {
        const uint16_t *w = router + (size_t)r * hidden;
        float sum = 0.0f;
        uint32_t c = 0;
        if ((((uintptr_t)w) & 15u) == 0) {
            for (; c + 8 <= hidden; c += 8) {
                u32x4 pk = *(const u32x4 *)(w + c);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    sum = __builtin_fmaf(__uint_as_float(pk[j] << 16), xt[c + 2 * j], sum);
                    sum = __builtin_fmaf(__uint_as_float(pk[j] & 0xffff0000u), xt[c + 2 * j + 1], sum);
                }
            }
        }
        for (; c < hidden; c++) sum = __builtin_fmaf(__uint_as_float((uint32_t)w[c] << 16), xt[c], sum);
        lt[r] = sum;
        s_logits[r] = sum;
    }
    __syncthreads();
    block_top_k(s_logits, experts, k, ids + (size_t)token * k, probabilities + (size_t)token * k,
                non_finite);
}

// The same router with the rows staged through LDS (at most 256 experts,
// hidden % 8 == 0, 16-byte aligned router and x).  Lane r still folds row r
// sequentially from column 0, so the logits are those of the kernel above;
// what changes is the memory path.  The columns go in chunks of CC: every
// thread loads 16-byte pieces of the chunk (rows of the workgroup's experts,
// then the chunk's x values) into registers and stores them to one of two
// LDS slots; three chunks are in flight while one is folded.  A
// row occupies CC * 2 + 16 bytes of its slot, so the 16-byte reads of
// consecutive lanes fall in distinct banks.  With host_ids/host_probs the
// selection is also written to (pinned) host memory.
typedef uint32_t v4a __attribute__((ext_vector_type(4)));  // 16-byte aligned

template <uint32_t CC>
__global__ void __launch_bounds__(256) router_staged_kernel(
    const uint16_t *__restrict__ router, uint32_t hidden, uint32_t experts, uint32_t k,
    const float *__restrict__ x, float *__restrict__ logits, uint32_t *ids, float *probabilities,
    BadFlag non_finite, uint32_t *host_ids, float *host_probs, uint32_t *host_bad) {
    constexpr uint32_t ROW = CC * 2 + 16;  // LDS bytes per expert row
    constexpr uint32_t PR = CC * 2 / 16;   // 16-byte pieces of a row per chunk
    constexpr uint32_t XP = CC * 4 / 16;   // 16-byte pieces of x per chunk
    constexpr uint32_t NP = 8;             // pieces per thread: rows of up to 2048 / PR experts
    extern __shared__ v4a r_stage[];
    __shared__ float s_logits[256];
    const uint32_t token = blockIdx.x, tid = threadIdx.x;
    const uint32_t E = experts;
    const uint32_t slot_bytes = (E * ROW + CC * 4 + 15) & ~15u;
    const uint32_t chunks = (hidden + CC - 1) / CC;
    const float *xt = x + (size_t)token * hidden;

    // Buffer loads: a piece past the router or past x reads zeros, so every
    // thread issues the same loads for every chunk (no branches around them,
    // which lets the compiler wait for one register set while the next two
    // stay in flight).  Pieces of rows >= E start at `nowhere`.
    constexpr uint32_t nowhere = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(router, E * hidden * 2);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xt, hidden * 4);
    uint32_t woff[NP];
#pragma unroll
    for (uint32_t j = 0; j < NP; j++) {
        const uint32_t item = j * 256 + tid, row = item / PR, p = item % PR;
        woff[j] = row < E ? row * hidden * 2 + 16 * p : nowhere;
    }
    const uint32_t xoff = 16 * (tid % XP);
    auto load = [&](v4a (&wr)[NP], v4a &xr, uint32_t chunk) {
        const uint32_t c0 = chunk * CC;
#pragma unroll
        for (uint32_t j = 0; j < NP; j++)
            wr[j] = __builtin_bit_cast(v4a, rsrc_load16(rw, woff[j] + 2 * c0));
        xr = __builtin_bit_cast(v4a, rsrc_load16(rx, xoff + 4 * c0));
    };
    auto store = [&](const v4a (&wr)[NP], const v4a &xr, uint32_t slot) {
        uint8_t *s = (uint8_t *)r_stage + slot * slot_bytes;
#pragma unroll
        for (uint32_t j = 0; j < NP; j++) {
            const uint32_t item = j * 256 + tid, row = item / PR, p = item % PR;
            if (row < E) *(v4a *)(s + row * ROW + 16 * p) = wr[j];
        }
        if (tid < XP) *(v4a *)(s + E * ROW + 16 * tid) = xr;
    };

    float acc = 0.0f;
    auto fold = [&](uint32_t slot, uint32_t chunk) {
        const uint8_t *s = (const uint8_t *)r_stage + slot * slot_bytes;
        const v4a *wrow = (const v4a *)(s + tid * ROW);
        const float *xs = (const float *)(s + E * ROW);
        const uint32_t n = hidden - chunk * CC < CC ? hidden - chunk * CC : CC;
        if (n == CC) {
            // The whole chunk of the row and of x first (one LDS wait per
            // chunk), then the dependent chain of CC fmas.
            v4a wv[PR], xv[2 * PR];
#pragma unroll
            for (uint32_t q = 0; q < PR; q++) wv[q] = wrow[q];
#pragma unroll
            for (uint32_t q = 0; q < 2 * PR; q++) xv[q] = *(const v4a *)(xs + 4 * q);
#pragma unroll
            for (uint32_t q = 0; q < PR; q++) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const v4a xq = xv[2 * q + (j >> 1)];
                    const float xa = __uint_as_float(xq[2 * (j & 1)]);
                    const float xb = __uint_as_float(xq[2 * (j & 1) + 1]);
                    acc = __builtin_fmaf(__uint_as_float(wv[q][j] << 16), xa, acc);
                    acc = __builtin_fmaf(__uint_as_float(wv[q][j] & 0xffff0000u), xb, acc);
                }
            }
        } else {
            const uint16_t *wh = (const uint16_t *)wrow;
            for (uint32_t c = 0; c < n; c++) acc = __builtin_fmaf(__uint_as_float((uint32_t)wh[c] << 16), xs[c], acc);
        }
    };

    // Three register sets rotate: while chunk c is folded from LDS slot c % 2,
    // chunks c + 1 .. c + 3 are in flight.  After the fold, chunk c + 1 goes
    // to the other slot (last read by the fold of chunk c - 1, before the
    // previous barrier) and its registers take chunk c + 4.
    v4a ra[NP], rb[NP], rc[NP], xa, xb, xc;
    load(ra, xa, 0);
    load(rb, xb, 1);
    load(rc, xc, 2);
    store(ra, xa, 0);
    __syncthreads();
    load(ra, xa, 3);
    auto step = [&](uint32_t c, v4a (&wr)[NP], v4a &xr) {
        if (c < chunks && tid < E) fold(c & 1u, c);
        store(wr, xr, (c + 1) & 1u);
        __syncthreads();
        load(wr, xr, c + 4);
    };
    for (uint32_t i = 0; i < chunks; i += 3) {
        step(i, rb, xb);
        step(i + 1, rc, xc);
        step(i + 2, ra, xa);
    }
    if (tid < E) {
        logits[(size_t)token * E + tid] = acc;
        s_logits[tid] = acc;
    }
    __syncthreads();
    uint32_t *ti = ids + (size_t)token * k;
    float *tp = probabilities + (size_t)token * k;
    const bool bad = block_top_k(s_logits, E, k, ti, tp, non_finite);
    if (host_ids && tid == 0) {
        for (uint32_t s = 0; s < k; s++) {
            host_ids[(size_t)token * k + s] = ti[s];
            host_probs[(size_t)token * k + s] = tp[s];
        }
        host_bad[token] = bad;
    }
}

// The selected experts' slots (MoE layer call): thread 0 of the token's
// last workgroup looks each id up and publishes the addresses and the
// token's go word (ExpertLookup).
__device__ void expert_lookup(const ExpertLookup &L, const uint32_t *ids, uint32_t k, uint32_t token, bool bad) {
    uint32_t go = bad ? 0u : 1u;
    for (uint32_t s = 0; s < k; s++) {
        const uint64_t gu = L.gate_up_of[ids[s]], dn = L.down_of[ids[s]];
        if (gu == 0 || dn == 0) go = 0;
        L.gate_up_w[(size_t)token * k + s] = gu;
        L.down_w[(size_t)token * k + s] = dn;
    }
    L.go[token] = go;
    L.host_go[token] = go;
}

// Expert-parallel form of the exact router for decode: workgroup (g, t) is
// one wave that folds the RF_EXPERTS rows g * RF_EXPERTS .. of token t.
// Lane e < RF_EXPERTS still folds its row sequentially from column 0 with
// fma, so the logits are bit-identical to the kernels above; what changes is
// that the router's rows stream through E / RF_EXPERTS compute units per
// token instead of one, and the dependent fma chain reads fp32 operands from
// LDS (two 16-byte reads per four fmas, no unpacking on the chain).  Columns
// go in chunks of RF_CHUNK through two LDS buffers: every lane loads 16-byte
// pieces of the next chunk's rows and x while the chain runs, then widens
// the bf16 pieces to fp32 into the other buffer.
constexpr uint32_t RF_EXPERTS = 8, RF_CHUNK = 512;
constexpr uint32_t RF_ROW = RF_CHUNK + 4;                        // floats per staged row (bank skew)
constexpr uint32_t RF_BUF = RF_EXPERTS * RF_ROW + RF_CHUNK;      // floats per buffer: rows, then x
constexpr uint32_t RF_WPIECES = RF_EXPERTS * RF_CHUNK * 2 / 16;  // 16-byte bf16 pieces of the rows
constexpr uint32_t RF_XPIECES = RF_CHUNK * 4 / 16;               // 16-byte pieces of x
constexpr uint32_t RF_LOADS = (RF_WPIECES + RF_XPIECES) / 64;    // per lane and chunk
static_assert((RF_WPIECES + RF_XPIECES) % 64 == 0, "whole loads per lane");

__global__ void __launch_bounds__(64) router_fold_kernel(const uint16_t *__restrict__ router, uint32_t hidden,
                                                         uint32_t experts, uint32_t k, const float *__restrict__ x,
                                                         float *logits, uint32_t *tickets, uint32_t *ids,
                                                         float *probabilities, BadFlag non_finite,
                                                         uint32_t *host_ids, float *host_probs, uint32_t *host_bad,
                                                         ExpertLookup lookup) {
    __shared__ v4a rf_lds[2 * RF_BUF / 4];
    const uint32_t lane = threadIdx.x, e0 = blockIdx.x * RF_EXPERTS, token = blockIdx.y;
    const uint32_t chunks = (hidden + RF_CHUNK - 1) / RF_CHUNK;
    // Piece j of a chunk: row piece (row j / 64, column 8 (j % 64)) for
    // j < RF_WPIECES, else x piece j - RF_WPIECES.  Rows past `experts`
    // and columns past `hidden` read zeros (buffer loads past the end).
    constexpr uint32_t nowhere = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(router, experts * hidden * 2);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (size_t)token * hidden, hidden * 4);
    uint32_t off[RF_LOADS];
#pragma unroll
    for (uint32_t i = 0; i < RF_LOADS; i++) {
        const uint32_t j = i * 64 + lane;
        if (j < RF_WPIECES) {
            const uint32_t row = e0 + j / (RF_CHUNK / 8);
            off[i] = row < experts ? row * hidden * 2 + 16 * (j % (RF_CHUNK / 8)) : nowhere;
        } else {
            off[i] = 16 * (j - RF_WPIECES);
        }
    }
    v4a r[RF_LOADS];
    auto load = [&](uint32_t c) {
        const uint32_t c0 = c * RF_CHUNK;
#pragma unroll
        for (uint32_t i = 0; i < RF_LOADS; i++) {
            const uint32_t j = i * 64 + lane;
            // the last chunk of a row may run past `hidden`: those columns are
            // never folded, so whatever they read is harmless
            if (j < RF_WPIECES)
                r[i] = __builtin_bit_cast(v4a, rsrc_load16(rw, off[i] == nowhere ? nowhere : off[i] + 2 * c0));
            else
                r[i] = __builtin_bit_cast(v4a, rsrc_load16(rx, off[i] + 4 * c0));
        }
    };
    auto store = [&](uint32_t b) {
        float *buf = (float *)rf_lds + b * RF_BUF;
#pragma unroll
        for (uint32_t i = 0; i < RF_LOADS; i++) {
            const uint32_t j = i * 64 + lane;
            if (j < RF_WPIECES) {
                float *dst = buf + (j / (RF_CHUNK / 8)) * RF_ROW + 8 * (j % (RF_CHUNK / 8));
                v4a lo, hi;
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    lo[2 * q] = r[i][q] << 16;
                    lo[2 * q + 1] = r[i][q] & 0xffff0000u;
                    hi[2 * q] = r[i][q + 2] << 16;
                    hi[2 * q + 1] = r[i][q + 2] & 0xffff0000u;
                }
                *(v4a *)dst = lo;
                *(v4a *)(dst + 4) = hi;
            } else {
                *(v4a *)(buf + RF_EXPERTS * RF_ROW + 4 * (j - RF_WPIECES)) = r[i];
            }
        }
    };
    float acc = 0.0f;
    const uint32_t my = lane < RF_EXPERTS ? lane : 0;
    load(0);
    store(0);
    for (uint32_t c = 0; c < chunks; c++) {
        if (c + 1 < chunks) load(c + 1);
        // One wave: its LDS operations run in order; the fences keep the
        // compiler from moving other lanes' reads across the stores.
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        const float *buf = (const float *)rf_lds + (c & 1u) * RF_BUF;
        const float *wr = buf + my * RF_ROW, *xr = buf + RF_EXPERTS * RF_ROW;
        const uint32_t n = hidden - c * RF_CHUNK < RF_CHUNK ? hidden - c * RF_CHUNK : RF_CHUNK;
        if (lane < RF_EXPERTS) {
            if (n == RF_CHUNK) {
#pragma unroll 8
                for (uint32_t q = 0; q < RF_CHUNK; q += 4) {
                    const v4a wv = *(const v4a *)(wr + q), xv = *(const v4a *)(xr + q);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc = __builtin_fmaf(__uint_as_float(wv[i]), __uint_as_float(xv[i]), acc);
                }
            } else {
                for (uint32_t q = 0; q < n; q++) acc = __builtin_fmaf(wr[q], xr[q], acc);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        if (c + 1 < chunks) store((c + 1) & 1u);
    }
    if (!tickets) {
        if (lane < RF_EXPERTS && e0 + lane < experts) logits[(size_t)token * experts + e0 + lane] = acc;
        return;
    }
    // Fused selection: publish the logits with device-scope exchanges, wait
    // for them to complete, then take the token's ticket; the workgroup that
    // draws the last one reads every logit of the token back and selects.
    float old = 0.0f;
    if (lane < RF_EXPERTS && e0 + lane < experts)
        old = __hip_atomic_exchange(&logits[(size_t)token * experts + e0 + lane], acc, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::"v"(old) : "memory");
    uint32_t drawn = 0;
    if (lane == 0) drawn = atomicAdd(&tickets[token], 1u);
    if (__builtin_amdgcn_readfirstlane(drawn) != gridDim.x - 1) return;
    __shared__ float s_row[256];
    for (uint32_t i = lane; i < experts; i += 64)
        s_row[i] = __hip_atomic_load(&logits[(size_t)token * experts + i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    uint32_t *ti = ids + (size_t)token * k;
    float *tp = probabilities + (size_t)token * k;
    const bool bad = block_top_k(s_row, experts, k, ti, tp, non_finite);
    if (lane == 0) {
        if (host_ids) {
            for (uint32_t s = 0; s < k; s++) {
                host_ids[(size_t)token * k + s] = ti[s];
                host_probs[(size_t)token * k + s] = tp[s];
            }
            host_bad[token] = bad;
        }
        if (lookup.go) expert_lookup(lookup, ti, k, token, bad);
        __hip_atomic_store(&tickets[token], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Rank of a key among keys[0 .. n): the count of larger keys.  The loop
// reads 16 keys at a time, so their LDS reads overlap.
__device__ __forceinline__ uint32_t key_rank(const uint64_t *keys, uint32_t n, uint64_t mine) {
    uint32_t rank = 0, j = 0;
    for (; j + 16 <= n; j += 16) {
        uint64_t w[16];
#pragma unroll
        for (uint32_t q = 0; q < 16; q++) w[q] = keys[j + q];
#pragma unroll
        for (uint32_t q = 0; q < 16; q++) rank += w[q] > mine ? 1u : 0u;
    }
    for (; j < n; j++) rank += keys[j] > mine ? 1u : 0u;
    return rank;
}

// Exact router for decode with the rows staged in LDS as f32.  Workgroup
// (g, t) of four waves first loads router rows R g .. R g + R - 1 and token
// t's x with up to 16 loads per thread in flight at once (contiguous 16-byte
// pieces), widens the bf16 values (bits << 16, exact) and stores them in LDS,
// so the rows cost one or two memory round trips.  R is the most rows that
// fit in LDS beside x (16 at hidden 2048).  Rows and x are zero-padded to
// whole rings of steps: the padding adds fma(0, 0, acc) = acc (the sum starts
// at +0 and an exactly zero sum of +0 and -0 is +0, so it is never -0).
// Lane e < R of wave 0 then folds row R g + e sequentially from column 0
// with fma (the reference's fold: logits and ids are bit-identical to the
// kernels above).  Each step of 8 columns takes the row's values and x's from
// two 16-byte LDS reads each (x: one address for all lanes), kRlAhead steps
// ahead, so the wave issues nothing but the chain's fmas and the reads.  The
// loop body is one ring of steps: ring slots keep fixed registers, every
// wait names the read it needs, and the code stays small (an unrolled chain
// is tens of KB run once per launch, more than instruction fetch keeps up
// with).  Rows are padded by 16 bytes in LDS, so the lanes' reads of one step
// start 4 banks apart.  The token's last workgroup (ticket) makes the
// selection by rank: each of up to 256 logits counts the keys above its own.
constexpr uint32_t kRlRing = 4;   // ring slots: steps of 8 columns per loop iteration
constexpr uint32_t kRlAhead = 3;  // steps read ahead of their use (4 LDS reads each, lgkmcnt <= 15)

struct LdsChainState {
    v4a wring[2 * kRlRing];  // the row's 8 values of a step, f32
    v4a xring[2 * kRlRing];  // x's 8 values of a step
    float acc;
    const v4a *wrow;  // this lane's row in LDS
    const v4a *xs;    // x in LDS
};

template <uint32_t C>
__device__ __forceinline__ void lds_chain_read(LdsChainState &st, uint32_t step) {
    st.wring[2 * C] = st.wrow[2 * step];
    st.wring[2 * C + 1] = st.wrow[2 * step + 1];
    st.xring[2 * C] = st.xs[2 * step];
    st.xring[2 * C + 1] = st.xs[2 * step + 1];
}

// Step base + C of a ring of steps: fold 8 columns, then (C < NREAD) read the
// operands of step base + C + kRlAhead into their slot.
template <uint32_t C, uint32_t NREAD>
__device__ __forceinline__ void lds_chain_step(LdsChainState &st, uint32_t base) {
    const v4a wa = st.wring[2 * C], wb = st.wring[2 * C + 1];
    const v4a xa = st.xring[2 * C], xb = st.xring[2 * C + 1];
#pragma unroll
    for (int i = 0; i < 4; i++) st.acc = __builtin_fmaf(__uint_as_float(wa[i]), __uint_as_float(xa[i]), st.acc);
#pragma unroll
    for (int i = 0; i < 4; i++) st.acc = __builtin_fmaf(__uint_as_float(wb[i]), __uint_as_float(xb[i]), st.acc);
    if constexpr (C < NREAD) lds_chain_read<(C + kRlAhead) % kRlRing>(st, base + C + kRlAhead);
    __builtin_amdgcn_sched_barrier(0);
}

template <uint32_t NREAD, uint32_t... C>
__device__ __forceinline__ void lds_chain_ring(LdsChainState &st, uint32_t base,
                                               std::integer_sequence<uint32_t, C...>) {
    (lds_chain_step<C, NREAD>(st, base), ...);
}

// Steps of 8 columns, padded to whole rings, and the LDS layout of a row:
// f32 pieces of 16 bytes plus one padding piece.
__host__ __device__ constexpr uint32_t router_lds_steps(uint32_t hidden) {
    return (hidden / 8 + kRlRing - 1) / kRlRing * kRlRing;
}
__host__ __device__ constexpr uint32_t router_lds_row_pieces(uint32_t hidden) {
    return 2 * router_lds_steps(hidden) + 1;
}
constexpr size_t router_lds_bytes(uint32_t hidden, uint32_t rows) {
    return ((size_t)rows * router_lds_row_pieces(hidden) + 2 * router_lds_steps(hidden)) * 16;
}

__global__ void __launch_bounds__(256) router_lds_kernel(const uint16_t *__restrict__ router, uint32_t hidden,
                                                         uint32_t experts, uint32_t R, uint32_t k,
                                                         const float *__restrict__ x, float *logits,
                                                         uint32_t *tickets, uint32_t *ids, float *probabilities,
                                                         BadFlag non_finite, uint32_t *host_ids, float *host_probs,
                                                         uint32_t *host_bad, ExpertLookup lookup) {
    constexpr uint32_t kBatch = 16;   // row loads per thread in flight
    constexpr uint32_t kXPieces = 8;  // x loads per thread: hidden <= 8192
    const uint32_t N8 = hidden / 8, NS = router_lds_steps(hidden), RS = router_lds_row_pieces(hidden);
    extern __shared__ __attribute__((aligned(16))) v4a lds_rows[];  // [R][RS], then x [2 NS]
    v4a *xs = lds_rows + R * RS;
    const uint32_t tid = threadIdx.x, e0 = blockIdx.x * R, token = blockIdx.y;
    constexpr uint32_t nowhere = 0x80000000u;  // every load from here reads zeros
    // rows past `experts` and columns past `hidden` read zeros (buffer loads
    // past the end, or nowhere)
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(router, experts * hidden * 2);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (size_t)token * hidden, hidden * 4);
    // x: 2 NS <= 2048 pieces of 4 floats (hidden % 8 == 0, so whole
    // pieces), requested together with the first batch of rows
    v4a xr[kXPieces];
#pragma unroll
    for (uint32_t j = 0; j < kXPieces; j++) {
        const uint32_t piece = j * 256 + tid;
        xr[j] = __builtin_bit_cast(v4a, rsrc_load16(rx, piece < 2 * N8 ? 16 * piece : nowhere));
    }
    // rows: R NS bf16 pieces of 8 values, kBatch per thread at a time; piece
    // p is (row p / NS, step p % NS), the quotient by a multiply-high (exact
    // for p NS < 2^32)
    const uint32_t total = R * NS, inv = (uint32_t)((0xffffffffull + NS) / NS);
    for (uint32_t p0 = 0; p0 < total; p0 += 256 * kBatch) {
        v4a wr[kBatch];
#pragma unroll
        for (uint32_t j = 0; j < kBatch; j++) {
            const uint32_t p = p0 + j * 256 + tid, row = __umulhi(p, inv), col = p - row * NS;
            const bool real = p < total && col < N8 && e0 + row < experts;
            wr[j] = __builtin_bit_cast(v4a, rsrc_load16(rw, real ? ((e0 + row) * N8 + col) * 16 : nowhere));
        }
        if (p0 == 0) {
#pragma unroll
            for (uint32_t j = 0; j < kXPieces; j++)
                if (j * 256 + tid < 2 * NS) xs[j * 256 + tid] = xr[j];
        }
#pragma unroll
        for (uint32_t j = 0; j < kBatch; j++) {
            const uint32_t p = p0 + j * 256 + tid, row = __umulhi(p, inv), col = p - row * NS;
            if (p < total) {
                const v4a w = wr[j];
                lds_rows[row * RS + 2 * col] = v4a{w[0] << 16, w[0] & 0xffff0000u, w[1] << 16, w[1] & 0xffff0000u};
                lds_rows[row * RS + 2 * col + 1] =
                    v4a{w[2] << 16, w[2] & 0xffff0000u, w[3] << 16, w[3] & 0xffff0000u};
            }
        }
    }
    __syncthreads();
    __shared__ uint32_t s_drawn;
    if (tid < 64) {
        const uint32_t lane = tid, e = e0 + lane;
        LdsChainState st;
        st.wrow = lds_rows + (lane % R) * RS;
        st.xs = xs;
        lds_chain_read<0>(st, 0);
        lds_chain_read<1>(st, 1);
        lds_chain_read<2>(st, 2);
        static_assert(kRlAhead == 3, "the prologue reads kRlAhead steps");
        st.acc = 0.0f;
        constexpr auto ring = std::make_integer_sequence<uint32_t, kRlRing>{};
        uint32_t base = 0;
#pragma unroll 1
        for (; base + kRlRing < NS; base += kRlRing) lds_chain_ring<kRlRing>(st, base, ring);
        lds_chain_ring<kRlRing - kRlAhead>(st, base, ring);
        const float acc = st.acc;
        const bool mine = lane < R && e < experts;
        if (!tickets) {
            if (mine) logits[(size_t)token * experts + e] = acc;
        } else {
            float old = 0.0f;
            if (mine)
                old = __hip_atomic_exchange(&logits[(size_t)token * experts + e], acc, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("" ::"v"(old) : "memory");
            uint32_t drawn = 0;
            if (lane == 0) drawn = atomicAdd(&tickets[token], 1u);
            if (lane == 0) s_drawn = drawn;
        }
    }
    if (!tickets) return;
    __syncthreads();
    if (s_drawn != gridDim.x - 1) return;
    // The token's last workgroup: the selection over every logit, by rank.
    __shared__ uint64_t s_keys[256];
    __shared__ uint32_t s_sel[256];
    __shared__ float s_logit[256], s_value[256];
    uint64_t mine = 0;
    bool bad = false;
    if (tid < experts) {
        const float v =
            __hip_atomic_load(&logits[(size_t)token * experts + tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bad = !__builtin_isfinite(v);
        mine = argmax_key(v, tid);
        s_keys[tid] = mine;
        s_logit[tid] = v;
    }
    if (bad) *non_finite.word = non_finite.mark;  // every writer stores the same value
    __shared__ float s_sum;
    __shared__ uint32_t s_missing;
    if (tid == 0) s_missing = 0;
    const bool row_bad = __syncthreads_or((int)bad) != 0;
    {
        // keys are unique (value, then index), so ranks are 0 .. experts - 1;
        // up to 128 experts two threads count a key's rank over half the keys
        __shared__ uint32_t s_rank[256];
        const uint32_t split = experts <= 128 ? 2u : 1u, span = (experts + split - 1) / split;
        const uint32_t me = split == 2 ? tid & 127u : tid, begin = split == 2 ? (tid >> 7) * span : 0u;
        s_rank[tid] = me < experts ? key_rank(s_keys + begin, span < experts - begin ? span : experts - begin,
                                              s_keys[me])
                                   : 0u;
        __syncthreads();
        const uint32_t rank = tid < experts ? s_rank[tid] + (split == 2 ? s_rank[tid + 128] : 0u) : experts;
        if (rank < k) s_sel[rank] = tid;
    }
    __syncthreads();
    // softmax_in_place over the selected logits (src/cpu.rs:195-230):
    // maximum, exp(v - max), sequential sum, divide; selection s by thread s
    // (k <= experts <= 256), the sum in selection order by thread 0.
    uint32_t *ti = ids + (size_t)token * k;
    float *tp = probabilities + (size_t)token * k;
    if (tid < k) {
        const uint32_t index = s_sel[tid];
        float maximum = -__builtin_inff();
        for (uint32_t j = 0; j < k; j++) maximum = fmaxf(maximum, s_logit[s_sel[j]]);
        s_value[tid] = expf(s_logit[index] - maximum);
        ti[tid] = index;
        if (host_ids) host_ids[(size_t)token * k + tid] = index;
        if (lookup.go) {
            // the selected expert's slot (ExpertLookup)
            const uint64_t gu = lookup.gate_up_of[index], dn = lookup.down_of[index];
            lookup.gate_up_w[(size_t)token * k + tid] = gu;
            lookup.down_w[(size_t)token * k + tid] = dn;
            if (gu == 0 || dn == 0) s_missing = 1;  // every writer stores the same value
        }
    }
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (uint32_t j = 0; j < k; j++) sum += s_value[j];
        s_sum = sum;
    }
    __syncthreads();
    if (tid < k) {
        const float p = s_value[tid] / s_sum;
        tp[tid] = p;
        if (host_ids) host_probs[(size_t)token * k + tid] = p;
    }
    if (tid == 0) {
        if (host_ids) host_bad[token] = row_bad;
        if (lookup.go) {
            const uint32_t go = row_bad || s_missing ? 0u : 1u;
            lookup.go[token] = go;
            lookup.host_go[token] = go;
        }
        __hip_atomic_store(&tickets[token], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Certified router for the MoE layer: the top-k ids (and their order) of
// the reference's sequential fold, from a parallel fold with a proven error
// bound; the exact fold runs only for the experts the bound cannot order.
//
// The reference folds a logit in f32 from +0, one fma per column
// (s^_{i+1} = fma(w_i, x_i, s^_i), src/cpu.rs:391-394 over widened bf16
// rows).  With s_i the exact prefix sums and u = 2^-24 each fma rounds once:
// |fl(r) - r| <= u |r| + 2^-150 (the second term for subnormal results), so
// the error E_i = |s^_i - s_i| obeys E_i <= (1 + u) E_{i-1} + u |s_i| + 2^-150
// and |s^_n - s_n| <= (1 + u)^n (u sum_i |s_i| + n 2^-150), as long as no
// intermediate |s_i| + E_i reaches FLT_MAX (then the fold could overflow).
// This kernel computes, per (token, expert) row, every product w_i x_i
// exactly in double (8 + 24 significant bits), the prefix sums in double
// (lane segments of 32 columns and one wave scan per 2048 columns), the
// total L, A = sum |s_i|, M = max |s_i| and P = sum |w_i x_i|.  Each of these
// double sums takes fewer than 128 roundings of at most 2^-53 P, so
// D = 2^-46 P bounds the distance of every computed prefix sum (and of L)
// from the exact one, and with n <= 8192 ((1 + u)^n < 1.0005):
//   B = 1.001 (u (A + n D) + n 2^-150)     bounds |s^_n - s_n|
//   rho = 1.001 (B + 2 D)                  bounds |s^_n - L|, with room for
//                                          the rounding of L -+ rho
// A row whose M + D + B is not below 3e38, or whose inputs are not finite,
// gets rho = +inf.
//
// Workgroup (g, t) of W waves: wave w takes row W g + w of token t and publishes f32(L)
// and rho (widened by the rounding of L, rounded up to f32) as one word with
// a device-scope exchange, then the workgroup takes the token's ticket.  The
// rounding slack D covers L -+ rho formed in double from those floats.  The
// last workgroup selects:
//  * every rho finite: k candidates, the top k by (f32(L), index).  When
//    the intervals [L - rho, L + rho] of consecutive candidates are disjoint
//    and every other row's interval lies below the k-th one's, the
//    reference selects the same ids in the same order; the probabilities
//    are then the reference's softmax over the f32 roundings of the
//    selected L (within rho of the reference's logits).
//  * otherwise C, the rows that can still be in the top k (every row whose
//    L + rho reaches the smallest L - rho of the k candidates; any row
//    outside C is below those k rows for certain), is ordered exactly: the
//    members whose interval meets another member's (X: typically two rows)
//    are folded exactly, the reference's way (staged in LDS, as
//    router_lds_kernel folds), and compared by their exact logits (value,
//    then index); every other pair of members has disjoint intervals, so L
//    or an exact logit orders it.  The selected members outside X take
//    their f32-rounded L.
//  * a non-finite L (a non-finite input of the row or of x, so a non-finite
//    reference logit) fails the call; a row whose fold may overflow (rho
//    infinite, finite L) makes every row a member of X, so the non-finite
//    check is the reference's.
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ double wave_max_f64(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmax(v, __shfl_xor(v, m, 64));
    return v;
}

template <uint32_t W>
__global__ void __launch_bounds__(64 * W) router_cert_kernel(const uint16_t *__restrict__ router, uint32_t hidden,
                                                          uint32_t experts, uint32_t k, const float *__restrict__ x,
                                                          uint64_t *cert, uint32_t *tickets, uint32_t *ids,
                                                          float *probabilities, BadFlag non_finite,
                                                          uint32_t *host_ids, float *host_probs, uint32_t *host_bad,
                                                          ExpertLookup lookup, uint32_t rf) {
    extern __shared__ __attribute__((aligned(16))) v4a cert_lds[];  // exact folds: rf rows, then x (router_lds_bytes)
    constexpr uint32_t nowhere = 0x80000000u;                      // every load from here reads zeros
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, token = blockIdx.y;
    constexpr uint32_t T = 64 * W;  // threads
    const uint32_t N8 = hidden / 8, e = blockIdx.x * W + wave;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(router, experts * hidden * 2);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (size_t)token * hidden, hidden * 4);
    uint64_t *tc = cert + (size_t)token * experts;
    {
        // lane: pieces (8 columns) pc0 .. pc0 + 3 of each 256-piece round
        double carry = 0.0, a = 0.0, sp = 0.0, m = 0.0;
        for (uint32_t r = 0; r * 256 < N8; r++) {
            const uint32_t pc0 = r * 256 + 4 * lane;
            v4a wv[4], xv[8];
#pragma unroll
            for (uint32_t j = 0; j < 4; j++)
                wv[j] = __builtin_bit_cast(
                    v4a, rsrc_load16(rw, e < experts && pc0 + j < N8 ? (e * N8 + pc0 + j) * 16 : nowhere));
#pragma unroll
            for (uint32_t j = 0; j < 8; j++)
                xv[j] = __builtin_bit_cast(v4a, rsrc_load16(rx, pc0 + j / 2 < N8 ? (2 * pc0 + j) * 16 : nowhere));
            double p[32], t = 0.0;
#pragma unroll
            for (uint32_t c = 0; c < 32; c++) {
                const uint32_t d = wv[c / 8][(c % 8) / 2];
                const float wf = __uint_as_float(c % 2 ? d & 0xffff0000u : d << 16);
                p[c] = (double)wf * (double)__uint_as_float(xv[c / 4][c % 4]);
                t += p[c];
                sp += fabs(p[c]);
            }
            // exclusive scan of the lane totals
            double incl = t;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const double o = __shfl_up(incl, off, 64);
                if (lane >= (uint32_t)off) incl += o;
            }
            double s = __shfl_up(incl, 1, 64);
            s = carry + (lane == 0 ? 0.0 : s);
#pragma unroll
            for (uint32_t c = 0; c < 32; c++) {
                if (pc0 + c / 8 < N8) {
                    s += p[c];
                    a += fabs(s);
                    m = fmax(m, fabs(s));
                }
            }
            carry += __shfl(incl, 63, 64);
        }
        const double A = wave_sum_f64(a), P = wave_sum_f64(sp), M = wave_max_f64(m), n = (double)hidden;
        const double D = P * 0x1p-46;
        const double B = 1.001 * (0x1p-24 * (A + n * D) + n * 0x1p-150);
        double rho = 1.001 * (B + 2.0 * D);
        if (!(M + D + B < 3.0e38)) rho = __builtin_inf();
        // One word per row: f32(L) and an f32 radius rounded up to cover rho
        // and the rounding of L (non-finite stays non-finite).
        const float lf = (float)carry;
        const double rd = rho + fabs(carry - (double)lf);
        float rf = (float)rd;
        if ((double)rf < rd) rf = __uint_as_float(__float_as_uint(rf) + 1u);  // rd >= 0: the next float up
        uint64_t o0 = 0;
        if (lane == 0 && e < experts)
            o0 = __hip_atomic_exchange(&tc[e], ((uint64_t)__float_as_uint(rf) << 32) | __float_as_uint(lf),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::"v"(o0) : "memory");  // the exchange has completed
    }
    __shared__ uint32_t s_drawn;
    __syncthreads();
    if (tid == 0) s_drawn = atomicAdd(&tickets[token], 1u);
    __syncthreads();
    if (s_drawn != gridDim.x - 1) return;

    // The token's last workgroup: thread i < experts owns row i.
    __shared__ double c_lo[256], c_hi[256];
    __shared__ double c_klo;
    __shared__ double c_d[256];
    __shared__ uint32_t c_sel[256], c_x[256], c_xn, c_c[256], c_cn, c_inx[256];
    __shared__ uint64_t c_keys[256];
    __shared__ uint32_t c_rank[T];
    __shared__ float c_v[256], s_value[256];
    __shared__ float s_sum;
    __shared__ uint32_t s_missing;
    const bool own = tid < experts;
    double L = 0.0, lo = 0.0, hi = 0.0;
    bool fin = true;
    if (own) {
        const uint64_t pk = __hip_atomic_load(&tc[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        L = (double)__uint_as_float((uint32_t)pk);
        const double rho = (double)__uint_as_float((uint32_t)(pk >> 32));
        fin = __builtin_isfinite(rho);
        lo = L - rho;
        hi = L + rho;
        c_lo[tid] = lo;
        c_hi[tid] = hi;
    }
    if (tid == 0) {
        c_xn = 0;
        c_cn = 0;
        s_missing = 0;
    }
    const bool all_fin = __syncthreads_and((int)fin) != 0;
    bool certified = false, member = own;
    if (all_fin) {
        // Candidate order: by (f32(L), index) keys.  Any order is sound (the
        // test below proves the reference's order or fails); L values that
        // round to one f32 lie within one ulp, inside their intervals, so
        // they fail it whichever order they take.  T / 128 threads (T / 256
        // above 128 experts) count each key's rank over a part of the keys.
        if (own) c_keys[tid] = argmax_key((float)L, tid);
        __syncthreads();
        const uint32_t per = experts <= 128 ? 128u : 256u, split = T / per;
        const uint32_t span = (experts + split - 1) / split, me = tid % per, begin = tid / per * span;
        c_rank[tid] = me < experts && begin < experts
                          ? key_rank(c_keys + begin, span < experts - begin ? span : experts - begin, c_keys[me])
                          : 0u;
        __syncthreads();
        uint32_t rank = experts;
        if (own) {
            rank = 0;
            for (uint32_t q = 0; q < split; q++) rank += c_rank[q * per + tid];
        }
        if (rank < k) c_sel[rank] = tid;
        __syncthreads();
        bool ok = true;
        if (own) ok = rank < k ? rank == k - 1 || lo > c_hi[c_sel[rank + 1]] : hi < c_lo[c_sel[k - 1]];
        certified = __syncthreads_and((int)ok) != 0;
        if (certified) {
            if (own) c_v[tid] = (float)L;
        } else {
            // every row whose interval lies below all k candidates' is below
            // k rows for certain
            if (tid == 0) {
                double m = c_lo[c_sel[0]];
                for (uint32_t j = 1; j < k; j++) m = fmin(m, c_lo[c_sel[j]]);
                c_klo = m;
            }
            __syncthreads();
            member = own && hi >= c_klo;
        }
    }
    bool row_bad = false;
    if (!certified) {
        // A non-finite L comes from a non-finite input of its row or of x:
        // the reference's logit is then NaN or infinite and the call fails,
        // whatever the selection (the ids only stay in range for the lookup).
        const bool nan_row = own && !__builtin_isfinite(L);
        if (nan_row) *non_finite.word = non_finite.mark;  // every writer stores the same value
        row_bad = __syncthreads_or((int)nan_row) != 0;
        if (row_bad) {
            if (tid < k) {
                c_sel[tid] = tid;
                c_v[tid] = 0.0f;
            }
        } else {
            // X: the members of C whose interval meets another member's (every
            // row when an interval is infinite: a fold that may overflow).  The
            // other members' intervals are disjoint from every other member's,
            // so their order follows from L.
            if (member) c_c[atomicAdd(&c_cn, 1u)] = tid;
            __syncthreads();
            bool in_x = member && !all_fin;
            if (member && all_fin)
                for (uint32_t j = 0; j < c_cn; j++) {
                    const uint32_t f = c_c[j];
                    in_x |= f != tid && lo <= c_hi[f] && c_lo[f] <= hi;
                }
            if (own) c_inx[tid] = in_x ? 1u : 0u;
            if (in_x) c_x[atomicAdd(&c_xn, 1u)] = tid;
            // x into LDS as f32 pieces after the row area, zero past `hidden`
            const uint32_t NS = router_lds_steps(hidden), RS = router_lds_row_pieces(hidden);
            v4a *xs = cert_lds + rf * RS;
            for (uint32_t p = tid; p < 2 * NS; p += T)
                xs[p] = __builtin_bit_cast(v4a, rsrc_load16(rx, p < 2 * N8 ? 16 * p : nowhere));
            __syncthreads();
            // The rows of X, rf at a time: widened to f32 into LDS (zero past
            // `hidden`), then lane i < rf of wave 0 folds row i sequentially
            // from column 0 with fma, as router_lds_kernel does.
            for (uint32_t b0 = 0; b0 < c_xn; b0 += rf) {
                const uint32_t nb = c_xn - b0 < rf ? c_xn - b0 : rf;
                for (uint32_t p0 = 0; p0 < nb * NS; p0 += 4 * T) {
                    v4a wr[4];
#pragma unroll
                    for (uint32_t j = 0; j < 4; j++) {
                        const uint32_t p = p0 + j * T + tid, rr = p / NS, col = p - rr * NS;
                        const bool real = p < nb * NS && col < N8;
                        wr[j] = __builtin_bit_cast(
                            v4a, rsrc_load16(rw, real ? (c_x[b0 + rr] * N8 + col) * 16 : nowhere));
                    }
#pragma unroll
                    for (uint32_t j = 0; j < 4; j++) {
                        const uint32_t p = p0 + j * T + tid, rr = p / NS, col = p - rr * NS;
                        if (p < nb * NS) {
                            const v4a w = wr[j];
                            cert_lds[rr * RS + 2 * col] =
                                v4a{w[0] << 16, w[0] & 0xffff0000u, w[1] << 16, w[1] & 0xffff0000u};
                            cert_lds[rr * RS + 2 * col + 1] =
                                v4a{w[2] << 16, w[2] & 0xffff0000u, w[3] << 16, w[3] & 0xffff0000u};
                        }
                    }
                }
                __syncthreads();
                if (tid < 64) {
                    LdsChainState st;
                    st.wrow = cert_lds + (tid % nb) * RS;
                    st.xs = xs;
                    lds_chain_read<0>(st, 0);
                    lds_chain_read<1>(st, 1);
                    lds_chain_read<2>(st, 2);
                    static_assert(kRlAhead == 3, "the prologue reads kRlAhead steps");
                    st.acc = 0.0f;
                    constexpr auto ring = std::make_integer_sequence<uint32_t, kRlRing>{};
                    uint32_t base = 0;
#pragma unroll 1
                    for (; base + kRlRing < NS; base += kRlRing) lds_chain_ring<kRlRing>(st, base, ring);
                    lds_chain_ring<kRlRing - kRlAhead>(st, base, ring);
                    if (tid < nb) c_v[c_x[b0 + tid]] = st.acc;
                }
                __syncthreads();
            }
            const bool bad = in_x && !__builtin_isfinite(c_v[tid]);
            if (bad) *non_finite.word = non_finite.mark;  // every writer stores the same value
            row_bad = __syncthreads_or((int)bad) != 0;
            // Order C: two members of X by their exact logits (value, then
            // index, as the reference sorts), any other pair by value (L, or a
            // member of X's exact logit: their intervals are disjoint).
            if (in_x) c_keys[tid] = argmax_key(c_v[tid], tid);
            if (member) c_d[tid] = in_x ? (double)c_v[tid] : L;
            __syncthreads();
            if (member) {
                uint32_t rank = 0;
                for (uint32_t j = 0; j < c_cn; j++) {
                    const uint32_t f = c_c[j];
                    if (f != tid) rank += in_x && c_inx[f] ? (c_keys[f] > c_keys[tid] ? 1u : 0u)
                                                           : (c_d[f] > c_d[tid] ? 1u : 0u);
                }
                if (rank < k) c_sel[rank] = tid;
                if (!in_x) c_v[tid] = (float)L;
            }
        }
    }
    __syncthreads();  // the selection and its values (c_sel, c_v) are complete
    // softmax_in_place over the selected logits (src/cpu.rs:195-230):
    // maximum, exp(v - max), sequential sum, divide; selection s by thread s,
    // the sum in selection order by thread 0.
    uint32_t *ti = ids + (size_t)token * k;
    float *tp = probabilities + (size_t)token * k;
    if (tid < k) {
        const uint32_t index = c_sel[tid];
        float maximum = -__builtin_inff();
        for (uint32_t j = 0; j < k; j++) maximum = fmaxf(maximum, c_v[c_sel[j]]);
        s_value[tid] = expf(c_v[index] - maximum);
        ti[tid] = index;
        if (host_ids) host_ids[(size_t)token * k + tid] = index;
        if (lookup.go) {
            const uint64_t gu = lookup.gate_up_of[index], dn = lookup.down_of[index];
            lookup.gate_up_w[(size_t)token * k + tid] = gu;
            lookup.down_w[(size_t)token * k + tid] = dn;
            if (gu == 0 || dn == 0) s_missing = 1;  // every writer stores the same value
        }
    }
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (uint32_t j = 0; j < k; j++) sum += s_value[j];
        s_sum = sum;
    }
    __syncthreads();
    if (tid < k) {
        const float p = s_value[tid] / s_sum;
        tp[tid] = p;
        if (host_ids) host_probs[(size_t)token * k + tid] = p;
    }
    if (tid == 0) {
        if (host_ids) host_bad[token] = row_bad;
        if (lookup.go) {
            const uint32_t go = row_bad || s_missing ? 0u : 1u;
            lookup.go[token] = go;
            lookup.host_go[token] = go;
        }
        __hip_atomic_store(&tickets[token], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Top-k softmax over the router logits (at most 256) of one token per
// workgroup, with the selection also written to (pinned) host memory when
// host_ids is set.
__global__ void __launch_bounds__(256) top_k_host_kernel(const float *__restrict__ logits, uint32_t count,
                                                         uint32_t k, uint32_t *ids, float *probabilities,
                                                         BadFlag non_finite, uint32_t *host_ids,
                                                         float *host_probs, uint32_t *host_bad) {
    __shared__ float s_row[256];
    const uint32_t row = blockIdx.x;
    uint32_t *ti = ids + (size_t)row * k;
    float *tp = probabilities + (size_t)row * k;
    // the row once into LDS (count <= 256), where the k selection rounds read it
    if (threadIdx.x < count) s_row[threadIdx.x] = logits[(size_t)row * count + threadIdx.x];
    __syncthreads();
    const bool bad = block_top_k(s_row, count, k, ti, tp, non_finite);
    if (host_ids && threadIdx.x == 0) {
        for (uint32_t s = 0; s < k; s++) {
            host_ids[(size_t)row * k + s] = ti[s];
            host_probs[(size_t)row * k + s] = tp[s];
        }
        host_bad[row] = bad;
    }
}

// ---- RMSNorm (src/cpu.rs:98-142) ---------------------------------------
__global__ void __launch_bounds__(256) rms_norm_kernel(const float *__restrict__ in, uint32_t n,
                                                       const float *__restrict__ weight, float eps,
                                                       float *__restrict__ out) {
    __shared__ float partial[4];
    const float *row = in + (size_t)blockIdx.x * n;
    float *orow = out + (size_t)blockIdx.x * n;
    float s = 0.0f;
    for (size_t i = threadIdx.x; i < n; i += blockDim.x) s = __builtin_fmaf(row[i], row[i], s);
    s = wave_sum(s);
    if ((threadIdx.x & 63u) == 0) partial[threadIdx.x >> 6] = s;
    __syncthreads();
    float total = 0.0f;
    for (uint32_t w = 0; w < blockDim.x / 64; w++) total += partial[w];
    // (sum / n + eps).sqrt().recip(): two correctly rounded steps.
    float inverse_rms = 1.0f / __builtin_sqrtf(total / (float)n + eps);
    for (size_t i = threadIdx.x; i < n; i += blockDim.x)
        orow[i] = weight ? row[i] * weight[i] * inverse_rms : row[i] * inverse_rms;
}

// silu(g) * u with the stable sigmoid of src/qwen35/cpu.rs:982-993.
__device__ __forceinline__ float silu_stable(float v) {
    float sigmoid;
    if (v >= 0.0f) {
        sigmoid = 1.0f / (1.0f + expf(-v));
    } else {
        float e = expf(v);
        sigmoid = e / (1.0f + e);
    }
    return v * sigmoid;
}

// No __restrict__ on the elementwise kernels: the output may be either
// input (each element is read by the thread that writes it).
__global__ void silu_mul_kernel(const float *gate, const float *up, size_t n, float *out) {
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = silu_stable(gate[i]) * up[i];
}

// Ordered expert combine (src/gemma4/cpu.rs:608-611): for every token and
// feature, y = fma(out_j, p_j, y) over the k selections in order.
__global__ void moe_combine_kernel(const float *__restrict__ expert_out, const float *__restrict__ p,
                                   uint32_t batch, uint32_t k, uint32_t hidden,
                                   float *__restrict__ y) {
    size_t total = (size_t)batch * hidden;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        uint32_t t = (uint32_t)(e / hidden), i = (uint32_t)(e - (size_t)t * hidden);
        float acc = 0.0f;
        for (uint32_t j = 0; j < k; j++)
            acc = __builtin_fmaf(expert_out[((size_t)t * k + j) * hidden + i], p[(size_t)t * k + j], acc);
        y[e] = acc;
    }
}

// (gate / (1 + exp(-gate))) * up, src/glm52/expert.rs:260-267, applied to
// `pairs` rows of [gate(width) | up(width)] into act[pairs][width].
__global__ void silu_mul_glm_pairs_kernel(const float *__restrict__ gate_up, uint32_t pairs,
                                          uint32_t width, float *__restrict__ act) {
    size_t total = (size_t)pairs * width;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        uint32_t p = (uint32_t)(e / width), i = (uint32_t)(e - (size_t)p * width);
        float g = gate_up[(size_t)p * 2 * width + i];
        float u = gate_up[(size_t)p * 2 * width + width + i];
        act[e] = (g / (1.0f + expf(-g))) * u;
    }
}

// Plain streaming copy: 16-byte vectors where both ends allow, bytes else.
__global__ void __launch_bounds__(256) copy_bytes_kernel(uint8_t *__restrict__ dst,
                                                         const uint8_t *__restrict__ src, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if ((((uintptr_t)dst | (uintptr_t)src) & 15u) == 0) {
        const size_t vec = n / 16;
        for (size_t i = tid; i < vec; i += stride)
            ((u32x4 *)dst)[i] = ((const u32x4 *)src)[i];
        for (size_t i = vec * 16 + tid; i < n; i += stride) dst[i] = src[i];
    } else {
        for (size_t i = tid; i < n; i += stride) dst[i] = src[i];
    }
}

// ---- host-side launchers -------------------------------------------------

hipError_t launch_copy_bytes(hipStream_t s, void *dst, const void *src, size_t n) {
    size_t blocks = (n / 16 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(copy_bytes_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, (uint8_t *)dst,
                       (const uint8_t *)src, n);
    return hipGetLastError();
}

hipError_t launch_dequantize(hipStream_t s, uint32_t type, const uint8_t *enc, uint32_t be,
                             uint32_t bb, size_t elements, float *out) {
    size_t blocks = (elements + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(dequantize_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, type, enc, be,
                       bb, elements, out);
    return hipGetLastError();
}

hipError_t launch_gemv_exact(hipStream_t s, uint32_t type, uint32_t be, uint32_t bb, uint32_t rows,
                             uint32_t columns, size_t row_bytes, const uint8_t *w, uint32_t batch,
                             const float *x, float *y) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(gemv_exact_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, type, be, bb, rows,
                       columns, row_bytes, w, batch, x, y);
    return hipGetLastError();
}

hipError_t launch_argmax(hipStream_t s, const float *v, size_t n, ArgmaxState *state,
                         uint32_t *index) {
    hipLaunchKernelGGL(argmax_init_kernel, dim3(1), dim3(1), 0, s, state);
    size_t blocks = (n + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(argmax_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, v, n, state);
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(1), 0, s, state, index);
    return hipGetLastError();
}

hipError_t launch_argmax_init(hipStream_t s, ArgmaxState *state) {
    hipLaunchKernelGGL(argmax_init_kernel, dim3(1), dim3(1), 0, s, state);
    return hipGetLastError();
}

hipError_t launch_argmax_finish(hipStream_t s, const ArgmaxState *state, uint32_t *index) {
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(1), 0, s, state, index);
    return hipGetLastError();
}

hipError_t launch_top_k(hipStream_t s, const float *logits, uint32_t rows, uint32_t count,
                        uint32_t k, uint32_t *ids, float *probabilities, BadFlag non_finite) {
    hipLaunchKernelGGL(top_k_kernel, dim3(rows), dim3(256), 0, s, logits, count, k, ids,
                       probabilities, non_finite);
    return hipGetLastError();
}

template <uint32_t CC>
static hipError_t launch_router_staged(hipStream_t s, const uint16_t *router, uint32_t hidden,
                                       uint32_t experts, uint32_t k, uint32_t batch, const float *x,
                                       float *logits, uint32_t *ids, float *probabilities,
                                       BadFlag non_finite, uint32_t *host_ids, float *host_probs,
                                       uint32_t *host_bad) {
    const size_t lds = 2 * (((size_t)experts * (CC * 2 + 16) + CC * 4 + 15) & ~(size_t)15);
    // the largest slot ring, once per device
    static LdsLimit limit;
    const size_t most = 2 * (((size_t)(2048 / (CC / 8)) * (CC * 2 + 16) + CC * 4 + 15) & ~(size_t)15);
    hipError_t e = limit.ensure((const void *)router_staged_kernel<CC>, most);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(router_staged_kernel<CC>, dim3(batch), dim3(256), lds, s, router, hidden, experts, k, x,
                       logits, ids, probabilities, non_finite, host_ids, host_probs, host_bad);
    return hipGetLastError();
}

namespace {
bool router_staged(uint32_t hidden, uint32_t experts, const void *router, const float *x) {
    return experts <= 256 && hidden % 8 == 0 && (uint64_t)experts * hidden * 2 < (1ull << 30) &&
           ((uintptr_t)router & 15u) == 0 && ((uintptr_t)x & 15u) == 0;
}
}  // namespace

bool router_takes_lookup(uint32_t hidden, uint32_t experts, uint32_t batch, const void *router, const float *x) {
    return batch >= 1 && batch <= kMaxLookupTokens && router_staged(hidden, experts, router, x) &&
           experts >= 2 * RF_EXPERTS;
}

hipError_t launch_router_top_k(hipStream_t s, const uint16_t *router, uint32_t hidden,
                               uint32_t experts, uint32_t k, uint32_t batch, const float *x,
                               float *logits, uint32_t *ids, float *probabilities,
                               BadFlag non_finite, uint32_t *host_ids, float *host_probs, uint32_t *tickets,
                               uint32_t *host_bad, const ExpertLookup *lookup, bool certified) {
    if (host_ids && (!host_probs || !host_bad)) return hipErrorInvalidValue;
    const bool staged = router_staged(hidden, experts, router, x);
    if (lookup && (!tickets || !router_takes_lookup(hidden, experts, batch, router, x)))
        return hipErrorInvalidValue;
    const ExpertLookup no_lookup{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    const ExpertLookup L = lookup ? *lookup : no_lookup;
    // Decode batches: the expert-parallel fold, then the selection.
    if (staged && experts >= 2 * RF_EXPERTS && certified && tickets && hidden <= 8192) {
        // exact folds of the rows the bounds cannot order: two at a time up
        // to 4096 columns (49 KB of LDS), one at a time above (up to 65 KB)
        const uint32_t rf = hidden <= 4096 ? 2u : 1u;
        const size_t lds = router_lds_bytes(hidden, rf);
        // Up to 8 tokens, 4 waves per workgroup (measured 1.2-1.7 us faster
        // at 1 and 4 tokens); above, 8 waves (2.4 us faster at 16 tokens:
        // half the workgroups take each token's ticket).
        auto launch = [&](auto kernel, uint32_t waves, LdsLimit &limit) {
            hipError_t e = limit.ensure((const void *)kernel, lds);
            if (e != hipSuccess) return e;
            hipLaunchKernelGGL(kernel, dim3((experts + waves - 1) / waves, batch), dim3(64 * waves), lds, s, router,
                               hidden, experts, k, x, (uint64_t *)logits, tickets, ids, probabilities, non_finite,
                               host_ids, host_probs, host_bad, L, rf);
            return hipGetLastError();
        };
        static LdsLimit limit4, limit8;
        return batch <= kMaxLookupTokens ? launch(router_cert_kernel<4>, 4, limit4)
                                         : launch(router_cert_kernel<8>, 8, limit8);
    }
    if (staged && experts >= 2 * RF_EXPERTS) {
        // as many rows per workgroup as fit in LDS beside x and the
        // kernel's own arrays (the rank selection's keys, ids, logits)
        constexpr size_t kLdsBudget = 160 * 1024 - 8 * 1024;
        const size_t row = (size_t)router_lds_row_pieces(hidden) * 16, xbytes = (size_t)router_lds_steps(hidden) * 32;
        const uint32_t R = xbytes < kLdsBudget ? (uint32_t)std::min<size_t>(64, (kLdsBudget - xbytes) / row) : 0;
        if (R >= 4 && router_lds_steps(hidden) <= 1024) {
            static LdsLimit limit;
            const size_t lds = router_lds_bytes(hidden, R);
            hipError_t e = limit.ensure((const void *)router_lds_kernel, lds);
            if (e != hipSuccess) return e;
            hipLaunchKernelGGL(router_lds_kernel, dim3((experts + R - 1) / R, batch), dim3(256), lds, s, router,
                               hidden, experts, R, k, x, logits, tickets, ids, probabilities, non_finite, host_ids,
                               host_probs, host_bad, L);
        } else
            hipLaunchKernelGGL(router_fold_kernel, dim3((experts + RF_EXPERTS - 1) / RF_EXPERTS, batch), dim3(64),
                               0, s, router, hidden, experts, k, x, logits, tickets, ids, probabilities, non_finite,
                               host_ids, host_probs, host_bad, L);
        if (!tickets)
            hipLaunchKernelGGL(top_k_host_kernel, dim3(batch), dim3(256), 0, s, logits, experts, k, ids,
                               probabilities, non_finite, host_ids, host_probs, host_bad);
        return hipGetLastError();
    }
    if (staged && experts <= 128)
        return launch_router_staged<128>(s, router, hidden, experts, k, batch, x, logits, ids, probabilities,
                                         non_finite, host_ids, host_probs, host_bad);
    if (staged)
        return launch_router_staged<64>(s, router, hidden, experts, k, batch, x, logits, ids, probabilities,
                                        non_finite, host_ids, host_probs, host_bad);
    // This kernel reports through the shared word only, which host_bad[0]
    // receives: cleared first, so it holds this call's mark or zero.
    if (host_ids) {
        hipError_t e0 = launch_fill_u32(s, non_finite.word, 1, 0);
        if (e0 != hipSuccess) return e0;
    }
    hipLaunchKernelGGL(router_top_k_kernel, dim3(batch), dim3(256), experts * sizeof(float), s,
                       router, hidden, experts,
                       k, x, logits, ids, probabilities, non_finite);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !host_ids) return e;
    e = hipMemcpyAsync(host_ids, ids, (size_t)batch * k * 4, hipMemcpyDeviceToHost, s);
    if (e != hipSuccess) return e;
    e = hipMemcpyAsync(host_probs, probabilities, (size_t)batch * k * 4, hipMemcpyDeviceToHost, s);
    if (e != hipSuccess) return e;
    // this kernel only sets the shared flag: it stands for every token
    return hipMemcpyAsync(host_bad, non_finite.word, 4, hipMemcpyDeviceToHost, s);
}

__global__ void fill_u32_kernel(uint32_t *p, uint32_t n, uint32_t value) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = value;
}

hipError_t launch_fill_u32(hipStream_t s, uint32_t *p, uint32_t n, uint32_t value) {
    hipLaunchKernelGGL(fill_u32_kernel, dim3((n + 255) / 256 < 64 ? (n + 255) / 256 : 64), dim3(256), 0, s, p, n,
                       value);
    return hipGetLastError();
}

hipError_t launch_rms_norm(hipStream_t s, const float *in, uint32_t batch, uint32_t n,
                           const float *weight, float eps, float *out) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(batch), dim3(256), 0, s, in, n, weight, eps, out);
    return hipGetLastError();
}

hipError_t launch_silu_mul(hipStream_t s, const float *gate, const float *up, size_t n, float *out) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, gate, up, n, out);
    return hipGetLastError();
}

// Logit softcap, src/cpu.rs:263-273: cap * tanh(value / cap), fp32 (the
// division, tanh and product each round once).
__global__ void softcap_kernel(const float *in, size_t n, float cap, float *out) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float q = in[i] / cap;
        out[i] = cap * tanhf(q);
    }
}

hipError_t launch_softcap(hipStream_t s, const float *in, size_t n, float cap, float *out) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(softcap_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, in, n, cap, out);
    return hipGetLastError();
}

// ---- Gemma 4 / GLM glue: vector add, GELU multiply, softmax, NeoX RoPE ----

// output = left + right (src/metal.rs:404-432, metal/kernels.metal:34-43).
__global__ void add_kernel(const float *a, const float *b, size_t n, float *out) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = a[i] + b[i];
}

hipError_t launch_add(hipStream_t s, const float *a, const float *b, size_t n, float *out) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(add_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, a, b, n, out);
    return hipGetLastError();
}

// Gemma 4's gelu_pytorch_tanh in the CPU's order (src/cpu.rs:144-149):
// 0.5 v (1 + tanh(0.7978846 (v + 0.044715 (v v) v))), each operation
// rounded once.
__device__ __forceinline__ float gelu_tanh(float v) {
    const float cubic = (v * v) * v;
    const float inner = 0.7978846f * (v + 0.044715f * cubic);
    return (0.5f * v) * (1.0f + tanhf(inner));
}

// gelu_tanh(gate) * up (src/metal.rs:530-552, src/gemma4/cpu.rs).
__global__ void gelu_mul_kernel(const float *gate, const float *up, size_t n, float *out) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = gelu_tanh(gate[i]) * up[i];
}

hipError_t launch_gelu_mul(hipStream_t s, const float *gate, const float *up, size_t n, float *out) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(gelu_mul_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, gate, up, n, out);
    return hipGetLastError();
}

// Softmax of one finite vector (src/metal.rs:578-598; src/cpu.rs:196-225):
// the maximum, e_i = exp(x_i - max), their sum, then e_i / sum.  One
// workgroup of 1024 threads: thread t takes i = t, t + 1024, ...; the sum
// is a fixed tree (in-thread, then the wave, then the 16 waves in order).
__global__ void __launch_bounds__(1024) softmax_kernel(const float *__restrict__ in, uint32_t n,
                                                       float *__restrict__ out) {
    __shared__ float red[16];
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    float mx = -INFINITY;
    for (size_t i = t; i < n; i += 1024) mx = fmaxf(mx, in[i]);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
    for (int w = 1; w < 16; w++) mx = fmaxf(mx, red[w]);
    __syncthreads();
    float sum = 0.0f;
    for (size_t i = t; i < n; i += 1024) {
        const float e = expf(in[i] - mx);
        out[i] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    sum = red[0];
    for (int w = 1; w < 16; w++) sum += red[w];
    // each thread divides the values it wrote
    for (size_t i = t; i < n; i += 1024) out[i] = out[i] / sum;
}

hipError_t launch_softmax(hipStream_t s, const float *in, uint32_t n, float *out) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(1024), 0, s, in, n, out);
    return hipGetLastError();
}

// NeoX rotary embedding in place (src/cpu.rs:151-193,
// metal/kernels.metal:74-94): for head h and pair p < rotated_pairs,
// (x[p], x[p + hd/2]) of the head turns by
// angle = position * theta^(-2p / hd); the division, powf, the product,
// sinf, cosf, the four products and the two sums each round once, in the
// CPU's order (no contraction).
__global__ void rope_neox_kernel(float *__restrict__ v, size_t heads, uint32_t head_dim, uint32_t pairs,
                                 uint32_t position, float theta) {
    const size_t total = heads * pairs;
    const uint32_t half = head_dim / 2;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const size_t head = idx / pairs;
        const uint32_t pair = (uint32_t)(idx - head * pairs);
        const float exponent = -(float)(2 * pair) / (float)head_dim;
        const float angle = (float)position * powf(theta, exponent);
        const float sine = sinf(angle), cosine = cosf(angle);
        float *x = v + head * head_dim;
        const float first = x[pair], second = x[half + pair];
        x[pair] = first * cosine - second * sine;
        x[half + pair] = first * sine + second * cosine;
    }
}

hipError_t launch_rope_neox(hipStream_t s, float *v, size_t heads, uint32_t head_dim, uint32_t pairs,
                            uint32_t position, float theta) {
    size_t blocks = (heads * pairs + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_neox_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, v, heads, head_dim, pairs,
                       position, theta);
    return hipGetLastError();
}

hipError_t launch_moe_combine(hipStream_t s, const float *expert_out, const float *p, uint32_t batch,
                              uint32_t k, uint32_t hidden, float *y) {
    size_t total = (size_t)batch * hidden;
    size_t blocks = (total + 255) / 256;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, expert_out, p,
                       batch, k, hidden, y);
    return hipGetLastError();
}

hipError_t launch_silu_mul_glm_pairs(hipStream_t s, const float *gate_up, uint32_t pairs,
                                     uint32_t width, float *act) {
    size_t total = (size_t)pairs * width;
    size_t blocks = (total + 255) / 256;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(silu_mul_glm_pairs_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, gate_up,
                       pairs, width, act);
    return hipGetLastError();
}

// A kernel of this file: resolving it loads the file's code object.
const void *module_anchor_simple() { return (const void *)fill_u32_kernel; }

}  // namespace dm
