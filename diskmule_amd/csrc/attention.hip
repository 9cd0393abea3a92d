// attention.hip -- decode attention of one query token over a KV ring:
// MetalContext::new_kv_layer / append_kv / attention_cached / attention and
// MetalKvLayer (src/metal.rs:245-277, :1196-1511, metal/kernels.metal:486-578).
//
// Layout: a layer holds two device rings, keys and values, of `capacity`
// slots x `width` floats (width = kv_heads * head_dimension, row-major, the
// reference's buffers).  Position p lives in slot p % capacity.
//
// Two kernels per call:
//  * attn_chunk_kernel: workgroup (chunk, kv head, head group) scores the
//    chunk's positions for the query heads that share the KV head, takes the
//    chunk's softmax statistics and its unnormalised weighted value sum;
//  * attn_combine_kernel: workgroup (query head, 64 dims) merges the chunks.
// Each score is the reference's sequential fma over the head dimension
// (d ascending, one lane per position), so scores are bit-identical to the
// CPU fold; the keys reach the lanes through LDS so that every HBM read is a
// coalesced row segment.
#include "dm_device.h"
#include "runtime.h"

#include <math.h>
#include <string.h>

#include <algorithm>

struct dmhip_kv_layer {
    dmhip_ctx *ctx = nullptr;
    int device = 0;
    float *keys = nullptr;    // device, [capacity][width]
    float *values = nullptr;  // device, [capacity][width]
    size_t width = 0, capacity = 0, max_context = 0, position = 0;
};

namespace dm {

constexpr uint32_t kAttnThreads = 256;
constexpr uint32_t kAttnRows = 64;        // positions per scoring pass (one per lane)
// key dims staged per pass: 128 (512-byte row segments) for 16-byte loads,
// 64 for element loads
template <bool KV4>
constexpr uint32_t key_tile() { return KV4 ? 128 : 64; }
template <bool KV4>
constexpr uint32_t key_stride() { return key_tile<KV4>() + (KV4 ? 4 : 1); }
constexpr uint32_t kAttnScores = 4096;    // LDS scores: heads per group x chunk
constexpr uint32_t kAttnMaxChunk = 512;
constexpr uint32_t kCombineBlock = 2048;  // chunk weights staged per combine pass
constexpr uint32_t kAttnQueryLds = 8192;  // query floats a workgroup stages in LDS

template <bool KV4>
struct KeyStage {
    // KV4: eight 16-byte units per thread (64 rows x 32 units); else sixteen
    // floats (64 rows x 64 columns).
    float v[KV4 ? key_tile<true>() / 4 : 16];
};

template <bool KV4>
__device__ __forceinline__ void attn_load_keys(KeyStage<KV4> &st, const float *__restrict__ keys,
                                               uint64_t capacity, uint64_t width, uint64_t head_off,
                                               uint64_t slot0, uint32_t row0, uint32_t n, uint32_t dim0,
                                               uint32_t head_dim) {
    constexpr uint32_t units = key_tile<KV4>() / (KV4 ? 4 : 1);  // per row
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < (KV4 ? (int)key_tile<true>() / 16 : 16); i++) {
        const uint32_t u = t + kAttnThreads * i;
        const uint32_t row = u / units;
        const uint32_t col = (u % units) * (KV4 ? 4 : 1);
        const uint32_t r = row0 + row;
        const uint32_t d = dim0 + col;
        // Every lane loads, from a row and column clamped into the chunk: no
        // branch and no use of the value before it is stored, so waiting for
        // one register stage leaves the next in flight.  A row past the
        // chunk's end scores garbage that is replaced by -inf; a column past
        // head_dim is never read.
        uint64_t slot = slot0 + min(r, n - 1);
        if (slot >= capacity) slot -= capacity;
        const float *src = keys + slot * width + head_off + min(d, head_dim - (KV4 ? 4 : 1));
        if constexpr (KV4) {
            const float4 k = *(const float4 *)src;
            st.v[4 * i + 0] = k.x;
            st.v[4 * i + 1] = k.y;
            st.v[4 * i + 2] = k.z;
            st.v[4 * i + 3] = k.w;
        } else {
            st.v[i] = *src;
        }
    }
}

template <bool KV4>
__device__ __forceinline__ void attn_store_keys(const KeyStage<KV4> &st, float *ktile) {
    constexpr uint32_t stride = key_stride<KV4>();
    constexpr uint32_t units = key_tile<KV4>() / (KV4 ? 4 : 1);
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < (KV4 ? (int)key_tile<true>() / 16 : 16); i++) {
        const uint32_t u = t + kAttnThreads * i;
        if constexpr (KV4) {
            const uint32_t row = u / units, col = (u % units) * 4;
            *(float4 *)&ktile[row * stride + col] =
                make_float4(st.v[4 * i], st.v[4 * i + 1], st.v[4 * i + 2], st.v[4 * i + 3]);
        } else {
            ktile[(u >> 6) * stride + (u & 63u)] = st.v[i];
        }
    }
}

// GT: query heads per workgroup (a power of two >= the heads it takes);
// KV4: head_dim % 4 == 0 with 16-byte aligned rows and query; VV: value
// dims per thread per pass (hd % VV == 0); QL: the workgroup's query rows
// are staged in LDS (dynamic, GT * head_dim floats), else read through the
// scalar cache.
template <int GT, bool KV4, int VV, bool QL>
__global__ void __launch_bounds__(256)
attn_chunk_kernel(const float *__restrict__ query, const float *__restrict__ keys,
                  const float *__restrict__ values, uint64_t capacity, uint64_t width, uint32_t group,
                  uint32_t head_dim, uint64_t start, uint32_t visible, uint32_t chunk, uint32_t chunks,
                  float *__restrict__ part_o, float2 *__restrict__ part_ml, BadFlag bad) {
    constexpr int CH = GT >= 4 ? GT / 4 : 1;  // score chains per lane
    constexpr int VU = VV == 4 ? 8 : 16;       // value rows in flight per thread
    constexpr uint32_t stride = key_stride<KV4>();
    constexpr uint32_t kAttnTile = key_tile<KV4>();
    __shared__ __attribute__((aligned(16))) float ktile[kAttnRows * stride];
    __shared__ __attribute__((aligned(16))) float sc[kAttnScores];
    __shared__ float s_m[GT], s_l[GT];
    extern __shared__ __attribute__((aligned(16))) float qs[];

    const uint32_t t = threadIdx.x, lane = t & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t c = blockIdx.x, kh = blockIdx.y;
    const uint32_t g_base = blockIdx.z * GT;
    const uint32_t gz = min((uint32_t)GT, group - g_base);  // heads of this workgroup
    const uint32_t p0 = c * chunk;
    const uint32_t n = min(chunk, visible - p0);
    const uint64_t head_off = (uint64_t)kh * head_dim;
    const uint64_t slot0 = (start + p0) % capacity;
    const uint64_t qbase = (uint64_t)kh * group + g_base;

    // ---- scores: lane = position, chains over d ascending ----
    // Wave w scores heads w, w+4, ... (GT >= 4) or head w (GT < 4); a chain
    // past the workgroup's heads reads a valid head and is dropped.
    // LDS reads keep every wait on the LDS counter short; scalar loads of
    // the query would share that counter and hold each wait for an L2 trip.
    if constexpr (QL) {
        const float *src = query + qbase * head_dim;
        for (uint32_t i = t; i < gz * head_dim; i += kAttnThreads) qs[i] = src[i];
    }
    const float *qrow[CH];
    int chain_head[CH];
    bool chain_on[CH];
#pragma unroll
    for (int ch = 0; ch < CH; ch++) {
        chain_head[ch] = (int)wave + 4 * ch;
        chain_on[ch] = (uint32_t)chain_head[ch] < gz;
        const uint32_t h = min((uint32_t)chain_head[ch], gz - 1);
        qrow[ch] = QL ? qs + h * head_dim : query + (qbase + h) * head_dim;
    }
    const uint32_t subs = (n + kAttnRows - 1) / kAttnRows;
    const uint32_t tiles = (head_dim + kAttnTile - 1) / kAttnTile;
    // Two register stages: the keys of step s + 2 are in flight while step s
    // is scored.
    const uint32_t steps = subs * tiles;
    float acc[CH];
    auto load_step = [&](KeyStage<KV4> &stage, uint32_t step) {
        // past the last step: reload the last tile (the loads stay
        // unconditional, so the waits count them exactly)
        step = min(step, steps - 1);
        const uint32_t sb = step / tiles, tl = step - sb * tiles;
        attn_load_keys<KV4>(stage, keys, capacity, width, head_off, slot0, sb * kAttnRows, n, tl * kAttnTile,
                            head_dim);
    };
    auto run_step = [&](KeyStage<KV4> &stage, uint32_t step) {
        __syncthreads();
        attn_store_keys<KV4>(stage, ktile);
        __syncthreads();
        load_step(stage, step + 2);
        const uint32_t sb = step / tiles, tl = step - sb * tiles;
        if (tl == 0) {
#pragma unroll
            for (int ch = 0; ch < CH; ch++) acc[ch] = 0.0f;
        }
        const uint32_t dim0 = tl * kAttnTile;
        const uint32_t dmax = min(kAttnTile, head_dim - dim0);
        const float *krow = ktile + lane * stride;
        if constexpr (KV4) {
#pragma unroll 4
            for (uint32_t dd = 0; dd < dmax; dd += 4) {
                const float4 k4 = *(const float4 *)(krow + dd);
#pragma unroll
                for (int ch = 0; ch < CH; ch++) {
                    const float4 q4 = *(const float4 *)(qrow[ch] + dim0 + dd);
                    acc[ch] = __builtin_fmaf(q4.x, k4.x, acc[ch]);
                    acc[ch] = __builtin_fmaf(q4.y, k4.y, acc[ch]);
                    acc[ch] = __builtin_fmaf(q4.z, k4.z, acc[ch]);
                    acc[ch] = __builtin_fmaf(q4.w, k4.w, acc[ch]);
                }
            }
        } else {
            for (uint32_t dd = 0; dd < dmax; dd++) {
                const float k = krow[dd];
#pragma unroll
                for (int ch = 0; ch < CH; ch++) acc[ch] = __builtin_fmaf(qrow[ch][dim0 + dd], k, acc[ch]);
            }
        }
        if (tl + 1 == tiles && sb < subs) {
            const uint32_t r = sb * kAttnRows + lane;
#pragma unroll
            for (int ch = 0; ch < CH; ch++)
                if (chain_on[ch]) sc[chain_head[ch] * chunk + r] = r < n ? acc[ch] : -INFINITY;
        }
    };
    // An odd step count runs one extra step over the last tile again; it
    // writes no scores (sb == subs).
    KeyStage<KV4> st0, st1;
    load_step(st0, 0);
    // keep stage 0's loads issued before stage 1's, as in the loop, so the
    // wait before the first store leaves stage 1 in flight
    __builtin_amdgcn_sched_barrier(0);
    load_step(st1, 1);
    for (uint32_t step = 0; step < steps; step += 2) {
        run_step(st0, step);
        run_step(st1, step + 1);
    }
    // positions of the last pass past the chunk's end (chunk is a multiple of 64)
    __syncthreads();

    // ---- chunk softmax statistics: wave w takes heads w, w+4, ... ----
    for (uint32_t g = wave; g < gz; g += 4) {
        float *row = sc + g * chunk;
        float mx = -INFINITY;
        bool flag = false;
        for (uint32_t r = lane; r < n; r += 64) {
            const float s = row[r];
            flag |= isnan(s) || s == INFINITY;
            mx = fmaxf(mx, s);
        }
        mx = wave_max(mx);
        float sum = 0.0f;
        for (uint32_t r = lane; r < chunk; r += 64) {
            const float e = (r < n && mx != -INFINITY) ? expf(row[r] - mx) : 0.0f;
            row[r] = e;
            sum += e;
        }
        sum = wave_sum(sum);
        if (flag) *bad.word = bad.mark;
        if (lane == 0) {
            s_m[g] = mx;
            s_l[g] = sum;
        }
    }
    __syncthreads();

    // ---- unnormalised value sums: thread = VV dims, positions ascending ----
    const uint64_t prow = ((uint64_t)kh * chunks + c) * group + g_base;
    for (uint32_t d0 = 0; d0 < head_dim; d0 += kAttnThreads * VV) {
        const uint32_t d = d0 + t * VV;
        const bool active = d < head_dim;
        float o[GT][VV];
#pragma unroll
        for (int g = 0; g < GT; g++)
#pragma unroll
            for (int k = 0; k < VV; k++) o[g][k] = 0.0f;
        // Loads are unconditional (rows clamped into the chunk) and a row past
        // the chunk's end is zeroed where it is used, not where it is
        // loaded, so accumulating one batch waits only for that batch.
        auto load_rows = [&](float (&v)[VU][VV], uint32_t j) {
#pragma unroll
            for (int i = 0; i < VU; i++) {
                uint64_t slot = slot0 + min(j + i, n - 1);
                if (slot >= capacity) slot -= capacity;
                const float *src = values + slot * width + head_off + min(d, head_dim - VV);
                if constexpr (VV == 4) {
                    const float4 x = *(const float4 *)src;
                    v[i][0] = x.x, v[i][1] = x.y, v[i][2] = x.z, v[i][3] = x.w;
                } else if constexpr (VV == 2) {
                    const float2 x = *(const float2 *)src;
                    v[i][0] = x.x, v[i][1] = x.y;
                } else {
                    v[i][0] = *src;
                }
            }
        };
        auto add_rows = [&](const float (&v)[VU][VV], uint32_t j) {
            float u[VU][VV];
#pragma unroll
            for (int i = 0; i < VU; i++)
#pragma unroll
                for (int k = 0; k < VV; k++) u[i][k] = active && j + i < n ? v[i][k] : 0.0f;
#pragma unroll
            for (int g = 0; g < GT; g++) {
                if ((uint32_t)g >= gz) break;
#pragma unroll
                for (int i0 = 0; i0 < VU; i0 += 4) {
                    const float4 e = *(const float4 *)&sc[g * chunk + j + i0];
                    const float ev[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int k = 0; k < VV; k++)
                            o[g][k] = __builtin_fmaf(u[i0 + i][k], ev[i], o[g][k]);
                }
            }
        };
        // two register batches: the rows of batch b + 1 are in flight while
        // batch b is accumulated
        float va[VU][VV], vb[VU][VV];
        load_rows(va, 0);
        __builtin_amdgcn_sched_barrier(0);
        for (uint32_t j = 0; j < n; j += 2 * VU) {
            load_rows(vb, j + VU);
            add_rows(va, j);
            load_rows(va, j + 2 * VU);
            if (j + VU < n) add_rows(vb, j + VU);
        }
        if (active) {
#pragma unroll
            for (int g = 0; g < GT; g++) {
                if ((uint32_t)g >= gz) break;
                float *dst = part_o + (prow + g) * head_dim + d;
#pragma unroll
                for (int k = 0; k < VV; k++) dst[k] = o[g][k];
            }
        }
    }
    if (t < gz) part_ml[prow + t] = make_float2(s_m[t], s_l[t]);
}

// out[h][d] = sum_c w_c o_c[d] / sum_c w_c l_c, w_c = exp(m_c - max_c m_c).
// Workgroup (query head, 64 dims, split s) sums the chunks of split s, in
// chunk order per wave and a fixed tree across the four waves.  With more
// than one split each workgroup publishes its sums and takes a ticket of its
// (head, dims) counter; the one that draws the last ticket adds the splits
// in split order, writes the output and resets the counter to zero.
__global__ void __launch_bounds__(256)
attn_combine_kernel(const float *__restrict__ part_o, const float2 *__restrict__ part_ml, uint32_t group,
                    uint32_t head_dim, uint32_t chunks, uint32_t per, float *__restrict__ stage_o,
                    float *__restrict__ stage_l, uint32_t *__restrict__ tickets, float *__restrict__ out,
                    BadFlag bad) {
    __shared__ float wts[kCombineBlock];
    __shared__ float red[4 * 64];
    __shared__ uint32_t s_ticket;
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    const uint32_t head = blockIdx.x, block = blockIdx.y, split = blockIdx.z;
    const uint32_t splits = gridDim.z, blocks = gridDim.y;
    const uint32_t kh = head / group, gg = head % group;
    const uint32_t d = block * 64 + lane;
    const uint64_t row0 = (uint64_t)kh * chunks * group + gg;  // chunk c at row0 + c * group
    const uint64_t rstride = group;
    const uint32_t c0 = split * per, cn = min(per, chunks - c0);

    float mx = -INFINITY;
    for (uint32_t c = t; c < chunks; c += 256) mx = fmaxf(mx, part_ml[row0 + c * rstride].x);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    if (mx == -INFINITY) {
        // every score -inf (or NaN): no ticket is taken
        if (t == 0) *bad.word = bad.mark;
        if (wave == 0 && d < head_dim) out[(uint64_t)head * head_dim + d] = NAN;
        return;
    }
    float l = 0.0f;
    for (uint32_t i = t; i < cn; i += 256) {
        const float2 ml = part_ml[row0 + (uint64_t)(c0 + i) * rstride];
        const float w = ml.x != -INFINITY ? expf(ml.x - mx) : 0.0f;
        wts[i] = w;
        l = __builtin_fmaf(w, ml.y, l);
    }
    l = wave_sum(l);
    if (lane == 0) red[wave] = l;
    __syncthreads();
    l = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();

    float acc = 0.0f;
    if (d < head_dim) {
        const float *src = part_o + (row0 + (uint64_t)c0 * rstride) * head_dim + d;
        const uint64_t step = rstride * head_dim;
        uint32_t i = wave;
        for (; i + 28 < cn; i += 32) {
            float a[8];
#pragma unroll
            for (int u = 0; u < 8; u++) a[u] = src[(i + 4 * u) * step];
#pragma unroll
            for (int u = 0; u < 8; u++) acc = __builtin_fmaf(a[u], wts[i + 4 * u], acc);
        }
        for (; i < cn; i += 4) acc = __builtin_fmaf(src[i * step], wts[i], acc);
    }
    red[wave * 64 + lane] = acc;
    __syncthreads();
    const float sum = (red[lane] + red[64 + lane]) + (red[128 + lane] + red[192 + lane]);
    if (splits == 1) {
        if (wave == 0 && d < head_dim) out[(uint64_t)head * head_dim + d] = sum / l;
        return;
    }
    const uint64_t slot = ((uint64_t)head * blocks + block) * splits;
    // Publish with device-scope exchanges (no cache flush), wait until they
    // have completed, then take the ticket.
    if (wave == 0) {
        float old = 0.0f;
        if (d < head_dim)
            old = __hip_atomic_exchange(&stage_o[(slot + split) * 64 + lane], sum, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0)
            old += __hip_atomic_exchange(&stage_l[slot + split], l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::"v"(old) : "memory");
    }
    __syncthreads();
    if (t == 0) s_ticket = atomicAdd(&tickets[(uint64_t)head * blocks + block], 1u);
    __syncthreads();
    if (s_ticket != splits - 1) return;
    // The last workgroup adds the splits: wave w takes splits w, w+4, ...
    // in order (loads issued eight at a time), then a fixed tree across the
    // waves; the split sums of l likewise, one per thread.
    float o = 0.0f;
    for (uint32_t s0 = wave; s0 < splits; s0 += 32) {
        float a[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t s2 = s0 + 4 * u;
            a[u] = s2 < splits && d < head_dim
                       ? __hip_atomic_load(&stage_o[(slot + s2) * 64 + lane], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT)
                       : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) o += a[u];
    }
    float lt = 0.0f;
    for (uint32_t s2 = t; s2 < splits; s2 += 256)
        lt += __hip_atomic_load(&stage_l[slot + s2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lt = wave_sum(lt);
    __syncthreads();
    red[wave * 64 + lane] = o;
    if (lane == 0) wts[wave] = lt;
    __syncthreads();
    if (wave == 0) {
        const float ot = (red[lane] + red[64 + lane]) + (red[128 + lane] + red[192 + lane]);
        const float lsum = (wts[0] + wts[1]) + (wts[2] + wts[3]);
        if (d < head_dim) out[(uint64_t)head * head_dim + d] = ot / lsum;
        if (lane == 0)
            __hip_atomic_store(&tickets[(uint64_t)head * blocks + block], 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int GT, bool KV4, int VV>
static hipError_t launch_chunk(dmhip_ctx *ctx, dim3 grid, const float *q, const float *k, const float *v,
                               uint64_t capacity, uint64_t width, uint32_t group, uint32_t hd,
                               uint64_t start, uint32_t visible, uint32_t chunk, uint32_t chunks,
                               float *po, float2 *pml, BadFlag bad) {
    if ((size_t)GT * hd <= kAttnQueryLds)
        return launch_kernel(ctx, attn_chunk_kernel<GT, KV4, VV, true>, grid, dim3(kAttnThreads),
                             (uint32_t)(GT * hd * 4), q, k, v, capacity, width, group, hd, start, visible, chunk,
                             chunks, po, pml, bad);
    return launch_kernel(ctx, attn_chunk_kernel<GT, KV4, VV, false>, grid, dim3(kAttnThreads), 0, q, k, v,
                         capacity, width, group, hd, start, visible, chunk, chunks, po, pml, bad);
}

template <int GT>
static hipError_t launch_chunk_gt(dmhip_ctx *ctx, bool kv4, int vv, dim3 grid, const float *q, const float *k,
                                  const float *v, uint64_t capacity, uint64_t width, uint32_t group,
                                  uint32_t hd, uint64_t start, uint32_t visible, uint32_t chunk,
                                  uint32_t chunks, float *po, float2 *pml, BadFlag bad) {
    if (!kv4) return launch_chunk<GT, false, 1>(ctx, grid, q, k, v, capacity, width, group, hd, start, visible, chunk, chunks, po, pml, bad);
    if (vv == 4 && GT <= 8) return launch_chunk<GT, true, GT <= 8 ? 4 : 2>(ctx, grid, q, k, v, capacity, width, group, hd, start, visible, chunk, chunks, po, pml, bad);
    if (vv == 2) return launch_chunk<GT, true, 2>(ctx, grid, q, k, v, capacity, width, group, hd, start, visible, chunk, chunks, po, pml, bad);
    return launch_chunk<GT, true, 1>(ctx, grid, q, k, v, capacity, width, group, hd, start, visible, chunk, chunks, po, pml, bad);
}

// The launch plan of one attention call.
struct AttnPlan {
    uint32_t gt, chunk, chunks, zgroups;
    bool kv4;
    int vv;
    uint32_t splits, per;  // combine: chunks per split, splits per (head, 64 dims)
    size_t part_o_floats, part_ml_pairs;
};

static AttnPlan attn_plan(size_t kv_heads, size_t group, size_t hd, size_t visible, bool aligned16) {
    AttnPlan p{};
    p.gt = group > 8 ? 16 : group > 4 ? 8 : group > 2 ? 4 : (uint32_t)group;
    p.zgroups = (uint32_t)((group + p.gt - 1) / p.gt);
    const uint32_t max_chunk = std::min<uint32_t>(kAttnMaxChunk, kAttnScores / p.gt);
    // about two workgroups per CU: chunk = 64 k positions
    size_t k = visible * kv_heads * p.zgroups / ((size_t)kAttnRows * 512);
    k = std::max<size_t>(1, std::min<size_t>(k, max_chunk / kAttnRows));
    p.chunk = (uint32_t)(k * kAttnRows);
    p.chunks = (uint32_t)((visible + p.chunk - 1) / p.chunk);
    p.kv4 = hd % 4 == 0 && aligned16;
    // four value dims per thread only up to 8 heads (16 x 4 accumulators spill)
    p.vv = p.kv4 && hd >= 1024 && p.gt <= 8 ? 4 : (p.kv4 && hd >= 512 ? 2 : 1);
    // about 32 chunks per combine workgroup, at most kCombineBlock
    p.splits = std::max<uint32_t>((p.chunks + 31) / 32, (p.chunks + kCombineBlock - 1) / kCombineBlock);
    p.splits = std::min<uint32_t>(p.splits, 32768);
    p.per = (p.chunks + p.splits - 1) / p.splits;
    p.splits = (p.chunks + p.per - 1) / p.per;
    p.part_o_floats = kv_heads * (size_t)p.chunks * group * hd;
    p.part_ml_pairs = kv_heads * (size_t)p.chunks * group;
    return p;
}

// Enqueues one attention call on the context stream.  Shapes are validated:
// query [kv_heads * group][hd], rings of `capacity` slots of `width` floats.
static int enqueue_attention(dmhip_ctx *ctx, const float *query, const float *keys, const float *values,
                             size_t capacity, size_t width, size_t query_heads, size_t kv_heads, size_t hd,
                             size_t start, size_t visible, float *output, BadFlag bad) {
    const size_t group = query_heads / kv_heads;
    const bool aligned16 = (((uintptr_t)query | (uintptr_t)keys | (uintptr_t)values) & 15u) == 0;
    const AttnPlan p = attn_plan(kv_heads, group, hd, visible, aligned16);
    const size_t blocks = (hd + 63) / 64;
    const size_t stage_o_floats = p.splits > 1 ? query_heads * blocks * p.splits * 64 : 0;
    const size_t stage_l_floats = p.splits > 1 ? query_heads * blocks * p.splits : 0;
    auto round256 = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t o_bytes = round256(p.part_o_floats * 4), ml_bytes = round256(p.part_ml_pairs * 8);
    const size_t so_bytes = round256(stage_o_floats * 4);
    DM_CHECK_STATUS(ctx->attn.ensure(o_bytes + ml_bytes + so_bytes + stage_l_floats * 4));
    uint8_t *base = (uint8_t *)ctx->attn.ptr;
    float *po = (float *)base;
    float2 *pml = (float2 *)(base + o_bytes);
    float *so = (float *)(base + o_bytes + ml_bytes);
    float *sl = (float *)(base + o_bytes + ml_bytes + so_bytes);
    uint32_t *tickets = nullptr;
    if (p.splits > 1) {
        const size_t need = query_heads * blocks;
        if (need > ctx->attn_ticket_count) {
            // counters start at zero and every call leaves them at zero
            DM_CHECK_STATUS(ctx->attn_tickets.ensure(need * 4));
            DM_HIP(launch_fill_u32(ctx->stream, (uint32_t *)ctx->attn_tickets.ptr, (uint32_t)need, 0));
            ctx->attn_ticket_count = need;
        }
        tickets = (uint32_t *)ctx->attn_tickets.ptr;
    }
    const dim3 grid(p.chunks, (uint32_t)kv_heads, p.zgroups);
    hipError_t e;
    switch (p.gt) {
    case 1: e = launch_chunk_gt<1>(ctx, p.kv4, p.vv, grid, query, keys, values, capacity, width, (uint32_t)group, (uint32_t)hd, start, (uint32_t)visible, p.chunk, p.chunks, po, pml, bad); break;
    case 2: e = launch_chunk_gt<2>(ctx, p.kv4, p.vv, grid, query, keys, values, capacity, width, (uint32_t)group, (uint32_t)hd, start, (uint32_t)visible, p.chunk, p.chunks, po, pml, bad); break;
    case 4: e = launch_chunk_gt<4>(ctx, p.kv4, p.vv, grid, query, keys, values, capacity, width, (uint32_t)group, (uint32_t)hd, start, (uint32_t)visible, p.chunk, p.chunks, po, pml, bad); break;
    case 8: e = launch_chunk_gt<8>(ctx, p.kv4, p.vv, grid, query, keys, values, capacity, width, (uint32_t)group, (uint32_t)hd, start, (uint32_t)visible, p.chunk, p.chunks, po, pml, bad); break;
    default: e = launch_chunk_gt<16>(ctx, p.kv4, p.vv, grid, query, keys, values, capacity, width, (uint32_t)group, (uint32_t)hd, start, (uint32_t)visible, p.chunk, p.chunks, po, pml, bad); break;
    }
    if (e != hipSuccess) return hip_fail(e, "attention chunk kernel");
    e = launch_kernel(ctx, attn_combine_kernel, dim3((uint32_t)query_heads, (uint32_t)blocks, p.splits), dim3(256),
                      0, (const float *)po, (const float2 *)pml, (uint32_t)group, (uint32_t)hd, p.chunks, p.per, so,
                      sl, tickets, output, bad);
    if (e != hipSuccess) return hip_fail(e, "attention combine kernel");
    return DMHIP_OK;
}

// A kernel of this file: resolving it loads the file's code object.
const void *module_anchor_attention() { return (const void *)attn_combine_kernel; }

// ---- validation, same checks in the same order as src/metal.rs ----

static int fail_shape(const char *reason) {
    fail(DMHIP_ERR_INVALID_ATTENTION_SHAPE, "invalid attention shape: %s", reason);
    last_detail().reason = reason;
    return DMHIP_ERR_INVALID_ATTENTION_SHAPE;
}

static int fail_kv_position(size_t expected, size_t actual) {
    fail(DMHIP_ERR_KV_POSITION, "HIP KV cache is at position %zu; expected %zu", actual, expected);
    last_detail().expected = expected;
    last_detail().actual = actual;
    return DMHIP_ERR_KV_POSITION;
}

static int fail_kv_width(size_t expected, size_t actual) {
    fail(DMHIP_ERR_KV_WIDTH, "HIP KV cache width is %zu; expected %zu", actual, expected);
    last_detail().expected = expected;
    last_detail().actual = actual;
    return DMHIP_ERR_KV_WIDTH;
}

static int fail_kv_context(size_t position, size_t limit) {
    fail(DMHIP_ERR_KV_CONTEXT, "HIP KV cache position %zu exceeds its context limit %zu", position, limit);
    last_detail().position = position;
    last_detail().limit = limit;
    return DMHIP_ERR_KV_CONTEXT;
}

static int fail_overflow() {
    return fail(DMHIP_ERR_OVERFLOW, "matrix dimensions or encoded byte length overflowed");
}

static int fail_u32() {
    return fail(DMHIP_ERR_VECTOR_TOO_LARGE, "HIP vector length exceeds the 32-bit kernel limit");
}

static bool mul_overflows(size_t a, size_t b, size_t *out) { return __builtin_mul_overflow(a, b, out); }

// The head checks shared by attention_cached (:1279-1294) and attention
// (:1336-1351): heads, then the widths' overflow, then the query/output
// lengths.
static int check_heads(size_t query_heads, size_t kv_heads, size_t hd, size_t query_len, size_t output_len,
                       size_t *cache_width) {
    if (query_heads == 0 || kv_heads == 0 || query_heads % kv_heads != 0)
        return fail_shape("query heads must be a non-zero multiple of KV heads");
    size_t query_width;
    if (mul_overflows(query_heads, hd, &query_width) || mul_overflows(kv_heads, hd, cache_width))
        return fail_overflow();
    if (query_len != query_width || output_len != query_width)
        return fail_shape("query and output must match query_heads * head_dimension");
    return DMHIP_OK;
}

// Kernel index limits (positions, widths and head counts are 32-bit there).
static int check_kernel_limits(size_t query_heads, size_t kv_heads, size_t hd, size_t visible) {
    // grid: (chunks, kv_heads, head groups) and (query_heads, hd / 64)
    if (query_heads > 0x7fffffffull || kv_heads > 65535 || hd > 0xffffffffull || visible > 0xffffffffull ||
        (hd + 63) / 64 > 65535 || (query_heads / kv_heads + 15) / 16 > 65535)
        return fail_u32();
    return DMHIP_OK;
}

static uint32_t next_mark(dmhip_ctx *ctx) {
    ctx->attn_mark = ctx->attn_mark + 1 ? ctx->attn_mark + 1 : 1;
    return ctx->attn_mark;
}

// The mark of a host-slice call: it ends the period of device calls awaiting
// a result, so while one is open it shares that period's mark and reports a
// non-finite score met by any of them, as dmhip_attention_result would.
static uint32_t host_call_mark(dmhip_ctx *ctx) {
    return ctx->attn_pending ? ctx->attn_mark : next_mark(ctx);
}

static int attention_finish_host(dmhip_ctx *ctx, HostCall &hc, float *output, const float *dout,
                                 size_t query_width) {
    uint32_t flag = 0;
    DM_CHECK_STATUS(hc.out(output, dout, query_width * 4));
    DM_CHECK_STATUS(hc.out(&flag, ctx->flags + kAttnFlagWord, 4));
    DM_CHECK_STATUS(hc.finish());
    ctx->attn_pending = false;
    if (flag == ctx->attn_mark) return fail_non_finite("softmax");
    return DMHIP_OK;
}

}  // namespace dm

using namespace dm;

#define DM_REQUIRE_PTR(ptr)                                                              \
    do {                                                                                 \
        if (!(ptr)) return fail(DMHIP_ERR_INVALID_ARGUMENT, "%s must not be null", #ptr); \
    } while (0)

extern "C" {

int dmhip_new_kv_layer(dmhip_ctx *ctx, size_t width, size_t max_context, int has_window, size_t sliding_window,
                       dmhip_kv_layer **out) {
    DM_REQUIRE_PTR(ctx);
    DM_REQUIRE_PTR(out);
    *out = nullptr;
    const size_t capacity = has_window ? std::min(sliding_window, max_context) : max_context;
    if (width == 0 || capacity == 0) return fail_shape("KV width and capacity must be non-zero");
    size_t elements, bytes;
    if (mul_overflows(width, capacity, &elements) || mul_overflows(elements, sizeof(float), &bytes))
        return fail_overflow();
    DM_CHECK_STATUS(set_device(ctx));
    dmhip_kv_layer *layer = new dmhip_kv_layer();
    layer->ctx = ctx;
    layer->device = ctx->device;
    layer->width = width;
    layer->capacity = capacity;
    layer->max_context = max_context;
    if (hipMalloc((void **)&layer->keys, bytes) != hipSuccess) {
        delete layer;
        return fail_alloc(bytes);
    }
    if (hipMalloc((void **)&layer->values, bytes) != hipSuccess) {
        (void)hipFree(layer->keys);
        delete layer;
        return fail_alloc(bytes);
    }
    *out = layer;
    return DMHIP_OK;
}

void dmhip_kv_layer_free(dmhip_kv_layer *layer) {
    if (!layer) return;
    (void)hipSetDevice(layer->device);
    // work already enqueued on the context stream may still read the rings
    if (layer->ctx && layer->ctx->stream) (void)hipStreamSynchronize(layer->ctx->stream);
    if (layer->keys) (void)hipFree(layer->keys);
    if (layer->values) (void)hipFree(layer->values);
    delete layer;
}

size_t dmhip_kv_layer_position(const dmhip_kv_layer *layer) { return layer ? layer->position : 0; }
size_t dmhip_kv_layer_capacity(const dmhip_kv_layer *layer) { return layer ? layer->capacity : 0; }
size_t dmhip_kv_layer_width(const dmhip_kv_layer *layer) { return layer ? layer->width : 0; }

size_t dmhip_kv_layer_allocated_bytes(const dmhip_kv_layer *layer) {
    if (!layer) return 0;
    // capacity * width * 4 * 2, saturating (src/metal.rs:264-269)
    size_t a;
    if (mul_overflows(layer->capacity, layer->width, &a) || mul_overflows(a, sizeof(float), &a) ||
        mul_overflows(a, 2, &a))
        return SIZE_MAX;
    return a;
}

void dmhip_kv_layer_clear(dmhip_kv_layer *layer) {
    if (layer) layer->position = 0;
}

void dmhip_kv_layer_truncate(dmhip_kv_layer *layer, size_t position) {
    if (layer) layer->position = std::min(layer->position, position);
}

void *dmhip_kv_layer_keys(const dmhip_kv_layer *layer) { return layer ? layer->keys : nullptr; }
void *dmhip_kv_layer_values(const dmhip_kv_layer *layer) { return layer ? layer->values : nullptr; }

static int append_checks(dmhip_kv_layer *layer, size_t position, size_t key_len, size_t value_len) {
    if (layer->position != position) return fail_kv_position(position, layer->position);
    if (position >= layer->max_context) return fail_kv_context(position, layer->max_context);
    if (key_len != layer->width || value_len != layer->width)
        return fail_kv_width(layer->width, std::min(key_len, value_len));
    return DMHIP_OK;
}

static int append_copy(dmhip_ctx *ctx, dmhip_kv_layer *layer, size_t position, const float *key,
                       const float *value, hipMemcpyKind kind) {
    const size_t slot = position % layer->capacity;
    size_t offset;
    if (mul_overflows(slot, layer->width, &offset)) return fail_overflow();
    const size_t bytes = layer->width * sizeof(float);
    DM_HIP(hipMemcpyAsync(layer->keys + offset, key, bytes, kind, ctx->stream));
    DM_HIP(hipMemcpyAsync(layer->values + offset, value, bytes, kind, ctx->stream));
    return DMHIP_OK;
}

int dmhip_append_kv(dmhip_ctx *ctx, dmhip_kv_layer *layer, size_t position, const float *key, size_t key_len,
                    const float *value, size_t value_len) {
    DM_REQUIRE_PTR(ctx);
    DM_REQUIRE_PTR(layer);
    DM_CHECK_STATUS(append_checks(layer, position, key_len, value_len));
    DM_REQUIRE_PTR(key);
    DM_REQUIRE_PTR(value);
    DM_CHECK_STATUS(set_device(ctx));
    DM_CHECK_STATUS(append_copy(ctx, layer, position, key, value, hipMemcpyHostToDevice));
    // the host slices may be reused once this returns
    DM_CHECK_STATUS(stream_wait(ctx));
    layer->position += 1;
    return DMHIP_OK;
}

int dmhip_append_kv_device(dmhip_ctx *ctx, dmhip_kv_layer *layer, size_t position, const float *key_device,
                           size_t key_len, const float *value_device, size_t value_len) {
    DM_REQUIRE_PTR(ctx);
    DM_REQUIRE_PTR(layer);
    DM_CHECK_STATUS(append_checks(layer, position, key_len, value_len));
    DM_REQUIRE_PTR(key_device);
    DM_REQUIRE_PTR(value_device);
    DM_CHECK_STATUS(set_device(ctx));
    DM_CHECK_STATUS(append_copy(ctx, layer, position, key_device, value_device, hipMemcpyDeviceToDevice));
    layer->position += 1;
    return DMHIP_OK;
}

static int cached_checks(const float *query, size_t query_len, const dmhip_kv_layer *layer, size_t query_heads,
                         size_t kv_heads, size_t hd, size_t output_len) {
    size_t cache_width;
    DM_CHECK_STATUS(check_heads(query_heads, kv_heads, hd, query_len, output_len, &cache_width));
    if (layer->width != cache_width) return fail_kv_width(cache_width, layer->width);
    if (layer->position == 0) return fail_empty("attention");
    (void)query;
    return DMHIP_OK;
}

int dmhip_attention_cached(dmhip_ctx *ctx, const float *query, size_t query_len, const dmhip_kv_layer *layer,
                           size_t query_heads, size_t kv_heads, size_t head_dimension, float *output,
                           size_t output_len) {
    DM_REQUIRE_PTR(ctx);
    DM_REQUIRE_PTR(layer);
    DM_CHECK_STATUS(cached_checks(query, query_len, layer, query_heads, kv_heads, head_dimension, output_len));
    DM_REQUIRE_PTR(query);
    DM_REQUIRE_PTR(output);
    const size_t visible = std::min(layer->position, layer->capacity);
    const size_t start = layer->position - visible;
    DM_CHECK_STATUS(check_kernel_limits(query_heads, kv_heads, head_dimension, visible));
    DM_CHECK_STATUS(set_device(ctx));
    const size_t bytes = query_len * sizeof(float);
    DM_CHECK_STATUS(ctx->in.ensure(bytes));
    DM_CHECK_STATUS(ctx->out.ensure(bytes));
    float *dq = (float *)ctx->in.ptr, *dout = (float *)ctx->out.ptr;
    HostCall hc(ctx);
    DM_CHECK_STATUS(hc.begin(2 * bytes + 4));
    DM_CHECK_STATUS(hc.in(dq, query, bytes));
    const uint32_t mark = host_call_mark(ctx);
    DM_CHECK_STATUS(enqueue_attention(ctx, dq, layer->keys, layer->values, layer->capacity, layer->width,
                                      query_heads, kv_heads, head_dimension, start, visible, dout,
                                      BadFlag{ctx->flags + kAttnFlagWord, mark}));
    return attention_finish_host(ctx, hc, output, dout, query_len);
}

int dmhip_attention_cached_device(dmhip_ctx *ctx, const float *query_device, size_t query_len,
                                  const dmhip_kv_layer *layer, size_t query_heads, size_t kv_heads,
                                  size_t head_dimension, float *output_device, size_t output_len) {
    DM_REQUIRE_PTR(ctx);
    DM_REQUIRE_PTR(layer);
    DM_CHECK_STATUS(cached_checks(query_device, query_len, layer, query_heads, kv_heads, head_dimension,
                                  output_len));
    DM_REQUIRE_PTR(query_device);
    DM_REQUIRE_PTR(output_device);
    const size_t visible = std::min(layer->position, layer->capacity);
    const size_t start = layer->position - visible;
    DM_CHECK_STATUS(check_kernel_limits(query_heads, kv_heads, head_dimension, visible));
    DM_CHECK_STATUS(set_device(ctx));
    // the device calls between two results share one mark, so the result
    // reports a non-finite score in any of them
    const uint32_t mark = ctx->attn_pending ? ctx->attn_mark : next_mark(ctx);
    DM_CHECK_STATUS(enqueue_attention(ctx, query_device, layer->keys, layer->values, layer->capacity,
                                      layer->width, query_heads, kv_heads, head_dimension, start, visible,
                                      output_device, BadFlag{ctx->flags + kAttnFlagWord, mark}));
    ctx->attn_pending = true;
    return DMHIP_OK;
}

int dmhip_attention_result(dmhip_ctx *ctx) {
    DM_REQUIRE_PTR(ctx);
    if (!ctx->attn_pending)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "no dmhip_attention_cached_device call awaits its result");
    DM_CHECK_STATUS(set_device(ctx));
    uint32_t flag = 0;
    DM_HIP(hipMemcpyAsync(&flag, ctx->flags + kAttnFlagWord, 4, hipMemcpyDeviceToHost, ctx->stream));
    DM_HIP(hipStreamSynchronize(ctx->stream));  // a copy into pageable memory precedes
    ctx->attn_pending = false;
    if (flag == ctx->attn_mark) return fail_non_finite("softmax");
    return DMHIP_OK;
}

int dmhip_attention(dmhip_ctx *ctx, const float *query, size_t query_len, const float *keys, size_t keys_len,
                    const float *values, size_t values_len, size_t query_heads, size_t kv_heads,
                    size_t head_dimension, int has_window, size_t window, float *output, size_t output_len) {
    DM_REQUIRE_PTR(ctx);
    size_t cache_width;
    DM_CHECK_STATUS(check_heads(query_heads, kv_heads, head_dimension, query_len, output_len, &cache_width));
    if (cache_width == 0 || keys_len != values_len || keys_len % cache_width != 0)
        return fail_shape("key/value caches must have equal whole-position lengths");
    const size_t sequence_length = keys_len / cache_width;
    if (sequence_length == 0) return fail_empty("attention");
    const size_t start = has_window ? (sequence_length > window ? sequence_length - window : 0) : 0;
    const size_t visible = sequence_length - start;
    if (visible == 0) return fail_empty("attention window");
    DM_REQUIRE_PTR(query);
    DM_REQUIRE_PTR(keys);
    DM_REQUIRE_PTR(values);
    DM_REQUIRE_PTR(output);
    DM_CHECK_STATUS(check_kernel_limits(query_heads, kv_heads, head_dimension, visible));
    DM_CHECK_STATUS(set_device(ctx));
    // only the window's rows travel: slots [start, seq) as a ring of `visible`
    const size_t q_bytes = query_len * sizeof(float);
    const size_t kv_bytes = visible * cache_width * sizeof(float);
    const size_t kv_span = (kv_bytes + 255) & ~(size_t)255;
    DM_CHECK_STATUS(ctx->in.ensure(q_bytes));
    DM_CHECK_STATUS(ctx->out.ensure(q_bytes));
    DM_CHECK_STATUS(ctx->enc.ensure(2 * kv_span));
    float *dq = (float *)ctx->in.ptr, *dout = (float *)ctx->out.ptr;
    float *dk = (float *)ctx->enc.ptr, *dv = (float *)((uint8_t *)ctx->enc.ptr + kv_span);
    HostCall hc(ctx);
    DM_CHECK_STATUS(hc.begin(2 * q_bytes + 2 * kv_bytes + 4));
    DM_CHECK_STATUS(hc.in(dq, query, q_bytes));
    DM_CHECK_STATUS(hc.in(dk, keys + start * cache_width, kv_bytes));
    DM_CHECK_STATUS(hc.in(dv, values + start * cache_width, kv_bytes));
    const uint32_t mark = host_call_mark(ctx);
    DM_CHECK_STATUS(enqueue_attention(ctx, dq, dk, dv, visible, cache_width, query_heads, kv_heads,
                                      head_dimension, 0, visible, dout, BadFlag{ctx->flags + kAttnFlagWord, mark}));
    return attention_finish_host(ctx, hc, output, dout, query_len);
}

}  // extern "C"
