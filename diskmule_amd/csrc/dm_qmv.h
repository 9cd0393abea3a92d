// dm_qmv.h -- MFMA quantized matvec (decode GEMV, batch 1..16) for gfx950.
#pragma once

#include "runtime.h"

namespace dm {

// Per-wave argmax candidate written by the fused epilogues; a one-workgroup
// pass reduces them.
struct ArgmaxPartial {
    unsigned long long key;
    uint32_t non_finite;
    uint32_t pad;
};

// Fused argmax finish of the int8 kernel: every workgroup folds its
// candidate into *best with a device-scope atomic maximum and then takes a
// ticket; the one that draws the last ticket writes `state` and `index` and
// resets *best and *ticket to zero (their value before every launch).  All
// null: the candidates go to `partials` for a separate pass.
struct ArgmaxFinish {
    ArgmaxState *state;
    uint32_t *index;
    uint32_t *ticket;
    unsigned long long *best;
};

// True when the int8-MFMA matvec (decode batches of 1-4 tokens, Q4_K/Q6_K/
// Q8_0, whose activation records fit the workgroup's LDS) takes this shape;
// the caller has already checked qmv_supported.
bool qmv8_supported(uint32_t type, size_t rows, size_t columns, size_t batch);

// y[b][r] = W[r] . x[b] with the int8-MFMA kernels.  With `partials` the
// epilogue also writes one ArgmaxPartial per workgroup (batch 1) and *count
// receives the number written; with a `finish` ticket the kernel reduces
// them itself into finish.state / finish.index.
hipError_t launch_qmv8(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns, const void *w,
                       uint32_t batch, const float *x, float *y, ArgmaxPartial *partials,
                       uint32_t *count, ArgmaxFinish finish = ArgmaxFinish{nullptr, nullptr, nullptr, nullptr});

// The int8-MFMA gate/up pair: act[b][r] = silu(gate[r] . n[b]) * (up[r] . n[b])
// with n = RMSNorm(x) (unit weight) when `normalize`, else n = x.
bool qmv8_gate_up_supported(uint32_t type, size_t rows, size_t columns, size_t batch);
hipError_t launch_qmv8_gate_up(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns,
                               const void *gate, const void *up, uint32_t batch, const float *x,
                               float *act, int normalize, float epsilon);

// One job of a grouped routed-expert launch: the matrix at `w` (in gate/up
// form the gate rows, the up rows following at up_offset bytes) applied to
// `tokens` (1 or 2) activation rows x + x_off + t * x_stride, writing
// y + y_off + t * y_stride (offsets and strides in floats).
constexpr uint32_t kMaxGroupedJobs = 64;  // jobs per launch of the grouped kernel

struct QmvJob {
    const void *w;
    uint32_t tokens;
    uint32_t x_off, y_off;
    int32_t x_stride, y_stride;
};

// True when the grouped int8-MFMA launch takes jobs of this shape (`mats`
// 2 for the gate/up form).  Slot buffers must be 4-byte aligned (16 for
// Q4_K) and hold whole rows.
bool qmv8_grouped_supported(uint32_t type, size_t rows, size_t columns, uint32_t mats);

// All jobs in one or a few launches.  gate_up == 0: y = W x.  gate_up == 1:
// y = (g / (1 + exp(-g))) * u with g = gate . x, u = up . x, the routed-expert
// activation of src/glm52/expert.rs:260-267.
// The ordered combine of each token's experts fused into their down launch:
// jobs t * k .. t * k + k - 1 are token t's selections, and
// y_final[t * y_stride + r] = sum over them in order of
// fma(y[p * rows + r], p_[p], .), with one zeroed ticket per token and
// row-tile workgroup (returned to zero).
struct QmvCombine {
    uint32_t *tickets;
    size_t tickets_count;
    const float *p;
    float *y;
    uint32_t k, y_stride;
};

// With dev_w (one-token jobs, at most 64, one launch) the job addresses are
// read on the device from dev_w[job] and the launch does nothing unless
// go[0 .. go_count) are all 1: both written by a kernel earlier on the
// stream (ExpertLookup).  With combine (one-token down jobs writing
// y + p * rows) the launch also makes the ordered combine.
hipError_t launch_qmv8_grouped(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns, int gate_up,
                               uint64_t up_offset, const QmvJob *jobs, size_t count, const float *x, float *y,
                               const uint64_t *dev_w = nullptr, const uint32_t *go = nullptr,
                               const QmvCombine *combine = nullptr, uint32_t go_count = 1);

// True when the MFMA matvec takes this shape: Q4_K or Q6_K rows of whole
// 256-value blocks, a weight base address aligned to 4 bytes (16 for Q4_K),
// and fewer than 4 GiB of weights (one buffer descriptor); or Q8_0 rows of
// whole 256-value super-blocks at a 16-byte aligned base, batch 1-2.
bool qmv_supported(uint32_t type, size_t rows, size_t columns, const void *w, size_t batch);

// Bytes of the activation fragments the fp16 kernel prepares for `batch`
// tokens (batches above 2) of rows of `columns` values.
size_t qmv_prepare_bytes(uint32_t type, size_t columns, size_t batch);

// y[b][r] = W[r] . x[b]; when `argmax` is non-null (batch 1) the kernels
// also reset `argmax`, fold a greedy argmax over the rows into it and write
// the winning row to *index_out.
hipError_t launch_qmv(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns,
                      const void *w, uint32_t batch, const float *x, float *y,
                      ArgmaxState *argmax, uint32_t *index_out);

// Two weight matrices of the same shape applied to the same x, writing
// silu(gate) * up (the dense FFN's gate/up pair, src/qwen35/cpu.rs:420-424),
// optionally with the RMSNorm scale of each token folded in.
hipError_t launch_qmv_gate_up(dmhip_ctx *ctx, uint32_t type, uint32_t rows, uint32_t columns,
                              const void *gate, const void *up, uint32_t batch, const float *x,
                              float *act, int normalize, float epsilon);

}  // namespace dm
