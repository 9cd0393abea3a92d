// dm_qmv.h -- MFMA quantized matvec (decode GEMV, batch 1..16) for gfx950.
#pragma once

#include "runtime.h"

namespace dm {

// True when the MFMA matvec takes this shape: Q4_K or Q6_K rows of whole
// 256-value blocks, a weight base address aligned to 4 bytes (16 for Q4_K),
// and fewer than 4 GiB of weights (one buffer descriptor).
bool qmv_supported(uint32_t type, size_t rows, size_t columns, const void *w, size_t batch);

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
