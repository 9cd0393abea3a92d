// dispatch.hip -- kernel selection for the matvec, FFN and GEMM operators.
#include "runtime.h"

#include <math.h>

#include "dm_qmv.h"

namespace dm {

int enqueue_matvec(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns, const void *w,
                   size_t batch, const float *x, float *y) {
    uint32_t be, bb;
    type_layout(type, &be, &bb);
    uint64_t row_bytes;
    row_byte_len(type, columns, &row_bytes);
    if (qmv_supported(type, rows, columns, w, batch)) {
        DM_HIP(launch_qmv(ctx, type, (uint32_t)rows, (uint32_t)columns, w, (uint32_t)batch, x, y,
                          nullptr, nullptr));
        return DMHIP_OK;
    }
    if (type == 8 && batch > 2 && qmv_supported(type, rows, columns, w, 2)) {
        // Q8_0 (8) has only the int8 kernel (1-2 tokens): one launch per pair
        // of tokens, each streaming the matrix at HBM rate, beats the exact
        // per-element kernel by an order of magnitude.
        for (size_t t = 0; t < batch; t += 2) {
            const uint32_t n = batch - t < 2 ? (uint32_t)(batch - t) : 2u;
            DM_HIP(launch_qmv(ctx, type, (uint32_t)rows, (uint32_t)columns, w, n, x + t * columns, y + t * rows,
                              nullptr, nullptr));
        }
        return DMHIP_OK;
    }
    KernelTimer timer(ctx);
    DM_HIP(launch_gemv_exact(ctx->stream, type, be, bb, (uint32_t)rows, (uint32_t)columns,
                             (size_t)row_bytes, (const uint8_t *)w, (uint32_t)batch, x, y));
    return DMHIP_OK;
}

int enqueue_matvec_argmax(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns,
                          const void *w, const float *x, float *y, uint32_t *index_device) {
    if (qmv_supported(type, rows, columns, w, 1)) {
        // Two launches: the activation pass resets the argmax state and the
        // matvec folds the argmax into its epilogue and publishes the index.
        DM_HIP(launch_qmv(ctx, type, (uint32_t)rows, (uint32_t)columns, w, 1, x, y,
                          ctx->argmax_state, index_device));
        return DMHIP_OK;
    }
    DM_CHECK_STATUS(enqueue_matvec(ctx, type, rows, columns, w, 1, x, y));
    DM_HIP(launch_argmax(ctx->stream, y, rows, ctx->argmax_state, index_device));
    return DMHIP_OK;
}

}  // namespace dm

using namespace dm;

extern "C" {

size_t dmhip_ffn_workspace_bytes(size_t batch, size_t hidden, size_t ffn) {
    // The unfused path's normalized copy of h, gate, up and activation rows
    // (the fused path uses only the activation rows), each region rounded to
    // 256 bytes.  0 when the size does not fit a size_t.
    size_t floats[4] = {batch * hidden, batch * ffn, batch * ffn, batch * ffn};
    if (batch && (hidden > SIZE_MAX / 4 / batch || ffn > SIZE_MAX / 4 / batch)) return 0;
    size_t total = 0;
    for (size_t f : floats) {
        const size_t bytes = (f * sizeof(float) + 255) & ~(size_t)255;
        if (bytes > SIZE_MAX - total) return 0;
        total += bytes;
    }
    return total;
}

int dmhip_ffn_device(dmhip_ctx *ctx, size_t batch, size_t hidden, size_t ffn, uint32_t gate_type,
                     const void *gate, uint32_t up_type, const void *up, uint32_t down_type,
                     const void *down, float epsilon, const float *h, float *y, void *workspace,
                     size_t workspace_len) {
    if (!ctx || !gate || !up || !down || !h || !y || !workspace)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "ffn arguments must not be null");
    if (batch < 1 || batch > 16)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "batch %zu is outside 1..=16", batch);
    if (hidden == 0 || ffn == 0) return fail_empty("FFN");
    const size_t need = dmhip_ffn_workspace_bytes(batch, hidden, ffn);
    if (need == 0 || workspace_len < need)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "FFN workspace holds %zu bytes; the shape needs %zu",
                    workspace_len, need);
    if (!isfinite(epsilon) || epsilon <= 0.0f)
        return fail_positive("RMSNorm epsilon");
    uint64_t rb;
    const uint32_t types[3] = {gate_type, up_type, down_type};
    const size_t cols[3] = {hidden, hidden, ffn};
    for (int i = 0; i < 3; i++) {
        uint32_t t = types[i];
        if (!(t == 0 || t == 1 || t == 6 || t == 8 || t == 12 || t == 14))
            return fail_unsupported(t, "HIP FFN");
        if (!row_byte_len(t, cols[i], &rb)) return fail_element_count(t, cols[i]);
    }
    if (hidden > 0xffffffffull || ffn > 0xffffffffull)
        return fail(DMHIP_ERR_VECTOR_TOO_LARGE, "HIP vector length exceeds the 32-bit kernel limit");
    DM_CHECK_STATUS(set_device(ctx));
    // [batch][ffn] activation rows first (all the fused path uses), then the
    // unfused path's [batch][hidden] normalized rows, gate and up rows.
    auto region = [](size_t floats) { return (floats * sizeof(float) + 255) & ~(size_t)255; };
    char *ws = (char *)workspace;
    float *a = (float *)ws;
    float *normalized = (float *)(ws + region(batch * ffn));
    float *g = (float *)((char *)normalized + region(batch * hidden));
    float *u = (float *)((char *)g + region(batch * ffn));
    // Fused (Q4_K or Q6_K pairs, the types of the gate/up kernels): RMSNorm
    // folded into the gate/up kernel's activation scale and silu(gate) * up
    // in its epilogue, then the down projection.
    if (gate_type == up_type && (gate_type == 12 || gate_type == 14) &&  // Q4_K, Q6_K
        qmv_supported(gate_type, ffn, hidden, gate, batch) &&
        qmv_supported(up_type, ffn, hidden, up, batch)) {
        if (qmv8_gate_up_supported(gate_type, ffn, hidden, batch))
            DM_HIP(launch_qmv8_gate_up(ctx, gate_type, (uint32_t)ffn, (uint32_t)hidden, gate, up,
                                       (uint32_t)batch, h, a, 1, epsilon));
        else
            DM_HIP(launch_qmv_gate_up(ctx, gate_type, (uint32_t)ffn, (uint32_t)hidden, gate, up,
                                      (uint32_t)batch, h, a, 1, epsilon));
        DM_CHECK_STATUS(enqueue_matvec(ctx, down_type, hidden, ffn, down, batch, a, y));
        return DMHIP_OK;
    }
    DM_HIP(launch_rms_norm(ctx->stream, h, (uint32_t)batch, (uint32_t)hidden, nullptr, epsilon, normalized));
    DM_CHECK_STATUS(enqueue_matvec(ctx, gate_type, ffn, hidden, gate, batch, normalized, g));
    DM_CHECK_STATUS(enqueue_matvec(ctx, up_type, ffn, hidden, up, batch, normalized, u));
    DM_HIP(launch_silu_mul(ctx->stream, g, u, batch * ffn, a));
    DM_CHECK_STATUS(enqueue_matvec(ctx, down_type, hidden, ffn, down, batch, a, y));
    return DMHIP_OK;
}

}  // extern "C"
