// dispatch.hip -- kernel selection for the matvec, FFN and GEMM operators.
#include "runtime.h"

#include <math.h>

#include <atomic>

#include "dm_qmv.h"

namespace dm {

// Device memory of the allocation-free FFN entry point: a fixed array in the
// code object, so each GPU that loads the library holds its own copy until
// the process ends.  In host code `scratch` names a host-side stand-in, not
// a device address: the address of a device's copy comes from
// hipGetSymbolAddress (noalloc_resolve), once per device, and only that
// address is handed to kernels.
constexpr size_t kNoAllocScratchBytes = 8u << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
static std::atomic<void *> g_scratch_address[64];

int noalloc_resolve(int device) {
    if (device < 0 || device >= 64) return fail(DMHIP_ERR_NO_DEVICE, "device %d is outside 0..63", device);
    // Every code object of the library is loaded onto the device here, at
    // set-up: the runtime loads one (and allocates its device memory) when
    // one of its kernels is first resolved, which must not happen inside an
    // allocation-free call.
    for (const void *anchor : {module_anchor_simple(), module_anchor_qmv(), module_anchor_qmv8(),
                               module_anchor_gemm(), module_anchor_expert(), module_anchor_dense(),
                               module_anchor_attention(), module_anchor_safetensor()}) {
        hipFuncAttributes attr;
        DM_HIP(hipFuncGetAttributes(&attr, anchor));
    }
    if (g_scratch_address[device].load(std::memory_order_acquire)) return DMHIP_OK;
    void *ptr = nullptr;
    DM_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) return fail(DMHIP_ERR_COMMAND, "no device address for the allocation-free scratch on device %d", device);
    g_scratch_address[device].store(ptr, std::memory_order_release);
    return DMHIP_OK;
}

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
    if (type == 8 && batch > 1 && qmv_supported(type, rows, columns, w, 1)) {
        // Q8_0 (8) has only the int8 kernel (1-4 tokens, fewer on long rows):
        // one launch per group of tokens, each streaming the matrix at HBM
        // rate, beats the exact per-element kernel by an order of magnitude.
        size_t per = 4;
        while (per > 1 && !qmv_supported(type, rows, columns, w, per)) per /= 2;
        for (size_t t = 0; t < batch; t += per) {
            const uint32_t n = batch - t < per ? (uint32_t)(batch - t) : (uint32_t)per;
            DM_HIP(launch_qmv(ctx, type, (uint32_t)rows, (uint32_t)columns, w, n, x + t * columns, y + t * rows,
                              nullptr, nullptr));
        }
        return DMHIP_OK;
    }
    if (dense_supported(type, rows, columns, w, x, batch)) {
        DM_HIP(launch_dense_gemv(ctx->stream, ctx->compute_units, type, w, (uint32_t)rows, (uint32_t)columns,
                                 (size_t)row_bytes, (uint32_t)batch, x, y));
        return DMHIP_OK;
    }
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

size_t dmhip_ffn_noalloc_scratch_bytes(void) { return dm::kNoAllocScratchBytes; }

int dmhip_ffn_device_noalloc(dmhip_ctx *ctx, size_t batch, size_t hidden, size_t ffn, uint32_t gate_type,
                             const void *gate, uint32_t up_type, const void *up, uint32_t down_type,
                             const void *down, float epsilon, const float *h, float *y) {
    if (!ctx) return fail(DMHIP_ERR_INVALID_ARGUMENT, "ctx must not be null");
    if (batch < 1 || batch > 16)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "batch %zu is outside 1..=16", batch);
    const size_t ws = dmhip_ffn_workspace_bytes(batch, hidden, ffn);
    // batches above 2 prepare activation fragments of h (gate and up, whose
    // types may differ and need different fragment sets) and of the
    // activation rows (down); the largest of the three regions is lent
    size_t lend = 0;
    if (batch > 2) {
        const uint32_t types[3] = {gate_type, up_type, down_type};
        const size_t cols[3] = {hidden, hidden, ffn};
        for (int i = 0; i < 3; i++) {
            const size_t b = qmv_prepare_bytes(types[i], cols[i], batch);
            lend = b > lend ? b : lend;
        }
    }
    if (ws == 0 || ws > kNoAllocScratchBytes || lend > kNoAllocScratchBytes - ws)
        return fail(DMHIP_ERR_INVALID_ARGUMENT,
                    "FFN of batch %zu, hidden %zu, ffn %zu needs %zu scratch bytes; the allocation-free entry "
                    "point holds %zu",
                    batch, hidden, ffn, ws + lend, kNoAllocScratchBytes);
    const int device = ctx->device;
    void *base = (device >= 0 && device < 64) ? g_scratch_address[device].load(std::memory_order_acquire) : nullptr;
    if (!base) return fail(DMHIP_ERR_COMMAND, "the allocation-free scratch of device %d is not resolved", device);
    // the fp16 path's fragments go to the lent region for this call only
    struct Lend {
        dmhip_ctx *c;
        ~Lend() {
            c->aux_lent = nullptr;
            c->aux_lent_bytes = 0;
        }
    } guard{ctx};
    ctx->aux_lent = batch > 2 ? (char *)base + ws : nullptr;
    ctx->aux_lent_bytes = batch > 2 ? lend : 0;
    return dmhip_ffn_device(ctx, batch, hidden, ffn, gate_type, gate, up_type, up, down_type, down, epsilon, h, y,
                           base, ws);
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
