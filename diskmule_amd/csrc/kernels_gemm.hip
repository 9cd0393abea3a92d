// kernels_gemm.hip -- prefill GEMM C[m][n] = sum_k A[m][k] * W[n][k].
//
// A is bf16 activations [m][k]; W is n encoded rows of k columns.  The
// reference has no batched prefill: it runs one matvec per token
// (src/gemma4/metal.rs:514-536), so the result for token m must match
// cpu::matvec(W, widen(A[m])) (src/cpu.rs:345-399) within fp32 tolerance.
#include "runtime.h"

#include "dm_qmv.h"

namespace dm {

__global__ void bf16_to_f32_kernel(const uint16_t *__restrict__ a, size_t count, float *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = __uint_as_float((uint32_t)a[i] << 16);
}

}  // namespace dm

using namespace dm;

extern "C" {

size_t dmhip_gemm_workspace_bytes(size_t m, size_t k) { return m * k * sizeof(float) + 256; }

int dmhip_gemm_device(dmhip_ctx *ctx, uint32_t type, size_t m, size_t n, size_t k,
                      const uint16_t *a_bf16, const void *weights, float *c, void *workspace) {
    if (!ctx || !a_bf16 || !weights || !c || !workspace)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "gemm arguments must not be null");
    if (!(type == 0 || type == 1 || type == 6 || type == 8 || type == 12 || type == 14))
        return fail(DMHIP_ERR_UNSUPPORTED_TENSOR_TYPE, "HIP GEMM does not support %s", type_name(type));
    uint64_t rb;
    if (!row_byte_len(type, k, &rb))
        return fail(DMHIP_ERR_INVALID_ELEMENT_COUNT, "%s row of %zu values is not whole blocks",
                    type_name(type), k);
    if (m == 0 || n == 0) return DMHIP_OK;
    if (k == 0) return fail(DMHIP_ERR_EMPTY_INPUT, "gemm requires a non-empty input");
    if (m > 0xffffffffull || n > 0xffffffffull || k > 0xffffffffull)
        return fail(DMHIP_ERR_VECTOR_TOO_LARGE, "HIP vector length exceeds the 32-bit kernel limit");
    DM_CHECK_STATUS(set_device(ctx));
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
