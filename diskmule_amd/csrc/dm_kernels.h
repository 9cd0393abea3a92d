// dm_kernels.h -- launchers of the gfx950 kernels (host-callable).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>

namespace dm {

constexpr uint32_t kMaxTopK = 256;

// A kernel's dynamic-LDS limit per device: raised to the size a launch asks
// for when that exceeds what was set on the device before (the attribute
// belongs to each device's copy of the code object).  Safe to share between
// threads (one instance per kernel, as a function-local static).
struct LdsLimit {
    std::atomic<uint32_t> set[64] = {};  // bytes allowed on device d (0..63)
    hipError_t ensure(const void *kernel, size_t bytes) {
        int device = 0;
        hipError_t e = hipGetDevice(&device);
        if (e != hipSuccess) return e;
        const bool cached = device >= 0 && device < 64;
        if (cached && set[device].load(std::memory_order_acquire) >= bytes) return hipSuccess;
        e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
        if (e != hipSuccess || !cached) return e;
        uint32_t have = set[device].load(std::memory_order_relaxed);
        while (have < bytes && !set[device].compare_exchange_weak(have, (uint32_t)bytes, std::memory_order_acq_rel)) {
        }
        return hipSuccess;
    }
};

// Device-side argmax accumulator: packed (ordered value, ~index) key and a
// non-finite flag.
struct ArgmaxState {
    unsigned long long key;
    uint32_t non_finite;
    uint32_t done;  // waves that have folded their key in (fused argmax)
};

// One kernel of each source file (each file is its own code object, which
// the runtime loads onto a device when one of its kernels is first used).
const void *module_anchor_simple();
const void *module_anchor_qmv();
const void *module_anchor_qmv8();
const void *module_anchor_gemm();
const void *module_anchor_dense();
// GEMV over F32 / F16 rows (whole 16-byte chunks, 16-byte aligned) and Q5_0
// rows (whole 64-value pairs of blocks, dword aligned), up to 64 KiB of
// activations per group of 4 tokens (kernels_dense.hip).
bool dense_supported(uint32_t type, size_t rows, size_t columns, const void *w, const float *x, size_t batch);
hipError_t launch_dense_gemv(hipStream_t s, int cus, uint32_t type, const void *w, uint32_t rows, uint32_t columns,
                             size_t row_bytes, uint32_t batch, const float *x, float *y);
const void *module_anchor_expert();
const void *module_anchor_attention();
const void *module_anchor_safetensor();

// GLM safetensors GEMV formats (kernels_safetensor.hip).
constexpr uint32_t kStBf16 = 0, kStF8 = 1, kStI8 = 2, kStI4 = 3;
// The wide-load form: 16-byte aligned W and x, whole 16-byte chunks per row,
// at most 16384 columns (the activation in LDS), INT4 groups of 16 or a
// multiple of 32.
bool st_wide_supported(uint32_t fmt, size_t rows, size_t columns, size_t group, const void *w, const float *x);
hipError_t launch_st_gemv(hipStream_t s, int cus, uint32_t fmt, const void *w, uint32_t rows, uint32_t columns,
                          const float *scales, uint32_t scale_columns, uint32_t group, const float *x, float *y,
                          bool wide);

hipError_t launch_copy_bytes(hipStream_t s, void *dst, const void *src, size_t n);
hipError_t launch_dequantize(hipStream_t s, uint32_t type, const uint8_t *enc, uint32_t be,
                             uint32_t bb, size_t elements, float *out);
hipError_t launch_gemv_exact(hipStream_t s, uint32_t type, uint32_t be, uint32_t bb, uint32_t rows,
                             uint32_t columns, size_t row_bytes, const uint8_t *w, uint32_t batch,
                             const float *x, float *y);
hipError_t launch_argmax(hipStream_t s, const float *v, size_t n, ArgmaxState *state,
                         uint32_t *index);
hipError_t launch_argmax_init(hipStream_t s, ArgmaxState *state);
hipError_t launch_argmax_finish(hipStream_t s, const ArgmaxState *state, uint32_t *index);
// Where a selection kernel records a row with a non-finite logit: it stores
// `mark` into *word.  A caller that checks the word after each call gives
// each call a new nonzero mark, so the word needs no reset between calls (a
// stale word equals the current mark only after 2^32 calls).
struct BadFlag {
    uint32_t *word;
    uint32_t mark;
};
hipError_t launch_top_k(hipStream_t s, const float *logits, uint32_t rows, uint32_t count,
                        uint32_t k, uint32_t *ids, float *probabilities, BadFlag non_finite);
// The routed experts' slots looked up on the device, for a MoE layer call
// of up to kMaxLookupTokens tokens whose expert launches are queued behind
// the router: per expert of the layer the device addresses of its slot's
// gate_up and down bytes (0 when not resident); out, per selection s of
// token t, the addresses at [t * k + s], and per token a go word (device and
// pinned host copies): 1 when every selected expert of the token is resident
// and its logits are finite, else 0.
constexpr uint32_t kMaxLookupTokens = 8;
struct ExpertLookup {
    const uint64_t *gate_up_of, *down_of;
    uint64_t *gate_up_w, *down_w;
    uint32_t *go, *host_go;
};
hipError_t launch_router_top_k(hipStream_t s, const uint16_t *router, uint32_t hidden,
                               uint32_t experts, uint32_t k, uint32_t batch, const float *x,
                               float *logits, uint32_t *ids, float *probabilities,
                               BadFlag non_finite, uint32_t *host_ids = nullptr,
                               float *host_probs = nullptr, uint32_t *tickets = nullptr,
                               uint32_t *host_bad = nullptr, const ExpertLookup *lookup = nullptr,
                               bool certified = false);
// With `certified` (the MoE layer, whose logits stay internal) and tickets,
// decode batches of up to 8192 columns take the certified router: the same
// ids in the same order as the exact fold, probabilities from logits within
// a proven bound of it; `logits` then holds 8 bytes per (token, expert).
// True when launch_router_top_k takes a lookup for this router: up to
// kMaxLookupTokens tokens, and the router runs as one of the
// expert-parallel kernels whose token's last workgroup makes the selection.
bool router_takes_lookup(uint32_t hidden, uint32_t experts, uint32_t batch, const void *router, const float *x);
// With host_ids, the selection and one word per token (nonzero when that
// token's logits held a non-finite value; with the one-workgroup-per-token
// fallback kernel word 0 stands for all tokens) are written to host memory.
// p[0..n) = value, stream-ordered (a kernel, so that callers may capture it
// in a graph).
hipError_t launch_fill_u32(hipStream_t s, uint32_t *p, uint32_t n, uint32_t value);
// Per-token counters of the fused router selection (zero between launches).
constexpr uint32_t kRouterTickets = 4096;
hipError_t launch_rms_norm(hipStream_t s, const float *in, uint32_t batch, uint32_t n,
                           const float *weight, float eps, float *out);
hipError_t launch_silu_mul(hipStream_t s, const float *gate, const float *up, size_t n, float *out);
hipError_t launch_softcap(hipStream_t s, const float *in, size_t n, float cap, float *out);
hipError_t launch_add(hipStream_t s, const float *a, const float *b, size_t n, float *out);
hipError_t launch_gelu_mul(hipStream_t s, const float *gate, const float *up, size_t n, float *out);
hipError_t launch_softmax(hipStream_t s, const float *in, uint32_t n, float *out);
hipError_t launch_rope_neox(hipStream_t s, float *v, size_t heads, uint32_t head_dim, uint32_t pairs,
                            uint32_t position, float theta);
hipError_t launch_moe_combine(hipStream_t s, const float *expert_out, const float *p, uint32_t batch,
                              uint32_t k, uint32_t hidden, float *y);
hipError_t launch_silu_mul_glm_pairs(hipStream_t s, const float *gate_up, uint32_t pairs,
                                     uint32_t width, float *act);

}  // namespace dm
