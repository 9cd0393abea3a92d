// runtime.h -- host-side state behind the dmhip C ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "../../include/dmhip.h"
#include "dm_kernels.h"

namespace dm {

// Records `code` with a formatted message as the calling thread's last error
// (its payload reset to the bare status).
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// The calling thread's last failure payload.
dmhip_error_detail &last_detail();
// Failures that carry a payload: the reference's message text and fields.
// `operation` / `argument` must be static strings.
int fail_alloc(size_t bytes);
int fail_empty(const char *operation);
int fail_vector_length(const char *operation, const char *argument, size_t expected, size_t actual);
int fail_positive(const char *operation);
int fail_non_finite(const char *operation);
int fail_unsupported(uint32_t type, const char *what);  // "<what> does not support <type>"
int fail_element_count(uint32_t type, uint64_t elements);
int fail_byte_length(uint32_t type, uint64_t expected, uint64_t actual);
int fail_input_length(size_t expected, size_t actual);
int fail_output_length(size_t expected, size_t actual);
int fail_top_k(size_t k, size_t length);
int fail_mapped_range(size_t offset, size_t end, size_t length);
int fail_layer(size_t layer, size_t count);
int fail_expert(size_t layer, size_t expert, size_t count);
int fail_pinned(size_t layer);
int fail_io(int os_error);  // 0: unexpected end of file
// Maps a HIP runtime error onto DMHIP_ERR_COMMAND (MetalError::Command).
int hip_fail(hipError_t e, const char *what);

#define DM_HIP(call)                                      \
    do {                                                  \
        hipError_t dm_e_ = (call);                        \
        if (dm_e_ != hipSuccess) return dm::hip_fail(dm_e_, #call); \
    } while (0)

#define DM_CHECK_STATUS(expr)               \
    do {                                    \
        int dm_s_ = (expr);                 \
        if (dm_s_ != DMHIP_OK) return dm_s_; \
    } while (0)

// Device allocation that grows on demand (scratch for the host-slice API),
// used by work on `stream`: replacing or freeing it first waits for that
// stream (no stream: the caller has already waited for its users).
struct Scratch {
    void *ptr = nullptr;
    size_t bytes = 0;
    hipStream_t stream = nullptr;
    int ensure(size_t need);
    void release();
};

// Pinned host memory that the synchronous host-slice calls stage their
// inputs and outputs through: one memcpy into it and one DMA copy each way,
// instead of the runtime's pageable copy path.  Every call that uses it waits
// for its stream before returning, so no copy out of it is in flight when it
// is refilled or replaced.
struct HostBounce {
    void *ptr = nullptr;
    size_t bytes = 0;
    int ensure(size_t need);
    void release();
};
// Inputs and outputs of one host-slice call up to this size go through the
// bounce buffer; larger ones (the unmapped matvec's whole matrix) keep the
// runtime's path.
constexpr size_t kHostBounceMax = 8u << 20;

// (block elements, block bytes) of a ggml type, src/gguf.rs:321-342.
bool type_layout(uint32_t type, uint32_t *block_elements, uint32_t *block_bytes);
const char *type_name(uint32_t type);
// TensorType::row_byte_len (src/gguf.rs:352-358); false when not a whole
// number of blocks.
bool row_byte_len(uint32_t type, uint64_t elements, uint64_t *out);

}  // namespace dm

struct dmhip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipStream_t upload = nullptr;
    // A second upload stream: two host->HBM copies in flight at once move
    // about 52 GB/s over PCIe where one stream moves 42 GB/s.
    hipStream_t upload2 = nullptr;
    uint32_t upload_next = 0;
    char name[256] = {0};
    int compute_units = 0;
    dm::Scratch in, out, enc, aux;          // host-slice staging
    dm::HostBounce bounce;                   // pinned host side of the host-slice copies
    dm::Scratch partials;                    // per-wave argmax candidates
    dm::Scratch attn;                        // attention chunk partials
    dm::Scratch attn_tickets;                // attention combine counters, zero between calls
    size_t attn_ticket_count = 0;            // counters in attn_tickets already zeroed
    // Device memory an allocation-free call lends the fp16 path in place of
    // `aux` for its duration (null otherwise).
    void *aux_lent = nullptr;
    size_t aux_lent_bytes = 0;
    dm::ArgmaxState *argmax_state = nullptr;  // device
    uint32_t *router_tickets = nullptr;       // device, kRouterTickets counters, zero between launches
    uint32_t router_mark = 0;                 // mark of the pending device router calls (BadFlag), never 0 once set
    uint32_t attn_mark = 0;                   // mark of the last attention call (flags[kAttnFlagWord])
    uint32_t *argmax_ticket = nullptr;        // device, zero between launches: ticket, then (at +8) the best key
    uint32_t *argmax_index = nullptr;         // device
    uint32_t *flags = nullptr;                // device: [0] router, [1] read probe, [2] top-k, [3] MoE router, [4] attention
    bool argmax_pending = false;
    bool router_pending = false;  // a dmhip_router_top_k_device awaits dmhip_router_result
    bool attn_pending = false;    // a dmhip_attention_cached_device awaits dmhip_attention_result
    uint32_t *argmax_user_index = nullptr;
    // Pinned word the stream writes a call's sequence number into once the
    // call's work is done (stream_wait), and its device address.
    volatile uint32_t *done_word = nullptr;
    void *done_word_dev = nullptr;
    uint32_t done_seq = 0;
};

struct dmhip_buf {
    dmhip_ctx *ctx = nullptr;
    int device = 0;
    void *dev = nullptr;
    size_t len = 0;
    // Owned by an expert cache (a slot's gate_up or down bytes):
    // dmhip_buffer_free leaves it alone; the cache frees it.
    bool cache_owned = false;
};

namespace dm {
constexpr uint32_t kAttnFlagWord = 4;
// flags word the MoE layer's router writes (a sink: the layer reads its
// per-token words on the host), apart from the device router's word 0
constexpr uint32_t kMoeFlagWord = 3;
// Enqueue y = W x on the context stream, choosing the fastest kernel that
// takes the shape.  Arguments are already validated.
int enqueue_matvec(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns, const void *w,
                   size_t batch, const float *x, float *y);
int enqueue_matvec_argmax(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns,
                          const void *w, const float *x, float *y, uint32_t *index_device);
int set_device(dmhip_ctx *ctx);
// Waits until the work enqueued so far on the context's stream is done: the
// stream writes a sequence number into a pinned word, which the host polls
// for a while before it falls back to hipStreamSynchronize.
int stream_wait(dmhip_ctx *ctx);

// The copies of one synchronous host-slice call.  begin(total) sizes the
// call's inputs and outputs together: up to kHostBounceMax they are staged in
// the context's pinned bounce buffer (in() copies the host data into it and
// enqueues the DMA; out() enqueues the DMA into it and finish() copies it to
// the caller after waiting for the stream); above that, the host pointers go
// to the runtime directly.  finish() always waits for the stream, and a call
// that returns early (an error after its first copy) waits in the
// destructor, so no copy out of the bounce buffer outlives the call.
struct HostCall {
    dmhip_ctx *ctx;
    bool staged = false;
    bool open = false;
    size_t used = 0;
    struct Pending {
        void *dst;
        const void *src;
        size_t n;
    } pending[2];
    int outs = 0;
    bool pageable_out = false;  // an output copied straight into pageable memory
    explicit HostCall(dmhip_ctx *c) : ctx(c) {}
    ~HostCall();
    HostCall(const HostCall &) = delete;
    HostCall &operator=(const HostCall &) = delete;
    int begin(size_t total);
    int in(void *device_dst, const void *host_src, size_t n);
    int out(void *host_dst, const void *device_src, size_t n);
    // A place in the pinned bounce buffer where kernels may write an output
    // of n bytes directly (no device-to-host copy), handed to host_dst at
    // finish(); nullptr when the call is not staged (then use out()).
    void *out_direct(void *host_dst, size_t n);
    int finish();
};

// Resolves (once per device, with that device current) the device address of
// the allocation-free FFN's scratch array.
int noalloc_resolve(int device);

// Launches `kernel` on the context's stream.
template <typename F, typename... Args>
hipError_t launch_kernel(dmhip_ctx *ctx, F kernel, dim3 grid, dim3 block, uint32_t lds, Args... args) {
    hipLaunchKernelGGL(kernel, grid, block, lds, ctx->stream, args...);
    return hipGetLastError();
}
}  // namespace dm
