// runtime.hip -- context, buffers and operators behind include/dmhip.h.
//
// Host-slice entry points follow src/metal.rs: validate everything first
// (same checks, same order, same error variants), then copy inputs in, run
// the kernels on the context's stream, wait and copy results out.
#include "runtime.h"
#include "dm_qmv.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

#include <chrono>
#include <string>

namespace dm {

static thread_local std::string g_last_error;
static thread_local dmhip_error_detail g_last_detail;

int fail(int code, const char *fmt, ...) {
    char buffer[512];
    va_list args;
    va_start(args, fmt);
    vsnprintf(buffer, sizeof buffer, fmt, args);
    va_end(args);
    g_last_error = buffer;
    g_last_detail = dmhip_error_detail{};
    g_last_detail.status = code;
    return code;
}

dmhip_error_detail &last_detail() { return g_last_detail; }

int fail_alloc(size_t bytes) {
    fail(DMHIP_ERR_BUFFER_ALLOCATION, "could not allocate a %zu-byte device buffer", bytes);
    g_last_detail.bytes = bytes;
    return DMHIP_ERR_BUFFER_ALLOCATION;
}

int fail_empty(const char *operation) {
    fail(DMHIP_ERR_EMPTY_INPUT, "%s requires a non-empty input", operation);
    g_last_detail.operation = operation;
    return DMHIP_ERR_EMPTY_INPUT;
}

int fail_vector_length(const char *operation, const char *argument, size_t expected, size_t actual) {
    fail(DMHIP_ERR_INVALID_VECTOR_LENGTH, "%s %s has length %zu; expected %zu", operation, argument, actual,
         expected);
    g_last_detail.operation = operation;
    g_last_detail.argument = argument;
    g_last_detail.expected = expected;
    g_last_detail.actual = actual;
    return DMHIP_ERR_INVALID_VECTOR_LENGTH;
}

int fail_positive(const char *operation) {
    fail(DMHIP_ERR_INVALID_POSITIVE_PARAMETER, "%s requires a finite positive parameter", operation);
    g_last_detail.operation = operation;
    return DMHIP_ERR_INVALID_POSITIVE_PARAMETER;
}

int fail_non_finite(const char *operation) {
    fail(DMHIP_ERR_NON_FINITE, "%s received a non-finite value", operation);
    g_last_detail.operation = operation;
    return DMHIP_ERR_NON_FINITE;
}

int fail_unsupported(uint32_t type, const char *what) {
    fail(DMHIP_ERR_UNSUPPORTED_TENSOR_TYPE, "%s does not support %s", what, type_name(type));
    g_last_detail.kind = type_name(type);
    return DMHIP_ERR_UNSUPPORTED_TENSOR_TYPE;
}

int fail_element_count(uint32_t type, uint64_t elements) {
    uint32_t be = 0, bb = 0;
    type_layout(type, &be, &bb);
    fail(DMHIP_ERR_INVALID_ELEMENT_COUNT, "%s output length %llu is not divisible by its %u-element block",
         type_name(type), (unsigned long long)elements, be);
    g_last_detail.kind = type_name(type);
    g_last_detail.elements = elements;
    g_last_detail.block_elements = be;
    return DMHIP_ERR_INVALID_ELEMENT_COUNT;
}

int fail_byte_length(uint32_t type, uint64_t expected, uint64_t actual) {
    fail(DMHIP_ERR_INVALID_BYTE_LENGTH, "%s requires %llu encoded bytes, got %llu", type_name(type),
         (unsigned long long)expected, (unsigned long long)actual);
    g_last_detail.kind = type_name(type);
    g_last_detail.expected = expected;
    g_last_detail.actual = actual;
    return DMHIP_ERR_INVALID_BYTE_LENGTH;
}

int fail_input_length(size_t expected, size_t actual) {
    fail(DMHIP_ERR_INVALID_INPUT_LENGTH, "matvec input has %zu columns; expected %zu", actual, expected);
    g_last_detail.expected = expected;
    g_last_detail.actual = actual;
    return DMHIP_ERR_INVALID_INPUT_LENGTH;
}

int fail_output_length(size_t expected, size_t actual) {
    fail(DMHIP_ERR_INVALID_OUTPUT_LENGTH, "matvec output has %zu rows; expected %zu", actual, expected);
    g_last_detail.expected = expected;
    g_last_detail.actual = actual;
    return DMHIP_ERR_INVALID_OUTPUT_LENGTH;
}

int fail_top_k(size_t k, size_t length) {
    fail(DMHIP_ERR_INVALID_TOP_K, "top-k count %zu is outside 1..=%zu", k, length);
    g_last_detail.k = k;
    g_last_detail.length = length;
    return DMHIP_ERR_INVALID_TOP_K;
}

int fail_mapped_range(size_t offset, size_t end, size_t length) {
    fail(DMHIP_ERR_MAPPED_RANGE, "mapped buffer range %zu..%zu exceeds its %zu-byte file mapping", offset, end,
         length);
    g_last_detail.offset = offset;
    g_last_detail.end = end;
    g_last_detail.length = length;
    return DMHIP_ERR_MAPPED_RANGE;
}

int fail_layer(size_t layer, size_t count) {
    fail(DMHIP_ERR_INVALID_LAYER, "expert cache layer %zu is outside its %zu layers", layer, count);
    g_last_detail.layer = layer;
    g_last_detail.count = count;
    return DMHIP_ERR_INVALID_LAYER;
}

int fail_expert(size_t layer, size_t expert, size_t count) {
    fail(DMHIP_ERR_INVALID_EXPERT, "expert %zu is outside layer %zu's %zu experts", expert, layer, count);
    g_last_detail.layer = layer;
    g_last_detail.expert = expert;
    g_last_detail.count = count;
    return DMHIP_ERR_INVALID_EXPERT;
}

int fail_pinned(size_t layer) {
    fail(DMHIP_ERR_ALL_SLOTS_PINNED, "all expert slots in layer %zu are pinned by in-flight work", layer);
    g_last_detail.layer = layer;
    return DMHIP_ERR_ALL_SLOTS_PINNED;
}

int fail_io(int os_error) {
    if (os_error)
        fail(DMHIP_ERR_IO, "%s", strerror(os_error));
    else
        fail(DMHIP_ERR_IO, "failed to fill whole buffer");
    g_last_detail.os_error = os_error;
    return DMHIP_ERR_IO;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(DMHIP_ERR_COMMAND, "HIP command failed: %s: %s", what, hipGetErrorString(e));
}

int Scratch::ensure(size_t need) {
    if (need <= bytes) return DMHIP_OK;
    release();
    size_t grow = need < 4096 ? 4096 : need;
    hipError_t e = hipMalloc(&ptr, grow + 256);
    if (e != hipSuccess) {
        ptr = nullptr;
        return fail_alloc(need);
    }
    bytes = grow;
    return DMHIP_OK;
}

void Scratch::release() {
    // Work already enqueued on the stream may still read the old allocation.
    if (ptr && stream) (void)hipStreamSynchronize(stream);
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
}

int HostBounce::ensure(size_t need) {
    if (need <= bytes) return DMHIP_OK;
    release();
    size_t grow = 64u << 10;
    while (grow < need) grow *= 2;
    if (hipHostMalloc(&ptr, grow, hipHostMallocDefault) != hipSuccess) {
        ptr = nullptr;
        return fail_alloc(need);
    }
    bytes = grow;
    return DMHIP_OK;
}

void HostBounce::release() {
    if (ptr) (void)hipHostFree(ptr);
    ptr = nullptr;
    bytes = 0;
}

HostCall::~HostCall() {
    if (open) (void)hipStreamSynchronize(ctx->stream);
}

int HostCall::begin(size_t total) {
    staged = total <= kHostBounceMax;
    used = 0;
    outs = 0;
    pageable_out = false;
    open = true;
    // room for the 256-byte alignment of up to four pieces
    return staged ? ctx->bounce.ensure(total + 4 * 256) : DMHIP_OK;
}

int HostCall::in(void *device_dst, const void *host_src, size_t n) {
    if (n == 0) return DMHIP_OK;
    if (!staged) {
        DM_HIP(hipMemcpyAsync(device_dst, host_src, n, hipMemcpyHostToDevice, ctx->stream));
        return DMHIP_OK;
    }
    char *b = (char *)ctx->bounce.ptr + used;
    used += (n + 255) & ~(size_t)255;
    memcpy(b, host_src, n);
    DM_HIP(hipMemcpyAsync(device_dst, b, n, hipMemcpyHostToDevice, ctx->stream));
    return DMHIP_OK;
}

int HostCall::out(void *host_dst, const void *device_src, size_t n) {
    if (n == 0) return DMHIP_OK;
    if (!staged) {
        DM_HIP(hipMemcpyAsync(host_dst, device_src, n, hipMemcpyDeviceToHost, ctx->stream));
        pageable_out = true;
        return DMHIP_OK;
    }
    if (outs == 2) return fail(DMHIP_ERR_COMMAND, "a host-slice call stages at most two outputs");
    char *b = (char *)ctx->bounce.ptr + used;
    used += (n + 255) & ~(size_t)255;
    DM_HIP(hipMemcpyAsync(b, device_src, n, hipMemcpyDeviceToHost, ctx->stream));
    pending[outs++] = Pending{host_dst, b, n};
    return DMHIP_OK;
}

void *HostCall::out_direct(void *host_dst, size_t n) {
    if (!staged || n == 0 || outs == 2) return nullptr;
    char *b = (char *)ctx->bounce.ptr + used;
    used += (n + 255) & ~(size_t)255;
    pending[outs++] = Pending{host_dst, b, n};
    return b;
}

int stream_wait(dmhip_ctx *ctx) {
    if (ctx->done_word) {
        const uint32_t v = ++ctx->done_seq;
        DM_HIP(hipStreamWriteValue32(ctx->stream, ctx->done_word_dev, v, 0));
        // A poll of the pinned word returns about 2 us sooner than
        // hipStreamSynchronize after a short kernel (MI355X: launch + wait
        // 9.4 against 11.7 us); long work falls back to the blocking wait.
        const auto deadline = std::chrono::steady_clock::now() + std::chrono::microseconds(2000);
        for (;;) {
            for (int i = 0; i < 64; i++)
                if (__atomic_load_n(ctx->done_word, __ATOMIC_ACQUIRE) == v) return DMHIP_OK;
            if (std::chrono::steady_clock::now() > deadline) break;
        }
    }
    DM_HIP(hipStreamSynchronize(ctx->stream));
    return DMHIP_OK;
}

int HostCall::finish() {
    open = false;
    // a copy into pageable memory is waited for by the blocking synchronisation
    if (pageable_out) {
        pageable_out = false;
        DM_HIP(hipStreamSynchronize(ctx->stream));
    } else {
        DM_CHECK_STATUS(stream_wait(ctx));
    }
    for (int i = 0; i < outs; i++) memcpy(pending[i].dst, pending[i].src, pending[i].n);
    outs = 0;
    return DMHIP_OK;
}

bool type_layout(uint32_t type, uint32_t *be, uint32_t *bb) {
    switch (type) {
    case 0: *be = 1; *bb = 4; return true;      // F32
    case 1: *be = 1; *bb = 2; return true;      // F16
    case 30: *be = 1; *bb = 2; return true;     // BF16
    case 2: *be = 32; *bb = 18; return true;    // Q4_0
    case 3: *be = 32; *bb = 20; return true;    // Q4_1
    case 6: *be = 32; *bb = 22; return true;    // Q5_0
    case 7: *be = 32; *bb = 24; return true;    // Q5_1
    case 8: *be = 32; *bb = 34; return true;    // Q8_0
    case 9: *be = 32; *bb = 40; return true;    // Q8_1
    case 10: *be = 256; *bb = 84; return true;  // Q2_K
    case 11: *be = 256; *bb = 110; return true; // Q3_K
    case 12: *be = 256; *bb = 144; return true; // Q4_K
    case 13: *be = 256; *bb = 176; return true; // Q5_K
    case 14: *be = 256; *bb = 210; return true; // Q6_K
    case 15: *be = 256; *bb = 292; return true; // Q8_K
    case 24: *be = 1; *bb = 1; return true;     // I8
    case 25: *be = 1; *bb = 2; return true;     // I16
    case 26: *be = 1; *bb = 4; return true;     // I32
    case 27: case 28: *be = 1; *bb = 8; return true;  // I64, F64
    default: return false;
    }
}

const char *type_name(uint32_t type) {
    switch (type) {
    case 0: return "F32"; case 1: return "F16"; case 2: return "Q4_0"; case 3: return "Q4_1";
    case 6: return "Q5_0"; case 7: return "Q5_1"; case 8: return "Q8_0"; case 9: return "Q8_1";
    case 10: return "Q2_K"; case 11: return "Q3_K"; case 12: return "Q4_K"; case 13: return "Q5_K";
    case 14: return "Q6_K"; case 15: return "Q8_K"; case 24: return "I8"; case 25: return "I16";
    case 26: return "I32"; case 27: return "I64"; case 28: return "F64"; case 30: return "BF16";
    default: return "unknown";
    }
}

bool row_byte_len(uint32_t type, uint64_t elements, uint64_t *out) {
    uint32_t be, bb;
    if (!type_layout(type, &be, &bb)) return false;
    if (elements % be) return false;
    uint64_t blocks = elements / be;
    if (blocks > UINT64_MAX / bb) return false;
    *out = blocks * bb;
    return true;
}

int set_device(dmhip_ctx *ctx) {
    DM_HIP(hipSetDevice(ctx->device));
    return DMHIP_OK;
}

static bool matvec_kind_supported(uint32_t type) {
    // The pipelines of MetalContext::prepare_matvec (src/metal.rs:1534-1542).
    return type == 0 || type == 1 || type == 6 || type == 8 || type == 12 || type == 14;
}

// MetalContext::prepare_matvec (src/metal.rs:1513-1560), same order of checks.
static int prepare_matvec(uint32_t type, size_t rows, size_t columns, size_t encoded_length,
                          size_t input_len, size_t output_len, size_t *row_bytes_out) {
    if (input_len != columns) return fail_input_length(columns, input_len);
    if (output_len != rows) return fail_output_length(rows, output_len);
    if (!matvec_kind_supported(type)) return fail_unsupported(type, "HIP matrix-vector multiplication");
    uint64_t row_bytes;
    if (!row_byte_len(type, columns, &row_bytes)) return fail_element_count(type, columns);
    if (rows != 0 && row_bytes > SIZE_MAX / rows)
        return fail(DMHIP_ERR_OVERFLOW, "matrix dimensions or encoded byte length overflowed");
    size_t matrix_bytes = rows * (size_t)row_bytes;
    if (encoded_length != matrix_bytes) return fail_byte_length(type, matrix_bytes, encoded_length);
    *row_bytes_out = (size_t)row_bytes;
    return DMHIP_OK;
}

static int count_u32(size_t n) {
    if (n > 0xffffffffull) return fail(DMHIP_ERR_VECTOR_TOO_LARGE, "HIP vector length exceeds the 32-bit kernel limit");
    return DMHIP_OK;
}

static int require_nonempty(const char *operation, size_t n) {
    if (n == 0) return fail_empty(operation);
    return DMHIP_OK;
}

static int validate_vector_length(const char *operation, const char *argument, size_t expected,
                                  size_t actual) {
    if (actual != expected) return fail_vector_length(operation, argument, expected, actual);
    return DMHIP_OK;
}

static int require_positive(const char *operation, float v) {
    if (!isfinite(v) || v <= 0.0f) return fail_positive(operation);
    return DMHIP_OK;
}

static bool all_finite(const float *v, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (!isfinite(v[i])) return false;
    return true;
}

// MetalError::VectorLength (src/metal.rs:29-34).
static int fail_vector_lengths(size_t left, size_t right, size_t output) {
    fail(DMHIP_ERR_VECTOR_LENGTH, "HIP vector lengths differ: left=%zu, right=%zu, output=%zu", left, right,
         output);
    g_last_detail.left = left;
    g_last_detail.right = right;
    g_last_detail.output = output;
    return DMHIP_ERR_VECTOR_LENGTH;
}

// rope_neox_in_place's checks in src/metal.rs:487-509's order, up to the
// no-op case: *noop is set when there is nothing to rotate.
static int check_rope(size_t values_len, size_t heads, size_t head_dimension, size_t rotated_pairs,
                      size_t position, float theta, bool *noop) {
    size_t length = 0;
    if (__builtin_mul_overflow(heads, head_dimension, &length) || length != values_len) {
        fail(DMHIP_ERR_INVALID_ROPE_SHAPE,
             "NeoX RoPE input length %zu does not match %zu heads of dimension %zu", values_len, heads,
             head_dimension);
        g_last_detail.length = values_len;
        g_last_detail.heads = heads;
        g_last_detail.head_dimension = head_dimension;
        return DMHIP_ERR_INVALID_ROPE_SHAPE;
    }
    if (head_dimension % 2 != 0 || rotated_pairs > head_dimension / 2)
        return fail(DMHIP_ERR_INVALID_ROPE_PAIRS,
                    "NeoX RoPE requires an even head dimension and at most half its dimensions as pairs");
    if (const int e = require_positive("NeoX RoPE theta", theta); e != DMHIP_OK) return e;
    *noop = rotated_pairs == 0 || heads == 0;
    if (*noop) return DMHIP_OK;
    size_t pairs = 0;
    if (__builtin_mul_overflow(heads, rotated_pairs, &pairs))
        return fail(DMHIP_ERR_VECTOR_TOO_LARGE, "HIP vector length exceeds the 32-bit kernel limit");
    if (const int e = count_u32(head_dimension); e != DMHIP_OK) return e;
    if (const int e = count_u32(rotated_pairs); e != DMHIP_OK) return e;
    if (const int e = count_u32(position); e != DMHIP_OK) return e;
    return DMHIP_OK;
}

}  // namespace dm

using namespace dm;

#define DM_CHECK(expr)                    \
    do {                                  \
        int dm_s_ = (expr);               \
        if (dm_s_ != DMHIP_OK) return dm_s_; \
    } while (0)

#define DM_REQUIRE(ptr)                                                                 \
    do {                                                                                \
        if (!(ptr)) return fail(DMHIP_ERR_INVALID_ARGUMENT, "%s must not be null", #ptr); \
    } while (0)

extern "C" {

const char *dmhip_last_error(void) { return dm::g_last_error.c_str(); }

int dmhip_last_error_detail(dmhip_error_detail *out) {
    if (!out) return DMHIP_ERR_INVALID_ARGUMENT;
    *out = dm::g_last_detail;
    return DMHIP_OK;
}

int dmhip_context_new(int device, dmhip_ctx **out) {
    DM_REQUIRE(out);
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0 || device < 0 || device >= count)
        return fail(DMHIP_ERR_NO_DEVICE, "no HIP device %d is available", device);
    dmhip_ctx *ctx = new dmhip_ctx();
    ctx->device = device;
    hipDeviceProp_t prop;
    if (hipSetDevice(device) != hipSuccess || hipGetDeviceProperties(&prop, device) != hipSuccess) {
        delete ctx;
        return fail(DMHIP_ERR_NO_DEVICE, "HIP device %d did not answer", device);
    }
    // some runtimes report an empty marketing name: then the arch alone
    if (prop.name[0])
        snprintf(ctx->name, sizeof ctx->name, "%s (%s)", prop.name, prop.gcnArchName);
    else
        snprintf(ctx->name, sizeof ctx->name, "%s", prop.gcnArchName);
    ctx->compute_units = prop.multiProcessorCount;
    // Default-priority streams only.
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&ctx->upload, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&ctx->upload2, hipStreamNonBlocking) != hipSuccess ||
        hipMalloc((void **)&ctx->argmax_state, sizeof(ArgmaxState)) != hipSuccess ||
        hipMalloc((void **)&ctx->argmax_index, 64) != hipSuccess ||
        hipMalloc((void **)&ctx->flags, 64) != hipSuccess ||
        hipMalloc((void **)&ctx->argmax_ticket, 64) != hipSuccess ||
        hipMalloc((void **)&ctx->router_tickets, kRouterTickets * 4) != hipSuccess ||
        // Counters start at zero.  Cleared by the library's own fill kernel:
        // the first launch from the library's code object materialises its
        // data (the allocation-free entry point's scratch array) on this
        // device here, at set-up, rather than inside a later call.
        launch_fill_u32(ctx->stream, ctx->argmax_ticket, 16, 0) != hipSuccess ||
        launch_fill_u32(ctx->stream, ctx->router_tickets, kRouterTickets, 0) != hipSuccess ||
        launch_fill_u32(ctx->stream, ctx->flags, 16, 0) != hipSuccess ||
        hipHostMalloc((void **)&ctx->done_word, 64, hipHostMallocDefault) != hipSuccess ||
        hipHostGetDevicePointer(&ctx->done_word_dev, (void *)ctx->done_word, 0) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
        dmhip_context_free(ctx);
        return fail(DMHIP_ERR_COMMAND, "could not create the HIP streams of device %d", device);
    }
    *ctx->done_word = 0;  // sequence numbers start at 1
    for (Scratch *sc : {&ctx->in, &ctx->out, &ctx->enc, &ctx->aux, &ctx->partials, &ctx->attn, &ctx->attn_tickets})
        sc->stream = ctx->stream;
    const int resolved = noalloc_resolve(device);
    if (resolved != DMHIP_OK) {
        dmhip_context_free(ctx);
        return resolved;
    }
    *out = ctx;
    return DMHIP_OK;
}

void dmhip_context_free(dmhip_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->upload) (void)hipStreamSynchronize(ctx->upload);
    if (ctx->upload2) (void)hipStreamSynchronize(ctx->upload2);
    ctx->in.release();
    ctx->bounce.release();
    ctx->out.release();
    ctx->enc.release();
    ctx->aux.release();
    ctx->partials.release();
    ctx->attn.release();
    ctx->attn_tickets.release();
    if (ctx->argmax_state) (void)hipFree(ctx->argmax_state);
    if (ctx->argmax_ticket) (void)hipFree(ctx->argmax_ticket);
    if (ctx->router_tickets) (void)hipFree(ctx->router_tickets);
    if (ctx->argmax_index) (void)hipFree(ctx->argmax_index);
    if (ctx->flags) (void)hipFree(ctx->flags);
    if (ctx->done_word) (void)hipHostFree((void *)ctx->done_word);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    if (ctx->upload) (void)hipStreamDestroy(ctx->upload);
    if (ctx->upload2) (void)hipStreamDestroy(ctx->upload2);
    delete ctx;
}

int dmhip_device_name(dmhip_ctx *ctx, char *buffer, size_t capacity) {
    DM_REQUIRE(ctx);
    DM_REQUIRE(buffer);
    if (capacity == 0) return fail(DMHIP_ERR_INVALID_ARGUMENT, "capacity must not be zero");
    snprintf(buffer, capacity, "%s", ctx->name);
    return DMHIP_OK;
}

int dmhip_synchronize(dmhip_ctx *ctx) {
    DM_REQUIRE(ctx);
    DM_CHECK(set_device(ctx));
    DM_HIP(hipStreamSynchronize(ctx->upload));
    DM_HIP(hipStreamSynchronize(ctx->upload2));
    DM_HIP(hipStreamSynchronize(ctx->stream));
    return DMHIP_OK;
}

void *dmhip_stream(dmhip_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

// ---- buffers -------------------------------------------------------------

static int new_buffer(dmhip_ctx *ctx, size_t length, dmhip_buf **out) {
    dmhip_buf *b = new dmhip_buf();
    b->ctx = ctx;
    b->device = ctx->device;
    b->len = length;
    // 256 spare bytes: vector loads of the last row may read a few bytes past
    // its end (they are discarded); the spare keeps them inside the allocation.
    if (hipMalloc(&b->dev, length + 256) != hipSuccess) {
        delete b;
        return fail_alloc(length);
    }
    *out = b;
    return DMHIP_OK;
}

int dmhip_map_read_only(dmhip_ctx *ctx, const void *host, size_t length, dmhip_buf **out) {
    DM_REQUIRE(ctx);
    DM_REQUIRE(out);
    *out = nullptr;
    if (length == 0) return fail_alloc(0);
    DM_REQUIRE(host);
    DM_CHECK(set_device(ctx));
    dmhip_buf *b;
    DM_CHECK(new_buffer(ctx, length, &b));
    hipError_t e = hipMemcpyAsync(b->dev, host, length, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync((char *)b->dev + length, 0, 256, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        dmhip_buffer_free(b);
        return hip_fail(e, "map_read_only upload");
    }
    *out = b;
    return DMHIP_OK;
}

int dmhip_new_owned_buffer(dmhip_ctx *ctx, size_t length, dmhip_buf **out) {
    DM_REQUIRE(ctx);
    DM_REQUIRE(out);
    *out = nullptr;
    if (length == 0) return fail_alloc(0);
    DM_CHECK(set_device(ctx));
    dmhip_buf *b;
    DM_CHECK(new_buffer(ctx, length, &b));
    hipError_t e = hipMemsetAsync(b->dev, 0, length + 256, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        dmhip_buffer_free(b);
        return hip_fail(e, "new_owned_buffer clear");
    }
    *out = b;
    return DMHIP_OK;
}

void dmhip_buffer_free(dmhip_buf *b) {
    if (!b || b->cache_owned) return;
    // The context may already be gone; only the device id is needed.  hipFree
    // waits for work still using the allocation.
    (void)hipSetDevice(b->device);
    if (b->dev) (void)hipFree(b->dev);
    delete b;
}

size_t dmhip_buffer_len(const dmhip_buf *b) { return b ? b->len : 0; }
void *dmhip_buffer_device_ptr(const dmhip_buf *b) { return b ? b->dev : nullptr; }

static int check_range(const dmhip_buf *b, size_t offset, size_t n) {
    size_t end;
    if (__builtin_add_overflow(offset, n, &end))
        return fail(DMHIP_ERR_OVERFLOW, "matrix dimensions or encoded byte length overflowed");
    if (end > b->len) return fail_mapped_range(offset, end, b->len);
    return DMHIP_OK;
}

int dmhip_buffer_write(dmhip_ctx *ctx, dmhip_buf *b, size_t offset, const void *src, size_t n) {
    DM_REQUIRE(ctx);
    DM_REQUIRE(b);
    DM_CHECK(check_range(b, offset, n));
    if (n == 0) return DMHIP_OK;
    DM_REQUIRE(src);
    DM_CHECK(set_device(ctx));
    DM_HIP(hipMemcpyAsync((char *)b->dev + offset, src, n, hipMemcpyHostToDevice, ctx->stream));
    DM_HIP(hipStreamSynchronize(ctx->stream));
    return DMHIP_OK;
}

int dmhip_buffer_read(dmhip_ctx *ctx, const dmhip_buf *b, size_t offset, void *dst, size_t n) {
    DM_REQUIRE(ctx);
    DM_REQUIRE(b);
    DM_CHECK(check_range(b, offset, n));
    if (n == 0) return DMHIP_OK;
    DM_REQUIRE(dst);
    DM_CHECK(set_device(ctx));
    DM_HIP(hipMemcpyAsync(dst, (const char *)b->dev + offset, n, hipMemcpyDeviceToHost, ctx->stream));
    DM_HIP(hipStreamSynchronize(ctx->stream));
    return DMHIP_OK;
}

int dmhip_copy_to_host(dmhip_ctx *ctx, void *dst, const void *device_src, size_t n) {
    DM_REQUIRE(ctx);
    if (n == 0) return DMHIP_OK;
    DM_REQUIRE(dst);
    DM_REQUIRE(device_src);
    DM_CHECK(set_device(ctx));
    DM_HIP(hipMemcpyAsync(dst, device_src, n, hipMemcpyDeviceToHost, ctx->stream));
    DM_HIP(hipStreamSynchronize(ctx->stream));
    return DMHIP_OK;
}

int dmhip_copy_to_device(dmhip_ctx *ctx, void *device_dst, const void *src, size_t n) {
    DM_REQUIRE(ctx);
    if (n == 0) return DMHIP_OK;
    DM_REQUIRE(device_dst);
    DM_REQUIRE(src);
    DM_CHECK(set_device(ctx));
    DM_HIP(hipMemcpyAsync(device_dst, src, n, hipMemcpyHostToDevice, ctx->stream));
    DM_HIP(hipStreamSynchronize(ctx->stream));
    return DMHIP_OK;
}

int dmhip_host_alloc_pinned(size_t bytes, void **out) {
    DM_REQUIRE(out);
    *out = nullptr;
    if (bytes == 0) return fail_alloc(0);
    if (hipHostMalloc(out, bytes, hipHostMallocDefault) != hipSuccess) {
        *out = nullptr;
        return fail_alloc(bytes);
    }
    return DMHIP_OK;
}

void dmhip_host_free_pinned(void *p) {
    if (p) (void)hipHostFree(p);
}

// ---- synchronous host-slice operators --------------------------------------

int dmhip_rms_norm(dmhip_ctx *ctx, const float *input, size_t input_len, const float *weight,
                   size_t weight_len, float epsilon, float *output, size_t output_len) {
    DM_REQUIRE(ctx);
    DM_CHECK(require_nonempty("RMSNorm", input_len));
    DM_CHECK(validate_vector_length("RMSNorm", "output", input_len, output_len));
    if (weight) DM_CHECK(validate_vector_length("RMSNorm", "weight", input_len, weight_len));
    DM_CHECK(require_positive("RMSNorm epsilon", epsilon));
    DM_REQUIRE(input);
    DM_REQUIRE(output);
    if (!all_finite(input, input_len))
        return fail_non_finite("RMSNorm");
    DM_CHECK(count_u32(input_len));
    DM_CHECK(set_device(ctx));
    size_t bytes = input_len * sizeof(float);
    DM_CHECK(ctx->in.ensure(2 * bytes));
    DM_CHECK(ctx->out.ensure(bytes));
    float *din = (float *)ctx->in.ptr;
    float *dw = weight ? din + input_len : nullptr;
    HostCall hc(ctx);
    DM_CHECK(hc.begin((weight ? 3 : 2) * bytes));
    DM_CHECK(hc.in(din, input, bytes));
    if (weight) DM_CHECK(hc.in(dw, weight, bytes));
    float *o = (float *)hc.out_direct(output, bytes);  // written by the kernel, no copy back
    DM_HIP(launch_rms_norm(ctx->stream, din, 1, (uint32_t)input_len, dw, epsilon, o ? o : (float *)ctx->out.ptr));
    if (!o) DM_CHECK(hc.out(output, ctx->out.ptr, bytes));
    return hc.finish();
}

int dmhip_silu_mul(dmhip_ctx *ctx, const float *gate, size_t gate_len, const float *up,
                   size_t up_len, float *output, size_t output_len) {
    DM_REQUIRE(ctx);
    DM_CHECK(require_nonempty("SiLU multiply", gate_len));
    DM_CHECK(validate_vector_length("SiLU multiply", "up", gate_len, up_len));
    DM_CHECK(validate_vector_length("SiLU multiply", "output", gate_len, output_len));
    DM_REQUIRE(gate);
    DM_REQUIRE(up);
    DM_REQUIRE(output);
    DM_CHECK(count_u32(gate_len));
    DM_CHECK(set_device(ctx));
    size_t bytes = gate_len * sizeof(float);
    DM_CHECK(ctx->in.ensure(2 * bytes));
    DM_CHECK(ctx->out.ensure(bytes));
    float *dg = (float *)ctx->in.ptr, *du = dg + gate_len;
    HostCall hc(ctx);
    DM_CHECK(hc.begin(3 * bytes));
    DM_CHECK(hc.in(dg, gate, bytes));
    DM_CHECK(hc.in(du, up, bytes));
    float *o = (float *)hc.out_direct(output, bytes);
    DM_HIP(launch_silu_mul(ctx->stream, dg, du, gate_len, o ? o : (float *)ctx->out.ptr));
    if (!o) DM_CHECK(hc.out(output, ctx->out.ptr, bytes));
    return hc.finish();
}

int dmhip_softcap(dmhip_ctx *ctx, const float *input, size_t input_len, float cap, float *output,
                  size_t output_len) {
    DM_REQUIRE(ctx);
    DM_CHECK(require_nonempty("logit softcap", input_len));
    DM_CHECK(validate_vector_length("logit softcap", "output", input_len, output_len));
    DM_CHECK(require_positive("logit softcap", cap));
    DM_REQUIRE(input);
    DM_REQUIRE(output);
    DM_CHECK(count_u32(input_len));
    DM_CHECK(set_device(ctx));
    size_t bytes = input_len * sizeof(float);
    DM_CHECK(ctx->in.ensure(bytes));
    DM_CHECK(ctx->out.ensure(bytes));
    HostCall hc(ctx);
    DM_CHECK(hc.begin(2 * bytes));
    DM_CHECK(hc.in(ctx->in.ptr, input, bytes));
    float *o = (float *)hc.out_direct(output, bytes);
    DM_HIP(launch_softcap(ctx->stream, (const float *)ctx->in.ptr, input_len, cap, o ? o : (float *)ctx->out.ptr));
    if (!o) DM_CHECK(hc.out(output, ctx->out.ptr, bytes));
    return hc.finish();
}

int dmhip_add(dmhip_ctx *ctx, const float *left, size_t left_len, const float *right, size_t right_len,
              float *output, size_t output_len) {
    DM_REQUIRE(ctx);
    if (left_len != right_len || left_len != output_len) return fail_vector_lengths(left_len, right_len, output_len);
    if (left_len == 0) return DMHIP_OK;
    DM_CHECK(count_u32(left_len));
    DM_REQUIRE(left);
    DM_REQUIRE(right);
    DM_REQUIRE(output);
    DM_CHECK(set_device(ctx));
    size_t bytes = left_len * sizeof(float);
    DM_CHECK(ctx->in.ensure(2 * bytes));
    DM_CHECK(ctx->out.ensure(bytes));
    float *da = (float *)ctx->in.ptr, *db = da + left_len;
    HostCall hc(ctx);
    DM_CHECK(hc.begin(3 * bytes));
    DM_CHECK(hc.in(da, left, bytes));
    DM_CHECK(hc.in(db, right, bytes));
    float *o = (float *)hc.out_direct(output, bytes);
    DM_HIP(launch_add(ctx->stream, da, db, left_len, o ? o : (float *)ctx->out.ptr));
    if (!o) DM_CHECK(hc.out(output, ctx->out.ptr, bytes));
    return hc.finish();
}

int dmhip_gelu_mul(dmhip_ctx *ctx, const float *gate, size_t gate_len, const float *up, size_t up_len,
                   float *output, size_t output_len) {
    DM_REQUIRE(ctx);
    DM_CHECK(require_nonempty("GELU multiply", gate_len));
    DM_CHECK(validate_vector_length("GELU multiply", "up", gate_len, up_len));
    DM_CHECK(validate_vector_length("GELU multiply", "output", gate_len, output_len));
    DM_CHECK(count_u32(gate_len));
    DM_REQUIRE(gate);
    DM_REQUIRE(up);
    DM_REQUIRE(output);
    DM_CHECK(set_device(ctx));
    size_t bytes = gate_len * sizeof(float);
    DM_CHECK(ctx->in.ensure(2 * bytes));
    DM_CHECK(ctx->out.ensure(bytes));
    float *dg = (float *)ctx->in.ptr, *du = dg + gate_len;
    HostCall hc(ctx);
    DM_CHECK(hc.begin(3 * bytes));
    DM_CHECK(hc.in(dg, gate, bytes));
    DM_CHECK(hc.in(du, up, bytes));
    float *o = (float *)hc.out_direct(output, bytes);
    DM_HIP(launch_gelu_mul(ctx->stream, dg, du, gate_len, o ? o : (float *)ctx->out.ptr));
    if (!o) DM_CHECK(hc.out(output, ctx->out.ptr, bytes));
    return hc.finish();
}

int dmhip_softmax(dmhip_ctx *ctx, const float *input, size_t input_len, float *output, size_t output_len) {
    DM_REQUIRE(ctx);
    DM_CHECK(require_nonempty("softmax", input_len));
    DM_CHECK(validate_vector_length("softmax", "output", input_len, output_len));
    DM_REQUIRE(input);
    DM_REQUIRE(output);
    if (!all_finite(input, input_len)) return fail_non_finite("softmax");
    DM_CHECK(count_u32(input_len));
    DM_CHECK(set_device(ctx));
    size_t bytes = input_len * sizeof(float);
    DM_CHECK(ctx->in.ensure(bytes));
    DM_CHECK(ctx->out.ensure(bytes));
    HostCall hc(ctx);
    DM_CHECK(hc.begin(2 * bytes));
    DM_CHECK(hc.in(ctx->in.ptr, input, bytes));
    DM_HIP(launch_softmax(ctx->stream, (const float *)ctx->in.ptr, (uint32_t)input_len, (float *)ctx->out.ptr));
    DM_CHECK(hc.out(output, ctx->out.ptr, bytes));
    return hc.finish();
}

int dmhip_rope_neox_in_place(dmhip_ctx *ctx, float *values, size_t values_len, size_t heads,
                             size_t head_dimension, size_t rotated_pairs, size_t position, float theta) {
    DM_REQUIRE(ctx);
    bool noop = false;
    DM_CHECK(check_rope(values_len, heads, head_dimension, rotated_pairs, position, theta, &noop));
    if (noop) return DMHIP_OK;
    DM_REQUIRE(values);
    DM_CHECK(set_device(ctx));
    size_t bytes = values_len * sizeof(float);
    DM_CHECK(ctx->in.ensure(bytes));
    float *dv = (float *)ctx->in.ptr;
    HostCall hc(ctx);
    DM_CHECK(hc.begin(2 * bytes));
    DM_CHECK(hc.in(dv, values, bytes));
    DM_HIP(launch_rope_neox(ctx->stream, dv, heads, (uint32_t)head_dimension, (uint32_t)rotated_pairs,
                            (uint32_t)position, theta));
    DM_CHECK(hc.out(values, dv, bytes));
    return hc.finish();
}

int dmhip_argmax(dmhip_ctx *ctx, const float *input, size_t input_len, size_t *index) {
    DM_REQUIRE(ctx);
    DM_REQUIRE(index);
    DM_CHECK(require_nonempty("argmax", input_len));
    DM_REQUIRE(input);
    if (!all_finite(input, input_len))
        return fail_non_finite("argmax");
    DM_CHECK(count_u32(input_len));
    DM_CHECK(set_device(ctx));
    size_t bytes = input_len * sizeof(float);
    DM_CHECK(ctx->in.ensure(bytes));
    HostCall hc(ctx);
    DM_CHECK(hc.begin(bytes + 4));
    DM_CHECK(hc.in(ctx->in.ptr, input, bytes));
    DM_HIP(launch_argmax(ctx->stream, (const float *)ctx->in.ptr, input_len, ctx->argmax_state,
                         ctx->argmax_index));
    uint32_t result = 0;
    DM_CHECK(hc.out(&result, ctx->argmax_index, 4));
    DM_CHECK(hc.finish());
    *index = result;
    return DMHIP_OK;
}

int dmhip_top_k_softmax(dmhip_ctx *ctx, const float *logits, size_t logits_len, size_t k,
                        size_t *indices, float *probabilities) {
    DM_REQUIRE(ctx);
    if (k == 0 || k > logits_len)
        return fail_top_k(k, logits_len);
    DM_REQUIRE(logits);
    DM_REQUIRE(indices);
    DM_REQUIRE(probabilities);
    if (!all_finite(logits, logits_len))
        return fail_non_finite("top-k softmax");
    DM_CHECK(count_u32(logits_len));
    if (k > kMaxTopK)
        return fail(DMHIP_ERR_VECTOR_TOO_LARGE, "top-k count %zu exceeds the kernel limit %u", k, kMaxTopK);
    DM_CHECK(set_device(ctx));
    size_t bytes = logits_len * sizeof(float);
    DM_CHECK(ctx->in.ensure(bytes));
    DM_CHECK(ctx->out.ensure(k * 8));
    uint32_t *dids = (uint32_t *)ctx->out.ptr;
    float *dp = (float *)(dids + k);
    HostCall hc(ctx);
    DM_CHECK(hc.begin(bytes + 8 * k));
    DM_CHECK(hc.in(ctx->in.ptr, logits, bytes));
    DM_HIP(launch_top_k(ctx->stream, (const float *)ctx->in.ptr, 1, (uint32_t)logits_len,
                        (uint32_t)k, dids, dp, BadFlag{ctx->flags + 2, 1}));  // checked on the host first
    uint32_t ids[kMaxTopK];
    DM_CHECK(hc.out(ids, dids, k * 4));
    DM_CHECK(hc.out(probabilities, dp, k * 4));
    DM_CHECK(hc.finish());
    for (size_t i = 0; i < k; i++) indices[i] = ids[i];
    return DMHIP_OK;
}

static int matvec_from_device(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns,
                              const void *w, const float *input, float *output) {
    if (rows == 0) return DMHIP_OK;
    DM_CHECK(require_nonempty("matvec", columns));
    DM_REQUIRE(input);
    DM_REQUIRE(output);
    DM_CHECK(count_u32(columns));
    DM_CHECK(count_u32(rows));
    const size_t in_bytes = columns * sizeof(float), out_bytes = rows * sizeof(float);
    DM_CHECK(ctx->in.ensure(in_bytes));
    DM_CHECK(ctx->out.ensure(out_bytes));
    HostCall hc(ctx);
    DM_CHECK(hc.begin(in_bytes + out_bytes));
    DM_CHECK(hc.in(ctx->in.ptr, input, in_bytes));
    // The kernels write y straight into the pinned bounce buffer (plain
    // stores; the rows travel to host memory while the rest is computed),
    // so no copy follows them.
    float *y = (float *)hc.out_direct(output, out_bytes);
    DM_CHECK(enqueue_matvec(ctx, type, rows, columns, w, 1, (const float *)ctx->in.ptr,
                            y ? y : (float *)ctx->out.ptr));
    if (!y) DM_CHECK(hc.out(output, ctx->out.ptr, out_bytes));
    return hc.finish();
}

int dmhip_matvec(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns,
                 const uint8_t *encoded, size_t encoded_len, const float *input, size_t input_len,
                 float *output, size_t output_len) {
    DM_REQUIRE(ctx);
    size_t row_bytes;
    DM_CHECK(prepare_matvec(type, rows, columns, encoded_len, input_len, output_len, &row_bytes));
    if (rows == 0) return DMHIP_OK;
    DM_CHECK(require_nonempty("matvec", input_len));
    DM_REQUIRE(encoded);
    DM_CHECK(set_device(ctx));
    // Like MetalContext::matvec (src/metal.rs:664), the encoded matrix is
    // copied to the device for this call.
    DM_CHECK(ctx->enc.ensure(encoded_len + 256));
    DM_HIP(hipMemcpyAsync(ctx->enc.ptr, encoded, encoded_len, hipMemcpyHostToDevice, ctx->stream));
    return matvec_from_device(ctx, type, rows, columns, ctx->enc.ptr, input, output);
}

static int matvec_buffer(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns,
                         const dmhip_buf *buf, size_t offset, size_t length, const float *input,
                         size_t input_len, float *output, size_t output_len) {
    DM_REQUIRE(ctx);
    DM_REQUIRE(buf);
    size_t row_bytes;
    DM_CHECK(prepare_matvec(type, rows, columns, length, input_len, output_len, &row_bytes));
    DM_CHECK(check_range(buf, offset, length));
    if (rows == 0) return DMHIP_OK;
    DM_CHECK(require_nonempty("matvec", input_len));
    DM_CHECK(set_device(ctx));
    return matvec_from_device(ctx, type, rows, columns, (const char *)buf->dev + offset, input, output);
}

int dmhip_matvec_mapped(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns,
                        const dmhip_buf *mapping, size_t offset, size_t length, const float *input,
                        size_t input_len, float *output, size_t output_len) {
    return matvec_buffer(ctx, type, rows, columns, mapping, offset, length, input, input_len,
                         output, output_len);
}

int dmhip_matvec_owned(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns,
                       const dmhip_buf *encoded, size_t offset, size_t length, const float *input,
                       size_t input_len, float *output, size_t output_len) {
    return matvec_buffer(ctx, type, rows, columns, encoded, offset, length, input, input_len,
                         output, output_len);
}

int dmhip_dequantize(dmhip_ctx *ctx, uint32_t type, const dmhip_buf *encoded, size_t offset,
                     size_t length, float *output, size_t elements) {
    DM_REQUIRE(ctx);
    DM_REQUIRE(encoded);
    // cpu::dequantize validation (src/cpu.rs:313-341).
    if (!(type == 0 || type == 1 || type == 6 || type == 8 || type == 12 || type == 14))
        return fail_unsupported(type, "HIP dequantization");
    uint64_t expected;
    uint32_t be, bb;
    type_layout(type, &be, &bb);
    if (!row_byte_len(type, elements, &expected)) return fail_element_count(type, elements);
    if (length != expected) return fail_byte_length(type, expected, length);
    DM_CHECK(check_range(encoded, offset, length));
    if (elements == 0) return DMHIP_OK;
    DM_REQUIRE(output);
    DM_CHECK(set_device(ctx));
    DM_CHECK(ctx->out.ensure(elements * sizeof(float)));
    DM_HIP(launch_dequantize(ctx->stream, type, (const uint8_t *)encoded->dev + offset, be, bb,
                             elements, (float *)ctx->out.ptr));
    DM_HIP(hipMemcpyAsync(output, ctx->out.ptr, elements * sizeof(float), hipMemcpyDeviceToHost,
                          ctx->stream));
    DM_HIP(hipStreamSynchronize(ctx->stream));  // a copy into pageable memory precedes
    return DMHIP_OK;
}

// ---- stream-ordered device operators ---------------------------------------

static int validate_device_matvec(uint32_t type, size_t rows, size_t columns, size_t batch) {
    if (!(type == 0 || type == 1 || type == 6 || type == 8 || type == 12 || type == 14))
        return fail_unsupported(type, "HIP matrix-vector multiplication");
    uint64_t rb;
    if (!row_byte_len(type, columns, &rb)) return fail_element_count(type, columns);
    if (batch < 1 || batch > 16)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "batch %zu is outside 1..=16", batch);
    DM_CHECK(count_u32(rows));
    DM_CHECK(count_u32(columns));
    if (rows != 0 && rb > SIZE_MAX / rows)
        return fail(DMHIP_ERR_OVERFLOW, "matrix dimensions or encoded byte length overflowed");
    return DMHIP_OK;
}

int dmhip_matvec_device(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns,
                        const void *weights, size_t batch, const float *x, float *y) {
    DM_REQUIRE(ctx);
    DM_CHECK(validate_device_matvec(type, rows, columns, batch));
    if (rows == 0) return DMHIP_OK;
    DM_CHECK(require_nonempty("matvec", columns));
    DM_REQUIRE(weights);
    DM_REQUIRE(x);
    DM_REQUIRE(y);
    DM_CHECK(set_device(ctx));
    return enqueue_matvec(ctx, type, rows, columns, weights, batch, x, y);
}

int dmhip_matvec_batch_device(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns, size_t count,
                              const void *const *weights, const float *x, size_t x_stride, float *y,
                              size_t y_stride) {
    DM_REQUIRE(ctx);
    DM_CHECK(validate_device_matvec(type, rows, columns, 1));
    if (rows == 0 || count == 0) return DMHIP_OK;
    DM_CHECK(require_nonempty("matvec", columns));
    DM_REQUIRE(weights);
    DM_REQUIRE(x);
    DM_REQUIRE(y);
    for (size_t i = 0; i < count; i++)
        if (!weights[i]) return fail(DMHIP_ERR_INVALID_ARGUMENT, "weights[%zu] must not be null", i);
    DM_CHECK(set_device(ctx));
    // One grouped launch when every matrix suits the int8 kernel and the
    // offsets fit its 32-bit job table; otherwise one matvec per matrix.
    const size_t lim = 0x80000000ull;
    bool grouped = qmv8_grouped_supported(type, rows, columns, 1) && count < lim && x_stride < lim &&
                   y_stride < lim && (count - 1) * x_stride + columns < lim &&
                   (count - 1) * y_stride + rows < lim;
    for (size_t i = 0; grouped && i < count; i++)
        grouped = ((uintptr_t)weights[i] & (type == 12u ? 15u : 3u)) == 0;  // 12 = Q4_K
    if (!grouped) {
        for (size_t i = 0; i < count; i++)
            DM_CHECK(enqueue_matvec(ctx, type, rows, columns, weights[i], 1, x + i * x_stride, y + i * y_stride));
        return DMHIP_OK;
    }
    std::vector<QmvJob> jobs(count);
    for (size_t i = 0; i < count; i++)
        jobs[i] = QmvJob{weights[i], 1u, (uint32_t)(i * x_stride), (uint32_t)(i * y_stride), 0, 0};
    DM_HIP(launch_qmv8_grouped(ctx, type, (uint32_t)rows, (uint32_t)columns, 0, 0, jobs.data(), count, x, y));
    return DMHIP_OK;
}

int dmhip_matvec_argmax_device(dmhip_ctx *ctx, uint32_t type, size_t rows, size_t columns,
                               const void *weights, const float *x, float *y,
                               uint32_t *index_device) {
    DM_REQUIRE(ctx);
    DM_CHECK(validate_device_matvec(type, rows, columns, 1));
    DM_CHECK(require_nonempty("argmax", rows));
    DM_CHECK(require_nonempty("matvec", columns));
    DM_REQUIRE(weights);
    DM_REQUIRE(x);
    DM_REQUIRE(y);
    DM_REQUIRE(index_device);
    DM_CHECK(set_device(ctx));
    DM_CHECK(enqueue_matvec_argmax(ctx, type, rows, columns, weights, x, y, index_device));
    ctx->argmax_pending = true;
    ctx->argmax_user_index = index_device;
    return DMHIP_OK;
}

int dmhip_argmax_result(dmhip_ctx *ctx, size_t *index) {
    DM_REQUIRE(ctx);
    DM_REQUIRE(index);
    if (!ctx->argmax_pending)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "no matvec_argmax is pending on this context");
    DM_CHECK(set_device(ctx));
    ArgmaxState state;
    uint32_t result = 0;
    DM_HIP(hipMemcpyAsync(&state, ctx->argmax_state, sizeof state, hipMemcpyDeviceToHost, ctx->stream));
    DM_HIP(hipMemcpyAsync(&result, ctx->argmax_user_index, 4, hipMemcpyDeviceToHost, ctx->stream));
    DM_HIP(hipStreamSynchronize(ctx->stream));  // a copy into pageable memory precedes
    ctx->argmax_pending = false;
    if (state.non_finite) return fail_non_finite("argmax");
    *index = result;
    return DMHIP_OK;
}

int dmhip_rms_norm_device(dmhip_ctx *ctx, size_t batch, size_t count, const float *input,
                          const float *weight, float epsilon, float *output) {
    DM_REQUIRE(ctx);
    DM_CHECK(require_nonempty("RMSNorm", count));
    DM_CHECK(require_positive("RMSNorm epsilon", epsilon));
    DM_REQUIRE(input);
    DM_REQUIRE(output);
    DM_CHECK(count_u32(count));
    DM_CHECK(count_u32(batch));
    if (batch == 0) return DMHIP_OK;
    DM_CHECK(set_device(ctx));
    DM_HIP(launch_rms_norm(ctx->stream, input, (uint32_t)batch, (uint32_t)count, weight, epsilon, output));
    return DMHIP_OK;
}

int dmhip_silu_mul_device(dmhip_ctx *ctx, size_t count, const float *gate, const float *up,
                          float *output) {
    DM_REQUIRE(ctx);
    DM_CHECK(require_nonempty("SiLU multiply", count));
    DM_REQUIRE(gate);
    DM_REQUIRE(up);
    DM_REQUIRE(output);
    DM_CHECK(set_device(ctx));
    DM_HIP(launch_silu_mul(ctx->stream, gate, up, count, output));
    return DMHIP_OK;
}

int dmhip_softcap_device(dmhip_ctx *ctx, size_t count, const float *input, float cap, float *output) {
    DM_REQUIRE(ctx);
    DM_CHECK(require_nonempty("logit softcap", count));
    DM_CHECK(require_positive("logit softcap", cap));
    DM_REQUIRE(input);
    DM_REQUIRE(output);
    DM_CHECK(set_device(ctx));
    DM_HIP(launch_softcap(ctx->stream, input, count, cap, output));
    return DMHIP_OK;
}

int dmhip_add_device(dmhip_ctx *ctx, size_t count, const float *left, const float *right, float *output) {
    DM_REQUIRE(ctx);
    if (count == 0) return DMHIP_OK;
    DM_CHECK(count_u32(count));
    DM_REQUIRE(left);
    DM_REQUIRE(right);
    DM_REQUIRE(output);
    DM_CHECK(set_device(ctx));
    DM_HIP(launch_add(ctx->stream, left, right, count, output));
    return DMHIP_OK;
}

int dmhip_gelu_mul_device(dmhip_ctx *ctx, size_t count, const float *gate, const float *up, float *output) {
    DM_REQUIRE(ctx);
    DM_CHECK(require_nonempty("GELU multiply", count));
    DM_CHECK(count_u32(count));
    DM_REQUIRE(gate);
    DM_REQUIRE(up);
    DM_REQUIRE(output);
    DM_CHECK(set_device(ctx));
    DM_HIP(launch_gelu_mul(ctx->stream, gate, up, count, output));
    return DMHIP_OK;
}

int dmhip_rope_neox_device(dmhip_ctx *ctx, float *values, size_t values_len, size_t heads,
                           size_t head_dimension, size_t rotated_pairs, size_t position, float theta) {
    DM_REQUIRE(ctx);
    bool noop = false;
    DM_CHECK(check_rope(values_len, heads, head_dimension, rotated_pairs, position, theta, &noop));
    if (noop) return DMHIP_OK;
    DM_REQUIRE(values);
    DM_CHECK(set_device(ctx));
    DM_HIP(launch_rope_neox(ctx->stream, values, heads, (uint32_t)head_dimension, (uint32_t)rotated_pairs,
                            (uint32_t)position, theta));
    return DMHIP_OK;
}

int dmhip_router_top_k_device(dmhip_ctx *ctx, size_t batch, size_t hidden, size_t experts,
                              size_t k, const uint16_t *router_bf16, const float *x,
                              float *logits, uint32_t *ids, float *probabilities) {
    DM_REQUIRE(ctx);
    if (k == 0 || k > experts)
        return fail_top_k(k, experts);
    if (k > kMaxTopK || experts > 16384)
        return fail(DMHIP_ERR_VECTOR_TOO_LARGE, "router with %zu experts, top-%zu exceeds the kernel limits",
                    experts, k);
    DM_CHECK(require_nonempty("router", hidden));
    DM_REQUIRE(router_bf16);
    DM_REQUIRE(x);
    DM_REQUIRE(logits);
    DM_REQUIRE(ids);
    DM_REQUIRE(probabilities);
    DM_CHECK(count_u32(hidden));
    if (batch == 0) return DMHIP_OK;
    DM_CHECK(set_device(ctx));
    // A new mark per call: the word needs no clearing launch.
    // the calls between two results share one mark, so the result reports
    // a non-finite logit in any of them
    if (!ctx->router_pending) ctx->router_mark = ctx->router_mark + 1 ? ctx->router_mark + 1 : 1;
    ctx->router_pending = true;
    DM_HIP(launch_router_top_k(ctx->stream, router_bf16, (uint32_t)hidden, (uint32_t)experts,
                               (uint32_t)k, (uint32_t)batch, x, logits, ids, probabilities,
                               BadFlag{ctx->flags, ctx->router_mark}, nullptr, nullptr,
                               batch <= kRouterTickets ? ctx->router_tickets : nullptr));
    return DMHIP_OK;
}

int dmhip_router_result(dmhip_ctx *ctx) {
    DM_REQUIRE(ctx);
    if (!ctx->router_pending)
        return fail(DMHIP_ERR_INVALID_ARGUMENT, "no router_top_k is pending on this context");
    DM_CHECK(set_device(ctx));
    uint32_t flag = 0;
    DM_HIP(hipMemcpyAsync(&flag, ctx->flags, 4, hipMemcpyDeviceToHost, ctx->stream));
    DM_HIP(hipStreamSynchronize(ctx->stream));  // a copy into pageable memory precedes
    ctx->router_pending = false;
    if (flag == ctx->router_mark) return fail_non_finite("top-k softmax");
    return DMHIP_OK;
}

int dmhip_copy_device(dmhip_ctx *ctx, void *dst, const void *src, size_t n) {
    DM_REQUIRE(ctx);
    if (n == 0) return DMHIP_OK;
    DM_REQUIRE(dst);
    DM_REQUIRE(src);
    DM_CHECK(set_device(ctx));
    DM_HIP(launch_copy_bytes(ctx->stream, dst, src, n));
    return DMHIP_OK;
}

int dmhip_event_record(dmhip_ctx *ctx, void **event) {
    DM_REQUIRE(ctx);
    DM_REQUIRE(event);
    DM_CHECK(set_device(ctx));
    hipEvent_t e;
    DM_HIP(hipEventCreate(&e));
    hipError_t r = hipEventRecord(e, ctx->stream);
    if (r != hipSuccess) {
        (void)hipEventDestroy(e);
        return hip_fail(r, "hipEventRecord");
    }
    *event = (void *)e;
    return DMHIP_OK;
}

int dmhip_event_elapsed_ms(void *start, void *stop, float *ms) {
    DM_REQUIRE(start);
    DM_REQUIRE(stop);
    DM_REQUIRE(ms);
    DM_HIP(hipEventSynchronize((hipEvent_t)stop));
    DM_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return DMHIP_OK;
}

void dmhip_event_free(void *event) {
    if (event) (void)hipEventDestroy((hipEvent_t)event);
}

}  // extern "C"
