/*
 * dmhip.h -- C ABI of the MI355X (gfx950) backend for DiskMule's
 * quantized-matrix path.
 *
 * This header is the drop-in boundary.  It replaces the public surface of the
 * reference's Metal backend (src/metal.rs, re-exported at :2571-2572) and of
 * its expert residency (src/expert.rs) for the operators on the quantized
 * path.  A Rust `hip` module binds these symbols 1:1 (an `extern "C"` block
 * over this header) so the graph code keeps calling `matvec_mapped`,
 * `matvec_owned`, `argmax`, `top_k_softmax`, `rms_norm`, `silu_mul`, `add`,
 * `gelu_mul`, `softmax`, `rope_neox_in_place`, the attention and KV-cache
 * methods and `ExpertCache::with_expert` by name.
 *
 * Conventions (kept from src/metal.rs):
 *  - Every entry point validates its arguments before any device work and
 *    returns a dmhip_status; nothing aborts, no C++ exception crosses the ABI.
 *    The message of the last failure on the calling thread is returned by
 *    dmhip_last_error().
 *  - The "host" entry points take host slices and are synchronous: they
 *    return after the device work finished, as the Metal backend does
 *    (src/metal.rs:1595-1596).
 *  - The "_device" entry points take device addresses and only enqueue work
 *    on the context's stream (stream-ordered, asynchronous); they exist so a
 *    graph can keep activations resident in HBM.  dmhip_synchronize() waits.
 *  - A context is used from one thread at a time, as MetalContext is owned by
 *    its model-worker thread (src/runtime.rs:741-760).
 *  - Tensor types are ggml ids (src/gguf.rs:295-318).  Rows are contiguous;
 *    row r of a matrix starts at r * row_byte_len(columns).
 */
#ifndef DMHIP_H
#define DMHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  Each mirrors a MetalError / ExpertCacheError variant
   (src/metal.rs:3-126, src/expert.rs:13-42). */
typedef enum dmhip_status {
    DMHIP_OK = 0,
    DMHIP_ERR_NO_DEVICE = 1,             /* MetalError::NoDevice */
    DMHIP_ERR_BUFFER_ALLOCATION = 2,     /* MetalError::BufferAllocation */
    DMHIP_ERR_VECTOR_LENGTH = 3,         /* MetalError::VectorLength */
    DMHIP_ERR_VECTOR_TOO_LARGE = 4,      /* MetalError::VectorTooLarge */
    DMHIP_ERR_EMPTY_INPUT = 5,           /* MetalError::EmptyInput */
    DMHIP_ERR_INVALID_VECTOR_LENGTH = 6, /* MetalError::InvalidVectorLength */
    DMHIP_ERR_INVALID_POSITIVE_PARAMETER = 7, /* MetalError::InvalidPositiveParameter */
    DMHIP_ERR_NON_FINITE = 8,            /* MetalError::NonFinite */
    DMHIP_ERR_UNSUPPORTED_TENSOR_TYPE = 9, /* MetalError::UnsupportedTensorType */
    DMHIP_ERR_INVALID_ELEMENT_COUNT = 10, /* MetalError::InvalidElementCount */
    DMHIP_ERR_INVALID_BYTE_LENGTH = 11,  /* MetalError::InvalidByteLength */
    DMHIP_ERR_OVERFLOW = 12,             /* MetalError::Overflow */
    DMHIP_ERR_INVALID_INPUT_LENGTH = 13, /* MetalError::InvalidInputLength */
    DMHIP_ERR_INVALID_OUTPUT_LENGTH = 14, /* MetalError::InvalidOutputLength */
    DMHIP_ERR_INVALID_TOP_K = 15,        /* MetalError::InvalidTopK */
    DMHIP_ERR_MAPPED_RANGE = 16,         /* MetalError::MappedRange */
    DMHIP_ERR_COMMAND = 17,              /* MetalError::Command (a HIP runtime error) */
    DMHIP_ERR_NO_SLOTS = 18,             /* ExpertCacheError::NoSlots */
    DMHIP_ERR_INVALID_LAYER = 19,        /* ExpertCacheError::InvalidLayer */
    DMHIP_ERR_INVALID_EXPERT = 20,       /* ExpertCacheError::InvalidExpert */
    DMHIP_ERR_ALL_SLOTS_PINNED = 21,     /* ExpertCacheError::AllSlotsPinned */
    DMHIP_ERR_CANCELLED = 22,            /* ExpertCacheError::Cancelled */
    DMHIP_ERR_INVALID_LAYOUT = 23,       /* ExpertCacheError::InvalidLayout */
    DMHIP_ERR_INVALID_ARGUMENT = 24,     /* a null handle or pointer, or a C-API misuse */
    DMHIP_ERR_IO = 25,                   /* ExpertCacheError::Io (a failed or short pread) */
    DMHIP_ERR_INVALID_ATTENTION_SHAPE = 26, /* MetalError::InvalidAttentionShape */
    DMHIP_ERR_KV_POSITION = 27,          /* MetalError::KvPosition */
    DMHIP_ERR_KV_WIDTH = 28,             /* MetalError::KvWidth */
    DMHIP_ERR_KV_CONTEXT = 29,           /* MetalError::KvContext */
    DMHIP_ERR_INVALID_ROPE_SHAPE = 30,   /* MetalError::InvalidRopeShape */
    DMHIP_ERR_INVALID_ROPE_PAIRS = 31    /* MetalError::InvalidRopePairs */
} dmhip_status;

/* The payload of the calling thread's last failure: the fields of the
   MetalError / ExpertCacheError variant its status mirrors (src/metal.rs:3-126,
   src/expert.rs:13-42), so a binding can rebuild the variant exactly.  Fields
   a variant does not use are zero / NULL.  The strings are static (they live
   as long as the library).
     BufferAllocation            bytes
     VectorLength                left, right, output
     EmptyInput                  operation
     InvalidVectorLength         operation, argument, expected, actual
     InvalidPositiveParameter    operation
     NonFinite                   operation
     UnsupportedTensorType       kind
     InvalidElementCount         kind, elements, block_elements
     InvalidByteLength           kind, expected, actual
     InvalidInputLength          expected, actual
     InvalidOutputLength         expected, actual
     InvalidTopK                 k, length
     MappedRange                 offset, end, length
     InvalidLayer                layer, count
     InvalidExpert               layer, expert, count
     AllSlotsPinned              layer
     Io                          os_error (an errno value; 0: unexpected end of file)
     InvalidAttentionShape       reason (the reference's static message)
     KvPosition, KvWidth         expected, actual
     KvContext                   position, limit
     InvalidRopeShape            length, heads, head_dimension
     Command, InvalidLayout      the message (dmhip_last_error) */
typedef struct dmhip_error_detail {
    int32_t status;
    int32_t os_error;
    const char *operation;
    const char *argument;
    const char *kind;
    uint64_t expected, actual;
    uint64_t offset, end, length;
    uint64_t left, right, output;
    uint64_t elements, block_elements;
    uint64_t k;
    uint64_t bytes;
    uint64_t layer, expert, count;
    uint64_t position, limit;
    const char *reason;
    uint64_t heads, head_dimension;
} dmhip_error_detail;

/* ggml tensor type ids accepted by the matvec entry points. */
enum {
    DMHIP_TYPE_F32 = 0,
    DMHIP_TYPE_F16 = 1,
    DMHIP_TYPE_Q5_0 = 6,
    DMHIP_TYPE_Q8_0 = 8,
    DMHIP_TYPE_Q4_K = 12,
    DMHIP_TYPE_Q6_K = 14,
    DMHIP_TYPE_BF16 = 30
};

typedef struct dmhip_ctx dmhip_ctx;
typedef struct dmhip_buf dmhip_buf;
typedef struct dmhip_expert_cache dmhip_expert_cache;
typedef struct dmhip_kv_layer dmhip_kv_layer;

/* ---------------------------------------------------------------------- */
/* Context, errors, device                                                 */
/* ---------------------------------------------------------------------- */

/* Last failure message on the calling thread ("" if none). */
const char *dmhip_last_error(void);
/* Payload of the calling thread's last failure (status DMHIP_OK if none). */
int dmhip_last_error_detail(dmhip_error_detail *out);

/* MetalContext::new (src/metal.rs:291-346): selects HIP device `device`,
   creates its compute stream and its upload stream (default priority). */
int dmhip_context_new(int device, dmhip_ctx **out);
void dmhip_context_free(dmhip_ctx *ctx);

/* MetalContext::device_name (src/metal.rs:348-350). */
int dmhip_device_name(dmhip_ctx *ctx, char *buffer, size_t capacity);

/* Waits for all work enqueued on the context's streams. */
int dmhip_synchronize(dmhip_ctx *ctx);

/* The context's compute stream, as a hipStream_t. */
void *dmhip_stream(dmhip_ctx *ctx);

/* ---------------------------------------------------------------------- */
/* Buffers                                                                 */
/* ---------------------------------------------------------------------- */

/* MetalContext::map_read_only (src/metal.rs:352-392).  Unified memory let the
   reference wrap the GGUF mmap in place; a discrete GPU cannot, so the whole
   mapping is uploaded to HBM once and keeps its byte offsets.  A zero length
   is BufferAllocation, as in the reference. */
int dmhip_map_read_only(dmhip_ctx *ctx, const void *host, size_t length, dmhip_buf **out);

/* MetalContext::new_owned_buffer (src/metal.rs:394-402): zero-filled device
   buffer; a zero length is BufferAllocation. */
int dmhip_new_owned_buffer(dmhip_ctx *ctx, size_t length, dmhip_buf **out);
void dmhip_buffer_free(dmhip_buf *buffer);
size_t dmhip_buffer_len(const dmhip_buf *buffer);
/* Device address of the buffer's first byte. */
void *dmhip_buffer_device_ptr(const dmhip_buf *buffer);
/* MetalOwnedBuffer::as_mut_bytes / as_bytes (src/metal.rs:228-243) as copies. */
int dmhip_buffer_write(dmhip_ctx *ctx, dmhip_buf *buffer, size_t offset, const void *src, size_t n);
int dmhip_buffer_read(dmhip_ctx *ctx, const dmhip_buf *buffer, size_t offset, void *dst, size_t n);

/* Synchronous copies between host memory and a device address (for callers
   that hold device addresses from the _device entry points or an expert
   slot, as MetalOwnedBuffer::as_bytes exposes slot bytes, src/metal.rs:228). */
int dmhip_copy_to_host(dmhip_ctx *ctx, void *dst, const void *device_src, size_t n);
int dmhip_copy_to_device(dmhip_ctx *ctx, void *device_dst, const void *src, size_t n);

/* Pinned host memory for upload sources (hipHostMalloc). */
int dmhip_host_alloc_pinned(size_t bytes, void **out);
void dmhip_host_free_pinned(void *ptr);

/* ---------------------------------------------------------------------- */
/* Synchronous host-slice operators (the MetalContext surface)            */
/* ---------------------------------------------------------------------- */

/* MetalContext::rms_norm (src/metal.rs:435-476); weight may be NULL. */
int dmhip_rms_norm(dmhip_ctx *ctx, const float *input, size_t input_len, const float *weight,
                   size_t weight_len, float epsilon, float *output, size_t output_len);

/* MetalContext::silu_mul (src/metal.rs:554-576). */
int dmhip_silu_mul(dmhip_ctx *ctx, const float *gate, size_t gate_len, const float *up,
                   size_t up_len, float *output, size_t output_len);

/* MetalContext::softcap (src/metal.rs:600-622): output = cap * tanh(input /
   cap), src/cpu.rs:263-273.  Checks in the reference's order: EmptyInput,
   VectorLength (output), InvalidPositiveParameter (cap not finite and > 0). */
int dmhip_softcap(dmhip_ctx *ctx, const float *input, size_t input_len, float cap, float *output,
                  size_t output_len);

/* MetalContext::add (src/metal.rs:404-432): output = left + right.  The
   three lengths must agree (VectorLength); empty vectors are a no-op. */
int dmhip_add(dmhip_ctx *ctx, const float *left, size_t left_len, const float *right, size_t right_len,
              float *output, size_t output_len);

/* MetalContext::gelu_mul (src/metal.rs:530-552): output =
   gelu_tanh(gate) * up with Gemma 4's gelu_pytorch_tanh (src/cpu.rs:144-149).
   Checks: EmptyInput, InvalidVectorLength (up, then output). */
int dmhip_gelu_mul(dmhip_ctx *ctx, const float *gate, size_t gate_len, const float *up, size_t up_len,
                   float *output, size_t output_len);

/* MetalContext::softmax (src/metal.rs:578-598): the stable softmax of
   src/cpu.rs:196-225.  Checks: EmptyInput, InvalidVectorLength (output),
   NonFinite "softmax" for any non-finite input. */
int dmhip_softmax(dmhip_ctx *ctx, const float *input, size_t input_len, float *output, size_t output_len);

/* MetalContext::rope_neox_in_place (src/metal.rs:478-528): NeoX rotary
   embedding of `heads` contiguous heads of `head_dimension` values; pair p <
   rotated_pairs of each head, (x[p], x[p + head_dimension / 2]), turns by
   position * theta^(-2p / head_dimension) (src/cpu.rs:151-193).  Checks in
   the reference's order: InvalidRopeShape (heads * head_dimension !=
   values_len), InvalidRopePairs (odd head_dimension or rotated_pairs >
   head_dimension / 2), InvalidPositiveParameter "NeoX RoPE theta"; no
   rotated pairs or no heads is a no-op; then VectorTooLarge. */
int dmhip_rope_neox_in_place(dmhip_ctx *ctx, float *values, size_t values_len, size_t heads,
                             size_t head_dimension, size_t rotated_pairs, size_t position, float theta);

/* MetalContext::argmax (src/metal.rs:624-644): first maximum, lowest index on
   ties, non-finite input rejected. */
int dmhip_argmax(dmhip_ctx *ctx, const float *input, size_t input_len, size_t *index);

/* MetalContext::top_k_softmax (src/metal.rs:1392-1434): k ids in selection
   order (value descending, index ascending on ties) and their softmax. */
int dmhip_top_k_softmax(dmhip_ctx *ctx, const float *logits, size_t logits_len, size_t k,
                        size_t *indices, float *probabilities);

/* MetalContext::matvec (src/metal.rs:648-683): encoded matrix from host memory. */
int dmhip_matvec(dmhip_ctx *ctx, uint32_t ggml_type, size_t rows, size_t columns,
                 const uint8_t *encoded, size_t encoded_len, const float *input,
                 size_t input_len, float *output, size_t output_len);

/* MetalContext::matvec_mapped (src/metal.rs:687-734). */
int dmhip_matvec_mapped(dmhip_ctx *ctx, uint32_t ggml_type, size_t rows, size_t columns,
                        const dmhip_buf *mapping, size_t encoded_offset, size_t encoded_length,
                        const float *input, size_t input_len, float *output, size_t output_len);

/* MetalContext::matvec_owned (src/metal.rs:1148-1194). */
int dmhip_matvec_owned(dmhip_ctx *ctx, uint32_t ggml_type, size_t rows, size_t columns,
                       const dmhip_buf *encoded, size_t encoded_offset, size_t encoded_length,
                       const float *input, size_t input_len, float *output, size_t output_len);

/* Dequantize `elements` values of a device-resident encoding into host f32
   (the GPU counterpart of cpu::dequantize, src/cpu.rs:312-343; bit-exact). */
int dmhip_dequantize(dmhip_ctx *ctx, uint32_t ggml_type, const dmhip_buf *encoded,
                     size_t encoded_offset, size_t encoded_length, float *output,
                     size_t elements);

/* ---------------------------------------------------------------------- */
/* Stream-ordered device operators (device addresses, asynchronous)        */
/* ---------------------------------------------------------------------- */

/* y[b][r] = sum_c W[r][c] * x[b][c] for b < batch (1..16); x is
   [batch][columns] f32, y is [batch][rows] f32, W is `rows` encoded rows. */
int dmhip_matvec_device(dmhip_ctx *ctx, uint32_t ggml_type, size_t rows, size_t columns,
                        const void *weights, size_t batch, const float *x, float *y);

/* Batch-1 matvec plus greedy argmax over the rows (src/cpu.rs:275-293).
   *index_device receives the row index as uint32; a non-finite row makes the
   next dmhip_argmax_result() report NonFinite.  The reduction uses counters
   owned by the context and reset by each launch, so calls on one context are
   ordered on its stream (as every call of a context is). */
int dmhip_matvec_argmax_device(dmhip_ctx *ctx, uint32_t ggml_type, size_t rows,
                               size_t columns, const void *weights, const float *x,
                               float *y, uint32_t *index_device);
/* Waits for the last dmhip_matvec_argmax_device and returns its index. */
int dmhip_argmax_result(dmhip_ctx *ctx, size_t *index);

/* `count` independent batch-1 matvecs of one shape in one dispatch:
   y + i*y_stride = W_i . (x + i*x_stride) for i < count, W_i = weights[i]
   (`rows` encoded rows of `columns` values; strides in floats, 0 allowed for
   x).  The work of `count` consecutive MetalContext::matvec_mapped calls
   (src/metal.rs:687-760), e.g. the projections of one layer that read the
   same activation; Q4_K/Q6_K run as one grouped int8 launch, other types
   as one matvec per matrix. */
int dmhip_matvec_batch_device(dmhip_ctx *ctx, uint32_t ggml_type, size_t rows, size_t columns,
                              size_t count, const void *const *weights, const float *x, size_t x_stride,
                              float *y, size_t y_stride);

/* RMSNorm of `batch` rows of `count` values (src/cpu.rs:98-142). */
int dmhip_rms_norm_device(dmhip_ctx *ctx, size_t batch, size_t count, const float *input,
                          const float *weight, float epsilon, float *output);

/* out = silu(gate) * up, count values (src/qwen35/cpu.rs:422-424); output
   may be either input. */
int dmhip_silu_mul_device(dmhip_ctx *ctx, size_t count, const float *gate, const float *up,
                          float *output);

/* Logit softcap over `count` device values (src/cpu.rs:263-273), as
   dmhip_softcap; input and output may be the same buffer. */
int dmhip_softcap_device(dmhip_ctx *ctx, size_t count, const float *input, float cap, float *output);

/* output = left + right over `count` device values, as dmhip_add; output may
   be either input. */
int dmhip_add_device(dmhip_ctx *ctx, size_t count, const float *left, const float *right, float *output);

/* output = gelu_tanh(gate) * up over `count` device values, as
   dmhip_gelu_mul; output may be either input. */
int dmhip_gelu_mul_device(dmhip_ctx *ctx, size_t count, const float *gate, const float *up, float *output);

/* NeoX RoPE in place over device values, with dmhip_rope_neox_in_place's
   checks (values_len is the number of floats at `values`). */
int dmhip_rope_neox_device(dmhip_ctx *ctx, float *values, size_t values_len, size_t heads,
                           size_t head_dimension, size_t rotated_pairs, size_t position, float theta);

/* Dense gated FFN at decode for `batch` tokens (src/qwen35/cpu.rs:415-427):
   y = down(silu(gate(n)) * up(n)) with n = rms_norm(h, eps), unit weight.
   `workspace` is device memory of workspace_len bytes, at least
   dmhip_ffn_workspace_bytes(batch, hidden, ffn); a shorter one is rejected
   (InvalidArgument) before any work. */
size_t dmhip_ffn_workspace_bytes(size_t batch, size_t hidden, size_t ffn);
int dmhip_ffn_device(dmhip_ctx *ctx, size_t batch, size_t hidden, size_t ffn,
                     uint32_t gate_type, const void *gate, uint32_t up_type, const void *up,
                     uint32_t down_type, const void *down, float epsilon, const float *h,
                     float *y, void *workspace, size_t workspace_len);

/* dmhip_ffn_device without a workspace argument, for callers that cannot
   allocate device memory (code under HIP graph capture, tight serving loops,
   harnesses that forbid allocation); no counterpart in the reference.  The
   scratch comes from a fixed array in the library's code object of
   dmhip_ffn_noalloc_scratch_bytes() bytes (8 MiB) per device, resolved when
   a context is created on that device; a shape whose workspace (and, for
   batches above 2, activation fragments) exceed it is rejected
   (InvalidArgument) before any work.  Nothing is allocated: no hipMalloc,
   no growth of the context's scratch.  Every call on one device shares that
   device's array, so calls that overlap on one device (two contexts, or two
   streams, in flight at once) race; calls ordered on one context's stream
   do not. */
size_t dmhip_ffn_noalloc_scratch_bytes(void);
int dmhip_ffn_device_noalloc(dmhip_ctx *ctx, size_t batch, size_t hidden, size_t ffn,
                             uint32_t gate_type, const void *gate, uint32_t up_type, const void *up,
                             uint32_t down_type, const void *down, float epsilon, const float *h,
                             float *y);

/* Router for `batch` tokens: logits = bf16 router rows . x (exact sequential
   fold, src/cpu.rs:391-394), then top_k_softmax per token
   (src/cpu.rs:232-260).  ids [batch][k] uint32, probabilities [batch][k]. */
int dmhip_router_top_k_device(dmhip_ctx *ctx, size_t batch, size_t hidden, size_t experts,
                              size_t k, const uint16_t *router_bf16, const float *x,
                              float *logits, uint32_t *ids, float *probabilities);
/* Waits for the dmhip_router_top_k_device calls made since the previous
   result and returns NonFinite when any token's logits in any of them held a
   non-finite value (top_k_softmax rejects them, src/cpu.rs:240-245); the ids
   and probabilities of such a call are not meaningful. */
int dmhip_router_result(dmhip_ctx *ctx);

/* Prefill GEMM: C[m][n] = sum_k A[m][k] * W[n][k], A bf16 [m][k] row-major,
   W `n` encoded rows of `k` columns, C f32 [m][n].  `workspace` is device
   memory of workspace_len bytes, at least dmhip_gemm_workspace_bytes(m, k);
   a shorter one is rejected (InvalidArgument) before any work. */
size_t dmhip_gemm_workspace_bytes(size_t m, size_t k);
int dmhip_gemm_device(dmhip_ctx *ctx, uint32_t ggml_type, size_t m, size_t n, size_t k,
                      const uint16_t *a_bf16, const void *weights, float *c, void *workspace,
                      size_t workspace_len);

/* Events on the compute stream, for timing. */
int dmhip_event_record(dmhip_ctx *ctx, void **event);
int dmhip_event_elapsed_ms(void *start, void *stop, float *ms);
void dmhip_event_free(void *event);

/* Stream-ordered device-to-device copy by a plain streaming kernel (also the
   calibration kernel for HBM byte counters). */
int dmhip_copy_device(dmhip_ctx *ctx, void *dst, const void *src, size_t n);

/* ---------------------------------------------------------------------- */
/* GLM safetensors matrices (src/metal.rs:738-1146)                        */
/* ---------------------------------------------------------------------- */

/* SafeDtype (src/safetensors.rs:171-187), in declaration order. */
enum {
    DMHIP_SAFE_BOOL = 0,
    DMHIP_SAFE_U8 = 1,
    DMHIP_SAFE_I8 = 2,
    DMHIP_SAFE_U16 = 3,
    DMHIP_SAFE_I16 = 4,
    DMHIP_SAFE_F16 = 5,
    DMHIP_SAFE_BF16 = 6,
    DMHIP_SAFE_U32 = 7,
    DMHIP_SAFE_I32 = 8,
    DMHIP_SAFE_F32 = 9,
    DMHIP_SAFE_U64 = 10,
    DMHIP_SAFE_I64 = 11,
    DMHIP_SAFE_F64 = 12,
    DMHIP_SAFE_F8_E4M3 = 13,
    DMHIP_SAFE_F8_E5M2 = 14
};

/* MetalContext::matvec_safetensor_mapped (src/metal.rs:738-881): y = W x for
   a safetensors matrix inside a mapped buffer.  F32 / F16 are
   dmhip_matvec_mapped.  BF16: rows x columns little-endian bf16.  F8_E4M3:
   bytes plus an f32 scale per 128 x 128 block ([ceil(rows/128)]
   [ceil(columns/128)] in `scale_mapping`).  U8: row INT8 (one f32 scale per
   row) or grouped INT4 (ceil(columns/2) bytes per row, low nibble first,
   value (n - 8) * scale), the layout inferred from the byte lengths as
   u8_matrix_encoding does (src/metal.rs:1893-1942).  scale_mapping NULL is
   the reference's None.  Errors and their order as the reference's:
   UnsupportedTensorType "safetensors dtype", InvalidInputLength,
   InvalidOutputLength, Overflow, InvalidByteLength ("BF16", "F8_E4M3FN",
   "F8_E4M3FN scale", "U8 quantized matrix", "U8 quantization scales"),
   MappedRange, EmptyInput ("safetensors matvec", "safetensors U8 matvec"). */
int dmhip_matvec_safetensor_mapped(dmhip_ctx *ctx, uint32_t safe_dtype, size_t rows, size_t columns,
                                   const dmhip_buf *mapping, size_t encoded_offset, size_t encoded_length,
                                   const dmhip_buf *scale_mapping, size_t scale_offset, size_t scale_length,
                                   const float *input, size_t input_len, float *output, size_t output_len);

/* MetalContext::matvec_safetensor (src/metal.rs:883-993, :1070-1146): the
   same from host bytes, with the scales as an f32 slice (NULL for None;
   InvalidVectorLength "safetensors U8 matvec" / "F8_E4M3FN matvec" "scales"
   when missing or of the wrong count). */
int dmhip_matvec_safetensor(dmhip_ctx *ctx, uint32_t safe_dtype, size_t rows, size_t columns,
                            const uint8_t *encoded, size_t encoded_len, const float *scales, size_t scales_len,
                            const float *input, size_t input_len, float *output, size_t output_len);

/* The same with the matrix, scales, x and y in device memory, enqueued on
   the stream (checks as dmhip_matvec_safetensor; one token). */
int dmhip_matvec_safetensor_device(dmhip_ctx *ctx, uint32_t safe_dtype, size_t rows, size_t columns,
                                   const void *weights, size_t weights_len, const float *scales,
                                   size_t scales_len, const float *x, float *y);

/* ---------------------------------------------------------------------- */
/* Decode attention over a KV ring (src/metal.rs:245-277, :1196-1511)      */
/* ---------------------------------------------------------------------- */

/* MetalContext::new_kv_layer (src/metal.rs:1196-1217): two device rings of
   capacity x width floats, capacity = min(sliding_window, max_context) when
   has_window, else max_context.  InvalidAttentionShape for a zero width or
   capacity, Overflow when width * capacity does not fit. */
int dmhip_new_kv_layer(dmhip_ctx *ctx, size_t width, size_t max_context, int has_window,
                       size_t sliding_window, dmhip_kv_layer **out);
/* Waits for the context's stream, then frees both rings. */
void dmhip_kv_layer_free(dmhip_kv_layer *layer);
/* MetalKvLayer::position / capacity / allocated_bytes / clear / truncate
   (src/metal.rs:255-277): host-side bookkeeping, no device work. */
size_t dmhip_kv_layer_position(const dmhip_kv_layer *layer);
size_t dmhip_kv_layer_capacity(const dmhip_kv_layer *layer);
size_t dmhip_kv_layer_allocated_bytes(const dmhip_kv_layer *layer);
void dmhip_kv_layer_clear(dmhip_kv_layer *layer);
void dmhip_kv_layer_truncate(dmhip_kv_layer *layer, size_t position);
/* The layer's width (kv_heads * head_dimension) and the device addresses of
   its rings ([capacity][width] f32, position p in slot p % capacity). */
size_t dmhip_kv_layer_width(const dmhip_kv_layer *layer);
void *dmhip_kv_layer_keys(const dmhip_kv_layer *layer);
void *dmhip_kv_layer_values(const dmhip_kv_layer *layer);

/* MetalContext::append_kv (src/metal.rs:1219-1268): KvPosition unless
   `position` is the layer's position, KvContext when it reaches max_context,
   KvWidth unless both slices hold `width` floats; then slot position %
   capacity takes the key and value and the position advances.  The _device
   form copies from device addresses on the stream (the lengths are the
   caller's statement of what they hold). */
int dmhip_append_kv(dmhip_ctx *ctx, dmhip_kv_layer *layer, size_t position, const float *key,
                    size_t key_len, const float *value, size_t value_len);
int dmhip_append_kv_device(dmhip_ctx *ctx, dmhip_kv_layer *layer, size_t position,
                           const float *key_device, size_t key_len, const float *value_device,
                           size_t value_len);

/* MetalContext::attention_cached (src/metal.rs:1270-1323): one query token
   ([query_heads][head_dimension]) against the layer's last min(position,
   capacity) positions; query head h reads KV head h / (query_heads /
   kv_heads).  Scores are the sequential fma of the reference's fold
   (unscaled), softmax over the window, output [query_heads][head_dimension].
   Checks, in order: InvalidAttentionShape (heads), Overflow, InvalidAttention-
   Shape (query/output lengths), KvWidth (layer width != kv_heads *
   head_dimension), EmptyInput "attention" (position 0).  A non-finite score
   (NaN or +inf) or a window whose scores are all -inf returns NonFinite
   "softmax", as the CPU softmax does (src/cpu.rs:196-225). */
int dmhip_attention_cached(dmhip_ctx *ctx, const float *query, size_t query_len,
                           const dmhip_kv_layer *layer, size_t query_heads, size_t kv_heads,
                           size_t head_dimension, float *output, size_t output_len);
/* The same from and to device memory, enqueued on the stream; the
   non-finite check is read by dmhip_attention_result. */
int dmhip_attention_cached_device(dmhip_ctx *ctx, const float *query_device, size_t query_len,
                                  const dmhip_kv_layer *layer, size_t query_heads, size_t kv_heads,
                                  size_t head_dimension, float *output_device, size_t output_len);
/* Waits for the dmhip_attention_cached_device calls made since the previous
   result (or since a host-slice attention call, which ends that period) and
   returns NonFinite "softmax" when any of them met a non-finite score (its
   output is then not meaningful).  A host-slice attention call made while
   device calls await their result reports for them too: it returns
   NonFinite "softmax" when it or any of them met a non-finite score, and
   the period then has no result left to read. */
int dmhip_attention_result(dmhip_ctx *ctx);

/* MetalContext::attention (src/metal.rs:1325-1385): keys and values are host
   caches of whole positions (keys_len == values_len, a multiple of kv_heads *
   head_dimension); with has_window the last `window` positions are attended.
   Checks as attention_cached, then InvalidAttentionShape "key/value caches
   must have equal whole-position lengths", EmptyInput "attention" (no
   position), EmptyInput "attention window" (window 0). */
int dmhip_attention(dmhip_ctx *ctx, const float *query, size_t query_len, const float *keys,
                    size_t keys_len, const float *values, size_t values_len, size_t query_heads,
                    size_t kv_heads, size_t head_dimension, int has_window, size_t window,
                    float *output, size_t output_len);

/* ---------------------------------------------------------------------- */
/* Routed-expert residency (src/expert.rs)                                 */
/* ---------------------------------------------------------------------- */

/* ExpertLayerLayout (src/expert.rs:44-51): byte ranges inside the source. */
typedef struct dmhip_expert_layer_layout {
    size_t expert_count;
    uint64_t gate_up_offset;
    size_t gate_up_bytes;
    uint64_t down_offset;
    size_t down_bytes;
} dmhip_expert_layer_layout;

/* ExpertCacheStats (src/expert.rs:53-62).  io_wait_ns is the time spent
   bringing missed experts in: for a file-backed cache the host's wall time in
   the positional reads (and in waiting for a staging buffer), as
   src/expert.rs:220 measures it; for a memory-backed cache, whose uploads the
   host never waits for, the summed device-measured duration of the uploads. */
typedef struct dmhip_expert_cache_stats {
    uint64_t hits;
    uint64_t misses;
    uint64_t evictions;
    uint64_t reads;
    uint64_t bytes_read;
    uint64_t io_wait_ns;
    uint64_t resident_bytes;
} dmhip_expert_cache_stats;

/* ExpertCache::new (src/expert.rs:88-128) over host memory: `source` holds the
   expert tensors at the layout offsets (ideally pinned memory from
   dmhip_host_alloc_pinned, so that uploads are asynchronous DMA) and must
   stay valid while the cache lives.  Each layer gets `slots_per_layer` HBM
   slots of gate_up_bytes + down_bytes. */
int dmhip_expert_cache_new(dmhip_ctx *ctx, const void *source, size_t source_len,
                           const dmhip_expert_layer_layout *layouts, size_t layer_count,
                           size_t slots_per_layer, dmhip_expert_cache **out);

/* ExpertCache::new (src/expert.rs:88-128) over a file, the reference's
   Arc<File>: a miss reads the expert's gate_up and down ranges (absolute
   file offsets, src/expert.rs:203-215) with two parallel positional reads
   into one of four pinned staging buffers and copies it into the slot
   asynchronously, so host memory stays bounded by the ring.  The descriptor
   must stay open while the cache lives.  A short file is found when an
   expert is first read: that acquire fails with Io (os_error 0, unexpected
   end of file), as read_exact_at does (src/expert.rs:241-256). */
int dmhip_expert_cache_new_file(dmhip_ctx *ctx, int fd, const dmhip_expert_layer_layout *layouts,
                                size_t layer_count, size_t slots_per_layer, dmhip_expert_cache **out);

/* Frees the slots after waiting for the cache's own uploads and for the
   work released from its slots. */
void dmhip_expert_cache_free(dmhip_expert_cache *cache);
/* ExpertCache::stats (src/expert.rs:130-132); waits for uploads in flight so
   that their duration is part of io_wait_ns. */
int dmhip_expert_cache_stats_get(dmhip_expert_cache *cache, dmhip_expert_cache_stats *stats);
size_t dmhip_expert_cache_slots_per_layer(const dmhip_expert_cache *cache);

/* ExpertCache::with_expert, split into acquire/release for a C caller
   (src/expert.rs:138-164).  acquire checks `cancelled` (may be NULL) before
   and after, finds or loads the expert into a slot (the LRU of
   src/expert.rs:166-229; a miss enqueues the upload and makes the compute
   stream wait for it), pins the slot and returns its gate_up and down bytes
   as buffers owned by the cache -- the &MetalOwnedBuffer pair the reference
   hands its closure, usable with dmhip_matvec_owned and dmhip_buffer_read
   (dmhip_buffer_free ignores them).  Work that reads the slot must be
   enqueued on the context's compute stream (every entry point of the
   context does) before the matching release.  Pins count: each acquire
   needs its own release, and a pinned slot is never evicted (all slots of
   the layer pinned: AllSlotsPinned).  release records the end of the work
   enqueued so far as the slot's last use (a later upload into it waits for
   it) and drops one pin; releasing an unpinned slot is InvalidArgument. */
int dmhip_expert_acquire(dmhip_expert_cache *cache, size_t layer, size_t expert,
                         const volatile int *cancelled, size_t *slot, const dmhip_buf **gate_up,
                         const dmhip_buf **down);
int dmhip_expert_release(dmhip_expert_cache *cache, size_t layer, size_t slot);

/* One routed-expert layer at decode for `batch` tokens (1..16), the
   structure of src/gemma4/cpu.rs:574-612 with the GLM SiLU expert
   (src/glm52/expert.rs:260-267): router -> top-k softmax -> for each
   selected expert (acquired through the cache in token order, then
   selection order) gate_up, silu*up, down -> y = fma(out, p, y) in selection
   order.  Expert gate_up rows are [gate; up] (2*width rows of `hidden`
   columns), down rows are `hidden` rows of `width` columns.  x and y are
   device [batch][hidden]; ids/probabilities receive host [batch][k].
   The ids, and their order, are those of the reference's sequential router
   fold; routers of up to 8192 columns and 256 experts compute the logits
   in parallel with a proven bound on their distance from that fold (the
   exact fold runs for the rows the bound cannot order), so the
   probabilities can differ from the reference's in the last bits.
   Non-finite router logits return NonFinite before any expert is acquired.
   The call returns after the layer finished. */
int dmhip_moe_layer(dmhip_ctx *ctx, dmhip_expert_cache *cache, size_t layer, size_t batch,
                    size_t hidden, size_t width, size_t experts, size_t k,
                    const uint16_t *router_bf16, uint32_t gate_up_type, uint32_t down_type,
                    const float *x, float *y, uint32_t *ids, float *probabilities);

#ifdef __cplusplus
}
#endif
#endif
