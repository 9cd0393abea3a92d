/*
 * dm_oracle.h -- CPU restatement of DiskMule's reference operators.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * MI355X kernels in diskmule_amd/.  Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load it.  The product path never
 * calls it, links it or falls back to it.
 *
 * Every function restates one function of the Rust reference
 * (/root/reference, crate `diskmule`) and cites the file:line it follows.
 * The arithmetic keeps the reference's operation order and rounding:
 * compiled with -ffp-contract=off, `mul_add` is fmaf (correctly rounded),
 * `exp` is expf, `sqrt().recip()` is 1.0f / sqrtf.
 *
 * Pinning (what checks each function against something other than itself):
 *   orc_f16_to_f32           all 65536 patterns vs numpy float16->float32
 *   orc_scale_min_q4_k       src/cpu.rs:732-739 known answer + numpy restatement
 *   orc_dequantize           src/cpu.rs:670-753 known answers + numpy
 *                            restatement that follows metal/kernels.metal
 *   orc_matvec               src/cpu.rs:755-764 known answer + exact-rational
 *                            brute force of the sequential fma fold
 *   orc_argmax / top_k       src/cpu.rs:819-833 known answers + numpy lexsort
 *   orc_softmax_in_place     src/cpu.rs:819-825 known answer; exp-dependent bits
 *                            are tolerance-checked (platform expf)
 *   orc_rms_norm             src/cpu.rs:778-795 known answer (bit-exact)
 *   orc_matvec_bf16          closed form bits<<16 + exact-rational brute force
 *   orc_lru_*                src/expert.rs:266-325 known answer + Python model
 *   orc_dense_ffn / orc_moe_layer / orc_gemm_tokenwise
 *                            compositions of the functions above, checked by
 *                            recomposing them from the pinned parts in numpy
 *   orc_st_*                 src/glm52/cpu.rs:1551-1606 and src/metal.rs:2315-2486
 *                            known answers; all 256 E4M3FN patterns against the
 *                            OCP formula and its landmark values; exact-rational
 *                            brute force of the product-then-sum fold
 *   orc_attention            src/gemma4/cpu.rs:967-985 and src/metal.rs:2499-2570
 *                            known answers; float64 closed form from the same
 *                            fp32 scores; equal-value and one-hot invariants;
 *                            ring-rotation invariance (bit-exact)
 */
#ifndef DM_ORACLE_H
#define DM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* CpuError variants, src/cpu.rs:10-96 (subset on this path). */
enum {
    ORC_OK = 0,
    ORC_UNSUPPORTED_TYPE = 1,
    ORC_INVALID_ELEMENT_COUNT = 2,
    ORC_INVALID_BYTE_LENGTH = 3,
    ORC_OVERFLOW = 4,
    ORC_INVALID_INPUT_LENGTH = 5,
    ORC_INVALID_OUTPUT_LENGTH = 6,
    ORC_EMPTY_INPUT = 7,
    ORC_INVALID_VECTOR_LENGTH = 8,
    ORC_NON_FINITE = 9,
    ORC_INVALID_TOP_K = 10,
    ORC_INVALID_POSITIVE_PARAMETER = 11,
    ORC_INVALID_LAYER = 12,
    ORC_INVALID_EXPERT = 13,
    ORC_ALL_SLOTS_PINNED = 14,
    ORC_NO_SLOTS = 15,
    ORC_INVALID_ROPE_SHAPE = 16,
    ORC_INVALID_ROPE_PAIRS = 17
};

/* ggml type ids, src/gguf.rs:295-318. */
enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q5_0 = 6,
    ORC_Q5_1 = 7, ORC_Q8_0 = 8, ORC_Q8_1 = 9, ORC_Q2_K = 10, ORC_Q3_K = 11,
    ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_Q8_K = 15, ORC_I8 = 24,
    ORC_I16 = 25, ORC_I32 = 26, ORC_I64 = 27, ORC_F64 = 28, ORC_BF16 = 30
};

int orc_type_layout(uint32_t ggml_type, uint64_t *block_elements, uint64_t *block_bytes);
int orc_row_byte_len(uint32_t ggml_type, uint64_t elements, uint64_t *row_bytes);

float orc_f16_to_f32(uint16_t bits);
void orc_scale_min_q4_k(size_t index, const uint8_t *scales, uint8_t *scale, uint8_t *minimum);
int orc_dequantize(uint32_t ggml_type, const uint8_t *encoded, size_t encoded_len,
                   float *output, size_t output_len);
int orc_matvec(uint32_t ggml_type, size_t rows, size_t columns, const uint8_t *encoded,
               size_t encoded_len, const float *input, size_t input_len, float *output,
               size_t output_len, int threads);
int orc_matvec_bf16(size_t rows, size_t columns, const uint16_t *weights, const float *input,
                    float *output, int threads);

int orc_argmax(const float *values, size_t count, size_t *index);
int orc_softmax_in_place(float *values, size_t count);
int orc_top_k_softmax(const float *logits, size_t count, size_t k, size_t *indices,
                      float *probabilities);
int orc_rms_norm(const float *input, size_t count, const float *weight, size_t weight_len,
                 float epsilon, float *output, size_t output_len);
float orc_silu(float value);
/* src/cpu.rs:263-273: values[i] = cap * tanh(values[i] / cap) in place;
   InvalidPositiveParameter unless cap is finite and > 0. */
int orc_softcap_in_place(float *values, size_t count, float cap);
float orc_gelu_tanh(float value);
void orc_gelu_mul(const float *gate, const float *up, size_t count, float *output);
int orc_rope_neox_in_place(float *values, size_t count, size_t heads, size_t head_dimension,
                           size_t rotated_pairs, size_t position, float theta);
void orc_silu_mul_glm(const float *gate, const float *up, size_t count, float *output);

int orc_dense_ffn(size_t batch, size_t hidden, size_t ffn, uint32_t gate_type,
                  const uint8_t *gate, uint32_t up_type, const uint8_t *up,
                  uint32_t down_type, const uint8_t *down, const float *hidden_in,
                  float epsilon, float *output, int threads);

int orc_moe_layer(size_t batch, size_t hidden, size_t expert_width, size_t experts, size_t k,
                  const uint16_t *router, uint32_t gate_up_type, const uint8_t *gate_up_all,
                  uint32_t down_type, const uint8_t *down_all, const float *tokens,
                  size_t *selected, float *weights, float *output, int threads);

int orc_gemm_tokenwise(uint32_t ggml_type, size_t m, size_t n, size_t k,
                       const uint16_t *activations_bf16, const uint8_t *encoded, float *output,
                       int threads);

/* GLM safetensors matrices (src/glm52/cpu.rs:1180-1420, src/metal.rs:1893-1942).
   Formats: BF16 rows; F8_E4M3FN rows with one f32 scale per 128 x 128 block
   (scales [ceil(rows/128)][ceil(columns/128)]); U8 row-INT8 (one scale per
   row); U8 grouped INT4 (two codes per byte, low nibble first, (n - 8) *
   scale[row][column / group_size], rows of ceil(columns / 2) bytes). */
enum { ORC_ST_BF16 = 0, ORC_ST_F8_E4M3 = 1, ORC_ST_INT8_ROW = 2, ORC_ST_INT4_GROUPED = 3 };
/* decode_f8_e4m3fn (src/glm52/cpu.rs:1397-1410): returns 0 and sets *value,
   or ORC_NON_FINITE for the NaN patterns 0x7f / 0xff. */
int orc_st_decode_f8_e4m3fn(uint8_t bits, float *value);
/* u8_matrix_encoding (src/metal.rs:1893-1942): ORC_OK with *format
   ORC_ST_INT8_ROW or ORC_ST_INT4_GROUPED (and *group_size / *scale_columns),
   else ORC_INVALID_BYTE_LENGTH (with *expected / *actual, and *scales_bad = 1
   when the scale length is what failed) or ORC_OVERFLOW. */
int orc_st_u8_encoding(size_t rows, size_t columns, size_t encoded_len, size_t scale_len, int *format,
                       size_t *group_size, size_t *scale_columns, size_t *expected, size_t *actual,
                       int *scales_bad);
/* One row dequantized (matrix_row_into_untracked / read_quantized_row /
   read_fp8_row / read_dense_values), then y[r] = sum_c w[c] * x[c] as a
   product followed by a sequential add (src/glm52/cpu.rs:1180-1190).
   group_size is used by ORC_ST_INT4_GROUPED only. */
int orc_st_matvec(int format, size_t rows, size_t columns, const uint8_t *encoded, const float *scales,
                  size_t group_size, const float *input, float *output);
int orc_st_dequantize_row(int format, size_t rows, size_t columns, const uint8_t *encoded, const float *scales,
                          size_t group_size, size_t row, float *output);

/* Decode attention of one query token over a KV ring, src/gemma4/cpu.rs:900-946
   (`attend`) with the ring addressing of metal/kernels.metal:486-578: position
   p lives in slot p % capacity of keys/values ([capacity][width] row-major,
   width = kv_heads * head_dimension), and the query attends positions
   [start, start + visible).  Output is [query_heads][head_dimension].
   EmptyInput when visible is 0; NonFinite from softmax_in_place. */
int orc_attention(const float *query, const float *keys, const float *values, size_t capacity,
                  size_t width, size_t query_heads, size_t kv_heads, size_t head_dimension,
                  size_t start, size_t visible, float *output);

/* src/expert.rs:44-229 bookkeeping, without the byte movement. */
typedef struct orc_lru orc_lru;
int orc_lru_new(size_t layers, const size_t *expert_counts, size_t slots_per_layer,
                uint64_t gate_up_bytes, uint64_t down_bytes, orc_lru **out);
void orc_lru_free(orc_lru *cache);
int orc_lru_acquire(orc_lru *cache, size_t layer, size_t expert, size_t *slot, int *hit,
                    int *evicted, size_t *evicted_expert);
void orc_lru_set_pinned(orc_lru *cache, size_t layer, size_t slot, int pinned);
void orc_lru_stats(const orc_lru *cache, uint64_t *hits, uint64_t *misses, uint64_t *evictions,
                   uint64_t *reads, uint64_t *bytes_read, uint64_t *resident_bytes);

#ifdef __cplusplus
}
#endif
#endif
