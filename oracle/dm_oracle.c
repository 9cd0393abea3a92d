/*
 * dm_oracle.c -- CPU restatement of DiskMule's reference operators.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker and the timed CPU baseline).
 * The product library in diskmule_amd/ never links or calls this file.
 *
 * Build: -O2 -ffp-contract=off (no FMA contraction: Rust never contracts),
 * explicit fmaf() wherever the reference calls f32::mul_add.
 * Citations are file:line into the reference crate.
 */
#include "dm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------- */
/* src/gguf.rs:321-358  TensorType::layout and row_byte_len                */
/* ---------------------------------------------------------------------- */
int orc_type_layout(uint32_t t, uint64_t *be, uint64_t *bb)
{
    uint64_t e, b;
    switch (t) {
    case ORC_F32: e = 1; b = 4; break;
    case ORC_F16: case ORC_BF16: e = 1; b = 2; break;
    case ORC_Q4_0: e = 32; b = 18; break;
    case ORC_Q4_1: e = 32; b = 20; break;
    case ORC_Q5_0: e = 32; b = 22; break;
    case ORC_Q5_1: e = 32; b = 24; break;
    case ORC_Q8_0: e = 32; b = 34; break;
    case ORC_Q8_1: e = 32; b = 40; break;
    case ORC_Q2_K: e = 256; b = 84; break;
    case ORC_Q3_K: e = 256; b = 110; break;
    case ORC_Q4_K: e = 256; b = 144; break;
    case ORC_Q5_K: e = 256; b = 176; break;
    case ORC_Q6_K: e = 256; b = 210; break;
    case ORC_Q8_K: e = 256; b = 292; break;
    case ORC_I8: e = 1; b = 1; break;
    case ORC_I16: e = 1; b = 2; break;
    case ORC_I32: e = 1; b = 4; break;
    case ORC_I64: case ORC_F64: e = 1; b = 8; break;
    default: return ORC_UNSUPPORTED_TYPE;
    }
    if (be) *be = e;
    if (bb) *bb = b;
    return ORC_OK;
}

int orc_row_byte_len(uint32_t t, uint64_t elements, uint64_t *row_bytes)
{
    uint64_t be, bb;
    if (orc_type_layout(t, &be, &bb) != ORC_OK) return ORC_UNSUPPORTED_TYPE;
    if (elements % be != 0) return ORC_INVALID_ELEMENT_COUNT;
    uint64_t blocks = elements / be;
    if (bb != 0 && blocks > UINT64_MAX / bb) return ORC_INVALID_ELEMENT_COUNT; /* checked_mul -> None */
    *row_bytes = blocks * bb;
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* src/cpu.rs:647-660  f16_to_f32                                           */
/* ---------------------------------------------------------------------- */
static float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_f16_to_f32(uint16_t value)
{
    uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
    uint32_t exponent = (value >> 10) & 0x1fu;
    uint32_t fraction = value & 0x03ffu;
    if (exponent == 0 && fraction == 0) return bits_to_f32(sign);
    if (exponent == 0) {
        /* fraction as f32 * 2^-24, exact */
        float magnitude = (float)fraction * 5.9604644775390625e-08f;
        return sign == 0 ? magnitude : -magnitude;
    }
    if (exponent == 0x1f) return bits_to_f32(sign | 0x7f800000u | (fraction << 13));
    return bits_to_f32(sign | ((exponent + 112u) << 23) | (fraction << 13));
}

static uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---------------------------------------------------------------------- */
/* src/cpu.rs:607-616  scale_min_q4_k                                       */
/* ---------------------------------------------------------------------- */
void orc_scale_min_q4_k(size_t index, const uint8_t *s, uint8_t *scale, uint8_t *minimum)
{
    if (index < 4) {
        *scale = s[index] & 0x3f;
        *minimum = s[index + 4] & 0x3f;
    } else {
        *scale = (uint8_t)((s[index + 4] & 0x0f) | ((s[index - 4] >> 6) << 4));
        *minimum = (uint8_t)((s[index + 4] >> 4) | ((s[index] >> 6) << 4));
    }
}

/* ---------------------------------------------------------------------- */
/* src/cpu.rs:546-645  block decoders                                       */
/* ---------------------------------------------------------------------- */
static void decode_f32(const uint8_t *enc, float *out, size_t n)      /* :546-550 */
{
    for (size_t i = 0; i < n; i++) memcpy(&out[i], enc + 4 * i, 4);
}

static void decode_f16(const uint8_t *enc, float *out, size_t n)      /* :552-558 */
{
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(le16(enc + 2 * i));
}

static void decode_q5_0(const uint8_t *enc, float *out, size_t n)     /* :560-574 */
{
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *block = enc + 22 * b;
        float *values = out + 32 * b;
        float delta = orc_f16_to_f32(le16(block));
        uint32_t high_bits = (uint32_t)block[2] | ((uint32_t)block[3] << 8) |
                             ((uint32_t)block[4] << 16) | ((uint32_t)block[5] << 24);
        for (int index = 0; index < 16; index++) {
            uint8_t packed = block[6 + index];
            uint8_t low_high_bit = (uint8_t)(((high_bits >> index) << 4) & 0x10);
            uint8_t high_high_bit = (uint8_t)((high_bits >> (index + 12)) & 0x10);
            int32_t low = (int32_t)((packed & 0x0f) | low_high_bit) - 16;
            int32_t high = (int32_t)((packed >> 4) | high_high_bit) - 16;
            values[index] = delta * (float)low;
            values[index + 16] = delta * (float)high;
        }
    }
}

static void decode_q8_0(const uint8_t *enc, float *out, size_t n)     /* :576-583 */
{
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *block = enc + 34 * b;
        float delta = orc_f16_to_f32(le16(block));
        for (int i = 0; i < 32; i++) out[32 * b + i] = delta * (float)(int8_t)block[2 + i];
    }
}

static void decode_q4_k(const uint8_t *enc, float *out, size_t n)     /* :585-605 */
{
    for (size_t b = 0; b < n / 256; b++) {
        const uint8_t *block = enc + 144 * b;
        float *values = out + 256 * b;
        float delta = orc_f16_to_f32(le16(block));
        float minimum = orc_f16_to_f32(le16(block + 2));
        const uint8_t *scales = block + 4;
        const uint8_t *quants = block + 16;
        for (int group_pair = 0; group_pair < 4; group_pair++) {
            uint8_t scale_low, min_low, scale_high, min_high;
            orc_scale_min_q4_k((size_t)group_pair * 2, scales, &scale_low, &min_low);
            orc_scale_min_q4_k((size_t)group_pair * 2 + 1, scales, &scale_high, &min_high);
            int quant_offset = group_pair * 32;
            int value_offset = group_pair * 64;
            for (int index = 0; index < 32; index++) {
                uint8_t packed = quants[quant_offset + index];
                /* ((delta * sc) * q) - (minimum * m), left to right, no FMA */
                values[value_offset + index] =
                    delta * (float)scale_low * (float)(packed & 0x0f) - minimum * (float)min_low;
                values[value_offset + index + 32] =
                    delta * (float)scale_high * (float)(packed >> 4) - minimum * (float)min_high;
            }
        }
    }
}

static void decode_q6_k(const uint8_t *enc, float *out, size_t n)     /* :618-645 */
{
    for (size_t b = 0; b < n / 256; b++) {
        const uint8_t *block = enc + 210 * b;
        const uint8_t *low_all = block;
        const uint8_t *high_all = block + 128;
        const uint8_t *scales_all = block + 192;
        float delta = orc_f16_to_f32(le16(block + 208));
        for (int half = 0; half < 2; half++) {
            const uint8_t *low = low_all + half * 64;
            const uint8_t *high = high_all + half * 32;
            const int8_t *scales = (const int8_t *)(scales_all + half * 8);
            float *values = out + 256 * b + half * 128;
            for (int index = 0; index < 32; index++) {
                int scale_pair = index / 16;
                uint8_t q1 = (uint8_t)((low[index] & 0x0f) | ((high[index] & 0x03) << 4));
                uint8_t q2 = (uint8_t)((low[index + 32] & 0x0f) | (((high[index] >> 2) & 0x03) << 4));
                uint8_t q3 = (uint8_t)((low[index] >> 4) | (((high[index] >> 4) & 0x03) << 4));
                uint8_t q4 = (uint8_t)((low[index + 32] >> 4) | (((high[index] >> 6) & 0x03) << 4));
                values[index] = delta * (float)scales[scale_pair] * ((float)q1 - 32.0f);
                values[index + 32] = delta * (float)scales[scale_pair + 2] * ((float)q2 - 32.0f);
                values[index + 64] = delta * (float)scales[scale_pair + 4] * ((float)q3 - 32.0f);
                values[index + 96] = delta * (float)scales[scale_pair + 6] * ((float)q4 - 32.0f);
            }
        }
    }
}

/* ---------------------------------------------------------------------- */
/* src/cpu.rs:312-343  dequantize                                           */
/* ---------------------------------------------------------------------- */
int orc_dequantize(uint32_t t, const uint8_t *encoded, size_t encoded_len, float *output,
                   size_t output_len)
{
    uint64_t expected;
    uint64_t be;
    if (orc_type_layout(t, &be, NULL) != ORC_OK) return ORC_UNSUPPORTED_TYPE;
    int status = orc_row_byte_len(t, output_len, &expected);
    if (status != ORC_OK) return status;
    if (encoded_len != expected) return ORC_INVALID_BYTE_LENGTH;
    switch (t) {
    case ORC_F32: decode_f32(encoded, output, output_len); break;
    case ORC_F16: decode_f16(encoded, output, output_len); break;
    case ORC_Q5_0: decode_q5_0(encoded, output, output_len); break;
    case ORC_Q8_0: decode_q8_0(encoded, output, output_len); break;
    case ORC_Q4_K: decode_q4_k(encoded, output, output_len); break;
    case ORC_Q6_K: decode_q6_k(encoded, output, output_len); break;
    default: return ORC_UNSUPPORTED_TYPE;
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* src/cpu.rs:345-399  matvec: per row, dequantize into scratch, then a     */
/* sequential fma fold from column 0.  Rows are split across threads the   */
/* way rayon's par_chunks_exact does; per-row results do not depend on it. */
/* ---------------------------------------------------------------------- */
typedef struct {
    uint32_t type;
    size_t row_begin, row_end, columns, row_bytes;
    const uint8_t *encoded;
    const float *input;
    float *output;
    int status;
} matvec_job;

static void *matvec_worker(void *arg)
{
    matvec_job *job = (matvec_job *)arg;
    float *row = (float *)malloc(sizeof(float) * (job->columns ? job->columns : 1));
    if (!row) { job->status = ORC_OVERFLOW; return NULL; }
    for (size_t r = job->row_begin; r < job->row_end; r++) {
        int status = orc_dequantize(job->type, job->encoded + r * job->row_bytes, job->row_bytes,
                                    row, job->columns);
        if (status != ORC_OK) { job->status = status; break; }
        float sum = 0.0f;
        for (size_t c = 0; c < job->columns; c++) sum = fmaf(row[c], job->input[c], sum);
        job->output[r] = sum;
    }
    free(row);
    return NULL;
}

static int run_rows(matvec_job *proto, size_t rows, int threads, void *(*fn)(void *))
{
    if (threads < 1) threads = 1;
    if ((size_t)threads > rows) threads = rows ? (int)rows : 1;
    matvec_job jobs[256];
    pthread_t tids[256];
    if (threads > 256) threads = 256;
    size_t per = (rows + (size_t)threads - 1) / (size_t)threads;
    int launched = 0;
    for (int t = 0; t < threads; t++) {
        jobs[t] = *proto;
        jobs[t].row_begin = (size_t)t * per;
        jobs[t].row_end = jobs[t].row_begin + per > rows ? rows : jobs[t].row_begin + per;
        jobs[t].status = ORC_OK;
        if (jobs[t].row_begin >= jobs[t].row_end) break;
        if (threads == 1) { fn(&jobs[t]); launched = 1; break; }
        pthread_create(&tids[t], NULL, fn, &jobs[t]);
        launched = t + 1;
    }
    if (threads > 1)
        for (int t = 0; t < launched; t++) pthread_join(tids[t], NULL);
    for (int t = 0; t < launched; t++)
        if (jobs[t].status != ORC_OK) return jobs[t].status;
    return ORC_OK;
}

int orc_matvec(uint32_t t, size_t rows, size_t columns, const uint8_t *encoded,
               size_t encoded_len, const float *input, size_t input_len, float *output,
               size_t output_len, int threads)
{
    if (input_len != columns) return ORC_INVALID_INPUT_LENGTH;
    if (output_len != rows) return ORC_INVALID_OUTPUT_LENGTH;
    uint64_t row_bytes;
    if (orc_type_layout(t, NULL, NULL) != ORC_OK) {
        /* row_byte_len of an unknown id cannot be formed; the reference's
           TensorType cannot hold one, so report the type as unsupported */
        return ORC_UNSUPPORTED_TYPE;
    }
    int status = orc_row_byte_len(t, columns, &row_bytes);
    if (status != ORC_OK) return status;
    if (rows != 0 && row_bytes > SIZE_MAX / rows) return ORC_OVERFLOW;
    if (encoded_len != rows * row_bytes) return ORC_INVALID_BYTE_LENGTH;
    matvec_job proto = {t, 0, 0, columns, (size_t)row_bytes, encoded, input, output, ORC_OK};
    return run_rows(&proto, rows, threads, matvec_worker);
}

/* bf16 router rows: f32::from_bits(bits << 16) (src/glm52/expert.rs:429-433,
   metal/kernels.metal:254), then the same sequential fma fold as
   src/cpu.rs:391-394.  src/cpu.rs has no BF16 arm, so this is the closed-form
   extension of matvec to bf16. */
typedef struct {
    size_t row_begin, row_end, columns;
    const uint16_t *weights;
    const float *input;
    float *output;
} bf16_job;

static void *bf16_worker(void *arg)
{
    bf16_job *job = (bf16_job *)arg;
    for (size_t r = job->row_begin; r < job->row_end; r++) {
        float sum = 0.0f;
        for (size_t c = 0; c < job->columns; c++) {
            float w = bits_to_f32((uint32_t)job->weights[r * job->columns + c] << 16);
            sum = fmaf(w, job->input[c], sum);
        }
        job->output[r] = sum;
    }
    return NULL;
}

int orc_matvec_bf16(size_t rows, size_t columns, const uint16_t *weights, const float *input,
                    float *output, int threads)
{
    if (threads < 1) threads = 1;
    if ((size_t)threads > rows) threads = rows ? (int)rows : 1;
    if (threads > 256) threads = 256;
    bf16_job jobs[256];
    pthread_t tids[256];
    size_t per = (rows + (size_t)threads - 1) / (size_t)threads;
    int launched = 0;
    for (int t = 0; t < threads; t++) {
        jobs[t] = (bf16_job){(size_t)t * per, 0, columns, weights, input, output};
        jobs[t].row_end = jobs[t].row_begin + per > rows ? rows : jobs[t].row_begin + per;
        if (jobs[t].row_begin >= jobs[t].row_end) break;
        if (threads == 1) { bf16_worker(&jobs[t]); break; }
        pthread_create(&tids[t], NULL, bf16_worker, &jobs[t]);
        launched = t + 1;
    }
    for (int t = 0; t < launched; t++) pthread_join(tids[t], NULL);
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* total_cmp (Rust core::f32::total_cmp): map the bits to a signed key.    */
/* ---------------------------------------------------------------------- */
static int32_t total_key(float v)
{
    int32_t bits;
    memcpy(&bits, &v, 4);
    bits ^= (int32_t)(((uint32_t)(bits >> 31)) >> 1);
    return bits;
}

/* src/cpu.rs:275-293  argmax: first maximum under total_cmp */
int orc_argmax(const float *values, size_t count, size_t *index)
{
    if (count == 0) return ORC_EMPTY_INPUT;
    for (size_t i = 0; i < count; i++)
        if (!isfinite(values[i])) return ORC_NON_FINITE;
    size_t best = 0;
    int32_t best_key = total_key(values[0]);
    for (size_t i = 1; i < count; i++) {
        int32_t key = total_key(values[i]);
        if (key > best_key) { best_key = key; best = i; }
    }
    *index = best;
    return ORC_OK;
}

/* src/cpu.rs:195-230  softmax_in_place */
int orc_softmax_in_place(float *values, size_t count)
{
    if (count == 0) return ORC_EMPTY_INPUT;
    for (size_t i = 0; i < count; i++)
        if (isnan(values[i]) || values[i] == INFINITY) return ORC_NON_FINITE;
    float maximum = -INFINITY;
    for (size_t i = 0; i < count; i++) maximum = fmaxf(maximum, values[i]);
    if (maximum == -INFINITY) return ORC_NON_FINITE;
    float sum = 0.0f;
    for (size_t i = 0; i < count; i++) {
        values[i] = expf(values[i] - maximum);
        sum += values[i];
    }
    if (!isfinite(sum) || sum <= 0.0f) return ORC_NON_FINITE;
    for (size_t i = 0; i < count; i++) values[i] /= sum;
    return ORC_OK;
}

typedef struct { float value; size_t index; } ranked;

static int ranked_cmp(const void *a, const void *b)
{
    const ranked *l = (const ranked *)a, *r = (const ranked *)b;
    int32_t kl = total_key(l->value), kr = total_key(r->value);
    /* right.1.total_cmp(left.1): descending value */
    if (kr != kl) return kr > kl ? 1 : -1;
    /* then left.0.cmp(right.0): ascending index */
    return l->index < r->index ? -1 : (l->index > r->index ? 1 : 0);
}

/* src/cpu.rs:232-260  top_k_softmax */
int orc_top_k_softmax(const float *logits, size_t count, size_t k, size_t *indices,
                      float *probabilities)
{
    if (k == 0 || k > count) return ORC_INVALID_TOP_K;
    for (size_t i = 0; i < count; i++)
        if (!isfinite(logits[i])) return ORC_NON_FINITE;
    ranked *sel = (ranked *)malloc(sizeof(ranked) * count);
    if (!sel) return ORC_OVERFLOW;
    for (size_t i = 0; i < count; i++) { sel[i].value = logits[i]; sel[i].index = i; }
    qsort(sel, count, sizeof(ranked), ranked_cmp);
    for (size_t i = 0; i < k; i++) probabilities[i] = sel[i].value;
    int status = orc_softmax_in_place(probabilities, k);
    for (size_t i = 0; i < k; i++) indices[i] = sel[i].index;
    free(sel);
    return status;
}

/* src/cpu.rs:98-142  rms_norm */
int orc_rms_norm(const float *input, size_t count, const float *weight, size_t weight_len,
                 float epsilon, float *output, size_t output_len)
{
    if (count == 0) return ORC_EMPTY_INPUT;
    if (output_len != count) return ORC_INVALID_VECTOR_LENGTH;
    if (weight && weight_len != count) return ORC_INVALID_VECTOR_LENGTH;
    if (!isfinite(epsilon) || epsilon <= 0.0f) return ORC_INVALID_POSITIVE_PARAMETER;
    float sum_squares = 0.0f;
    for (size_t i = 0; i < count; i++) sum_squares = fmaf(input[i], input[i], sum_squares);
    float inverse_rms = 1.0f / sqrtf(sum_squares / (float)count + epsilon);
    if (!isfinite(inverse_rms)) return ORC_NON_FINITE;
    if (weight) {
        for (size_t i = 0; i < count; i++) output[i] = input[i] * weight[i] * inverse_rms;
    } else {
        for (size_t i = 0; i < count; i++) output[i] = input[i] * inverse_rms;
    }
    return ORC_OK;
}

/* src/qwen35/cpu.rs:982-993  stable sigmoid and silu */
float orc_silu(float value)
{
    float sigmoid;
    if (value >= 0.0f) {
        sigmoid = 1.0f / (1.0f + expf(-value));
    } else {
        float exponential = expf(value);
        sigmoid = exponential / (1.0f + exponential);
    }
    return value * sigmoid;
}

/* src/cpu.rs:263-273  logit softcap: the division, tanh and product each
   round once in f32 (Rust's f32::tanh is the C library's tanhf). */
int orc_softcap_in_place(float *values, size_t count, float cap)
{
    if (!isfinite(cap) || cap <= 0.0f) return ORC_INVALID_POSITIVE_PARAMETER;
    for (size_t i = 0; i < count; i++) {
        float q = values[i] / cap;
        values[i] = cap * tanhf(q);
    }
    return ORC_OK;
}

/* src/cpu.rs:144-149  Gemma 4's gelu_pytorch_tanh,
   0.5 v (1 + tanh(0.7978846 (v + 0.044715 v^3))): Rust's powi(3) multiplies
   (v v) v, f32::tanh is the C library's tanhf, each operation rounds once. */
float orc_gelu_tanh(float value)
{
    float cubic = (value * value) * value;
    float inner = 0.7978846f * (value + 0.044715f * cubic);
    return (0.5f * value) * (1.0f + tanhf(inner));
}

/* gelu_tanh(gate) * up, as the reference's Metal test states the CPU side
   of MetalContext::gelu_mul (src/metal.rs:2201-2209). */
void orc_gelu_mul(const float *gate, const float *up, size_t count, float *output)
{
    for (size_t i = 0; i < count; i++) output[i] = orc_gelu_tanh(gate[i]) * up[i];
}

/* src/cpu.rs:151-193  NeoX rotary embedding in place: for each head and
   pair p < rotated_pairs, angle = position * powf(theta, -(2p) / hd) (f32
   division, powf, product), (sin, cos) = (sinf, cosf)(angle) (Rust's
   f32::sin_cos), then first' = first cos - second sin, second' = first sin +
   second cos, no fused operations. */
int orc_rope_neox_in_place(float *values, size_t count, size_t heads, size_t head_dimension,
                           size_t rotated_pairs, size_t position, float theta)
{
    size_t length;
    if (__builtin_mul_overflow(heads, head_dimension, &length) || length != count) return ORC_INVALID_ROPE_SHAPE;
    if (head_dimension % 2 != 0 || rotated_pairs > head_dimension / 2) return ORC_INVALID_ROPE_PAIRS;
    if (!isfinite(theta) || theta <= 0.0f) return ORC_INVALID_POSITIVE_PARAMETER;
    size_t half = head_dimension / 2;
    for (size_t h = 0; h < heads; h++) {
        float *head = values + h * head_dimension;
        for (size_t pair = 0; pair < rotated_pairs; pair++) {
            float exponent = -(float)(2 * pair) / (float)head_dimension;
            float angle = (float)position * powf(theta, exponent);
            float sine = sinf(angle), cosine = cosf(angle);
            float first = head[pair], second = head[half + pair];
            head[pair] = first * cosine - second * sine;
            head[half + pair] = first * sine + second * cosine;
        }
    }
    return ORC_OK;
}

/* src/glm52/expert.rs:260-267  (gate / (1 + exp(-gate))) * up */
void orc_silu_mul_glm(const float *gate, const float *up, size_t count, float *output)
{
    for (size_t i = 0; i < count; i++) output[i] = (gate[i] / (1.0f + expf(-gate[i]))) * up[i];
}

/* src/qwen35/cpu.rs:415-427: normalized = rms_norm(h); gate/up matvecs;
   gate = silu(gate) * up; down matvec.  Unit norm weight == no weight. */
int orc_dense_ffn(size_t batch, size_t hidden, size_t ffn, uint32_t gate_type,
                  const uint8_t *gate, uint32_t up_type, const uint8_t *up,
                  uint32_t down_type, const uint8_t *down, const float *hidden_in,
                  float epsilon, float *output, int threads)
{
    uint64_t g_row, u_row, d_row;
    int status;
    if ((status = orc_row_byte_len(gate_type, hidden, &g_row))) return status;
    if ((status = orc_row_byte_len(up_type, hidden, &u_row))) return status;
    if ((status = orc_row_byte_len(down_type, ffn, &d_row))) return status;
    float *normalized = (float *)malloc(sizeof(float) * hidden);
    float *g = (float *)malloc(sizeof(float) * ffn);
    float *u = (float *)malloc(sizeof(float) * ffn);
    if (!normalized || !g || !u) { free(normalized); free(g); free(u); return ORC_OVERFLOW; }
    for (size_t b = 0; b < batch && status == ORC_OK; b++) {
        status = orc_rms_norm(hidden_in + b * hidden, hidden, NULL, 0, epsilon, normalized, hidden);
        if (status) break;
        status = orc_matvec(gate_type, ffn, hidden, gate, ffn * g_row, normalized, hidden, g, ffn, threads);
        if (status) break;
        status = orc_matvec(up_type, ffn, hidden, up, ffn * u_row, normalized, hidden, u, ffn, threads);
        if (status) break;
        for (size_t i = 0; i < ffn; i++) g[i] = orc_silu(g[i]) * u[i];
        status = orc_matvec(down_type, hidden, ffn, down, hidden * d_row, g, ffn,
                            output + b * hidden, hidden, threads);
    }
    free(normalized); free(g); free(u);
    return status;
}

/* Routed-expert layer (src/gemma4/cpu.rs:574-612 structure):
   logits = router(x) (bf16 rows), selected = top_k_softmax(logits, k);
   for each (expert, p) in selection order:
     gate_up = expert_matvec(gate_up[e], x)  (rows = 2*width, gate first)
     act = silu_mul(gate, up)                (GLM expert form, glm52/expert.rs:260-267)
     out_e = expert_matvec(down[e], act)
     routed = fma(out_e, p, routed)          (src/gemma4/cpu.rs:608-611)
   Expert e's bytes are the e-th contiguous slice (src/cpu.rs:473-509). */
int orc_moe_layer(size_t batch, size_t hidden, size_t width, size_t experts, size_t k,
                  const uint16_t *router, uint32_t gu_type, const uint8_t *gate_up_all,
                  uint32_t dn_type, const uint8_t *down_all, const float *tokens,
                  size_t *selected, float *weights, float *output, int threads)
{
    uint64_t gu_row, dn_row;
    int status;
    if ((status = orc_row_byte_len(gu_type, hidden, &gu_row))) return status;
    if ((status = orc_row_byte_len(dn_type, width, &dn_row))) return status;
    size_t gu_bytes = 2 * width * (size_t)gu_row;
    size_t dn_bytes = hidden * (size_t)dn_row;
    float *logits = (float *)malloc(sizeof(float) * experts);
    float *gu = (float *)malloc(sizeof(float) * 2 * width);
    float *act = (float *)malloc(sizeof(float) * width);
    float *eo = (float *)malloc(sizeof(float) * hidden);
    if (!logits || !gu || !act || !eo) { status = ORC_OVERFLOW; goto done; }
    for (size_t t = 0; t < batch; t++) {
        const float *x = tokens + t * hidden;
        float *routed = output + t * hidden;
        orc_matvec_bf16(experts, hidden, router, x, logits, 1);
        status = orc_top_k_softmax(logits, experts, k, selected + t * k, weights + t * k);
        if (status) goto done;
        for (size_t i = 0; i < hidden; i++) routed[i] = 0.0f;
        for (size_t j = 0; j < k; j++) {
            size_t e = selected[t * k + j];
            float p = weights[t * k + j];
            status = orc_matvec(gu_type, 2 * width, hidden, gate_up_all + e * gu_bytes, gu_bytes,
                                x, hidden, gu, 2 * width, threads);
            if (status) goto done;
            orc_silu_mul_glm(gu, gu + width, width, act);
            status = orc_matvec(dn_type, hidden, width, down_all + e * dn_bytes, dn_bytes, act,
                                width, eo, hidden, threads);
            if (status) goto done;
            for (size_t i = 0; i < hidden; i++) routed[i] = fmaf(eo[i], p, routed[i]);
        }
    }
done:
    free(logits); free(gu); free(act); free(eo);
    return status;
}

/* Prefill as the reference runs it: one matvec per token
   (src/gemma4/metal.rs:514-536 token loop; src/cpu.rs:345-399 per token),
   with bf16 activations widened exactly to f32. */
int orc_gemm_tokenwise(uint32_t t, size_t m, size_t n, size_t k, const uint16_t *a,
                       const uint8_t *encoded, float *output, int threads)
{
    uint64_t row_bytes;
    int status = orc_row_byte_len(t, k, &row_bytes);
    if (status) return status;
    float *x = (float *)malloc(sizeof(float) * k);
    if (!x) return ORC_OVERFLOW;
    for (size_t r = 0; r < m && status == ORC_OK; r++) {
        for (size_t c = 0; c < k; c++) x[c] = bits_to_f32((uint32_t)a[r * k + c] << 16);
        status = orc_matvec(t, n, k, encoded, n * (size_t)row_bytes, x, k, output + r * n, n, threads);
    }
    free(x);
    return status;
}

/* ---------------------------------------------------------------------- */
/* src/expert.rs:44-229  LRU slot bookkeeping                              */
/* ---------------------------------------------------------------------- */
typedef struct {
    int has_expert;
    size_t expert;
    uint64_t last_used;
    int pinned;
} orc_slot;

struct orc_lru {
    size_t layers, slots;
    size_t *expert_counts;
    uint64_t *clocks;
    orc_slot *slot;      /* layers * slots */
    uint64_t hits, misses, evictions, reads, bytes_read, resident_bytes;
    uint64_t gate_up_bytes, down_bytes;
};

int orc_lru_new(size_t layers, const size_t *expert_counts, size_t slots_per_layer,
                uint64_t gate_up_bytes, uint64_t down_bytes, orc_lru **out)
{
    if (slots_per_layer == 0) return ORC_NO_SLOTS;                 /* :94-96 */
    orc_lru *c = (orc_lru *)calloc(1, sizeof(orc_lru));
    if (!c) return ORC_OVERFLOW;
    c->layers = layers;
    c->slots = slots_per_layer;
    c->expert_counts = (size_t *)calloc(layers ? layers : 1, sizeof(size_t));
    c->clocks = (uint64_t *)calloc(layers ? layers : 1, sizeof(uint64_t));
    c->slot = (orc_slot *)calloc((layers ? layers : 1) * slots_per_layer, sizeof(orc_slot));
    if (!c->expert_counts || !c->clocks || !c->slot) { orc_lru_free(c); return ORC_OVERFLOW; }
    for (size_t l = 0; l < layers; l++) c->expert_counts[l] = expert_counts[l];
    c->gate_up_bytes = gate_up_bytes;
    c->down_bytes = down_bytes;
    c->resident_bytes = (uint64_t)layers * slots_per_layer * (gate_up_bytes + down_bytes);
    *out = c;
    return ORC_OK;
}

void orc_lru_free(orc_lru *c)
{
    if (!c) return;
    free(c->expert_counts); free(c->clocks); free(c->slot); free(c);
}

/* acquire, src/expert.rs:166-229 */
int orc_lru_acquire(orc_lru *c, size_t layer, size_t expert, size_t *slot, int *hit,
                    int *evicted, size_t *evicted_expert)
{
    if (layer >= c->layers) return ORC_INVALID_LAYER;
    if (expert >= c->expert_counts[layer]) return ORC_INVALID_EXPERT;
    orc_slot *s = c->slot + layer * c->slots;
    c->clocks[layer] += 1;
    *evicted = 0;
    for (size_t i = 0; i < c->slots; i++) {
        if (s[i].has_expert && s[i].expert == expert) {
            s[i].last_used = c->clocks[layer];
            c->hits += 1;
            *slot = i;
            *hit = 1;
            return ORC_OK;
        }
    }
    c->misses += 1;
    /* min over unpinned slots of (is_some, last_used, index) */
    size_t best = SIZE_MAX;
    for (size_t i = 0; i < c->slots; i++) {
        if (s[i].pinned) continue;
        if (best == SIZE_MAX) { best = i; continue; }
        int a = s[i].has_expert, b = s[best].has_expert;
        if (a < b || (a == b && s[i].last_used < s[best].last_used)) best = i;
    }
    if (best == SIZE_MAX) return ORC_ALL_SLOTS_PINNED;
    if (s[best].has_expert) {
        c->evictions += 1;
        *evicted = 1;
        *evicted_expert = s[best].expert;
    }
    c->reads += 2;
    c->bytes_read += c->gate_up_bytes + c->down_bytes;
    s[best].has_expert = 1;
    s[best].expert = expert;
    s[best].last_used = c->clocks[layer];
    *slot = best;
    *hit = 0;
    return ORC_OK;
}

void orc_lru_set_pinned(orc_lru *c, size_t layer, size_t slot, int pinned)
{
    c->slot[layer * c->slots + slot].pinned = pinned;
}

void orc_lru_stats(const orc_lru *c, uint64_t *hits, uint64_t *misses, uint64_t *evictions,
                   uint64_t *reads, uint64_t *bytes_read, uint64_t *resident_bytes)
{
    *hits = c->hits; *misses = c->misses; *evictions = c->evictions;
    *reads = c->reads; *bytes_read = c->bytes_read; *resident_bytes = c->resident_bytes;
}

/* src/gemma4/cpu.rs:900-946  attend, with the ring addressing of
   metal/kernels.metal:486-578 (slot = position % capacity). */
int orc_attention(const float *query, const float *keys, const float *values, size_t capacity,
                  size_t width, size_t query_heads, size_t kv_heads, size_t head_dimension,
                  size_t start, size_t visible, float *output)
{
    if (visible == 0) return ORC_EMPTY_INPUT;
    size_t group_size = query_heads / kv_heads;
    float *scores = (float *)malloc(visible * sizeof(float));
    if (!scores) return ORC_OVERFLOW;
    for (size_t i = 0; i < query_heads * head_dimension; i++) output[i] = 0.0f;
    for (size_t query_head = 0; query_head < query_heads; query_head++) {
        size_t kv_head = query_head / group_size;
        const float *q = query + query_head * head_dimension;
        for (size_t s = 0; s < visible; s++) {
            size_t slot = (start + s) % capacity;
            const float *k = keys + slot * width + kv_head * head_dimension;
            float sum = 0.0f;
            /* query.mul_add(key, sum), d ascending */
            for (size_t d = 0; d < head_dimension; d++) sum = fmaf(q[d], k[d], sum);
            scores[s] = sum;
        }
        int status = orc_softmax_in_place(scores, visible);
        if (status != ORC_OK) {
            free(scores);
            return status;
        }
        float *o = output + query_head * head_dimension;
        for (size_t s = 0; s < visible; s++) {
            size_t slot = (start + s) % capacity;
            const float *v = values + slot * width + kv_head * head_dimension;
            /* value.mul_add(probability, output), positions ascending */
            for (size_t d = 0; d < head_dimension; d++) o[d] = fmaf(v[d], scores[s], o[d]);
        }
    }
    free(scores);
    return ORC_OK;
}

/* src/glm52/cpu.rs:1397-1410  decode_f8_e4m3fn */
int orc_st_decode_f8_e4m3fn(uint8_t bits, float *value)
{
    float sign = (bits & 0x80) == 0 ? 1.0f : -1.0f;
    unsigned exponent = (bits >> 3) & 0x0f;
    unsigned fraction = bits & 0x07;
    if (exponent == 0x0f && fraction == 0x07) return ORC_NON_FINITE;
    float magnitude = exponent == 0 ? (float)fraction * ldexpf(1.0f, -9)
                                    : (1.0f + (float)fraction / 8.0f) * ldexpf(1.0f, (int)exponent - 7);
    *value = sign * magnitude;
    return ORC_OK;
}

/* src/metal.rs:1893-1942  u8_matrix_encoding */
int orc_st_u8_encoding(size_t rows, size_t columns, size_t encoded_len, size_t scale_len, int *format,
                       size_t *group_size, size_t *scale_columns, size_t *expected, size_t *actual,
                       int *scales_bad)
{
    size_t int8_bytes, row_scale_bytes, int4_bytes;
    *scales_bad = 0;
    if (__builtin_mul_overflow(rows, columns, &int8_bytes)) return ORC_OVERFLOW;
    if (__builtin_mul_overflow(rows, (size_t)4, &row_scale_bytes)) return ORC_OVERFLOW;
    if (encoded_len == int8_bytes && scale_len == row_scale_bytes) {
        *format = ORC_ST_INT8_ROW;
        *group_size = 0;
        *scale_columns = 1;
        return ORC_OK;
    }
    if (__builtin_mul_overflow(rows, (columns + 1) / 2, &int4_bytes)) return ORC_OVERFLOW;
    if (encoded_len != int4_bytes) {
        *expected = int4_bytes;
        *actual = encoded_len;
        return ORC_INVALID_BYTE_LENGTH;
    }
    if (scale_len == row_scale_bytes) {
        *format = ORC_ST_INT4_GROUPED;
        *group_size = columns > 0 ? columns : 1;
        *scale_columns = 1;
        return ORC_OK;
    }
    static const size_t sizes[8] = {16, 32, 48, 64, 96, 128, 192, 256};
    for (int i = 0; i < 8; i++) {
        if (sizes[i] > columns) break;
        size_t sc = (columns + sizes[i] - 1) / sizes[i], want;
        if (__builtin_mul_overflow(rows, sc, &want) || __builtin_mul_overflow(want, (size_t)4, &want))
            return ORC_OVERFLOW;
        if (scale_len == want) {
            *format = ORC_ST_INT4_GROUPED;
            *group_size = sizes[i];
            *scale_columns = sc;
            return ORC_OK;
        }
    }
    *scales_bad = 1;
    *expected = row_scale_bytes;
    *actual = scale_len;
    return ORC_INVALID_BYTE_LENGTH;
}

/* read_dense_values (BF16), read_fp8_row, read_quantized_row:
   src/glm52/cpu.rs:1224-1270, :1278-1337, :1339-1394 */
int orc_st_dequantize_row(int format, size_t rows, size_t columns, const uint8_t *encoded, const float *scales,
                          size_t group_size, size_t row, float *output)
{
    (void)rows;
    switch (format) {
    case ORC_ST_BF16: {
        const uint8_t *p = encoded + row * columns * 2;
        for (size_t c = 0; c < columns; c++) {
            uint32_t bits = (uint32_t)(p[2 * c] | (p[2 * c + 1] << 8)) << 16;
            memcpy(&output[c], &bits, 4);
        }
        return ORC_OK;
    }
    case ORC_ST_F8_E4M3: {
        const uint8_t *p = encoded + row * columns;
        size_t scale_columns = (columns + 127) / 128;
        const float *s = scales + (row / 128) * scale_columns;
        for (size_t c = 0; c < columns; c++) {
            float d;
            if (orc_st_decode_f8_e4m3fn(p[c], &d) != ORC_OK) return ORC_NON_FINITE;
            output[c] = d * s[c / 128];
        }
        return ORC_OK;
    }
    case ORC_ST_INT8_ROW: {
        const uint8_t *p = encoded + row * columns;
        for (size_t c = 0; c < columns; c++) output[c] = (float)(int8_t)p[c] * scales[row];
        return ORC_OK;
    }
    case ORC_ST_INT4_GROUPED: {
        size_t row_bytes = (columns + 1) / 2;
        size_t scale_columns = (columns + group_size - 1) / group_size;
        const uint8_t *p = encoded + row * row_bytes;
        const float *s = scales + row * scale_columns;
        for (size_t c = 0; c < columns; c++) {
            uint8_t byte = p[c / 2];
            uint8_t nibble = (c % 2 == 0) ? (byte & 0x0f) : (byte >> 4);
            output[c] = ((float)nibble - 8.0f) * s[c / group_size];
        }
        return ORC_OK;
    }
    default:
        return ORC_UNSUPPORTED_TYPE;
    }
}

/* src/glm52/cpu.rs:1180-1190  row, then sum of products */
int orc_st_matvec(int format, size_t rows, size_t columns, const uint8_t *encoded, const float *scales,
                  size_t group_size, const float *input, float *output)
{
    float *row = (float *)malloc((columns ? columns : 1) * sizeof(float));
    if (!row) return ORC_OVERFLOW;
    for (size_t r = 0; r < rows; r++) {
        int status = orc_st_dequantize_row(format, rows, columns, encoded, scales, group_size, r, row);
        if (status != ORC_OK) {
            free(row);
            return status;
        }
        float sum = 0.0f;
        for (size_t c = 0; c < columns; c++) {
            float product = row[c] * input[c];
            sum = sum + product;
        }
        output[r] = sum;
    }
    free(row);
    return ORC_OK;
}
