/*
 * ORACLE — test infrastructure only (see qmv_oracle.h for who may use it and
 * what pins each function). Restates the reference's CPU algorithm:
 *   f16 decode              src/quantization.cpp:22-49 (portable x86 branch)
 *   Q8_0 decode / dot       src/quantization.cpp:54-67 / :151-156
 *   Q5_0 decode / dot       src/quantization.cpp:161-184 / :331-346
 *   Q4_K unpack/decode/dot  src/quantization.cpp:351-378 / :380-409 / :536-554
 *   Q6_K unpack/decode/dot  src/quantization.cpp:559-586 / :588-615 / :734-752
 *   row loop + validation   src/quantized_matvec.cpp:10-84, :86-162
 *   batched loop            src/quantized_matvec.cpp:164-224
 *   greedy argmax           src/sampler.cpp:29-51
 * Built with -ffp-contract=off so every product and sum rounds exactly where
 * the reference's scalar C++ does; the row loop may run under OpenMP because
 * each row's accumulation order is independent of the thread count.
 */
#include "qmv_oracle.h"

#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

static uint16_t load_u16(const unsigned char *p)
{
    return (uint16_t)(p[0] | (p[1] << 8));
}

float oracle_f16_to_f32(uint16_t bits)
{
    const uint32_t sign = (uint32_t)(bits >> 15) << 31;
    const uint32_t exp5 = (bits >> 10) & 31u;
    uint32_t mant = bits & 1023u;
    uint32_t out;
    if (exp5 == 31u) {
        /* Inf keeps a zero fraction; NaN payloads are widened and quieted. */
        out = sign | 0x7f800000u | (mant << 13) | (mant ? 0x00400000u : 0u);
    } else if (exp5 != 0u) {
        out = sign | ((exp5 - 15u + 127u) << 23) | (mant << 13);
    } else if (mant == 0u) {
        out = sign;
    } else {
        /* Subnormal: value = mant * 2^-24; renormalise to a 1.f mantissa. */
        int e = -14;
        while (!(mant & 0x400u)) {
            mant <<= 1;
            e -= 1;
        }
        out = sign | ((uint32_t)(e + 127) << 23) | ((mant & 1023u) << 13);
    }
    float f;
    memcpy(&f, &out, sizeof f);
    return f;
}

/* ---- unpack helpers ---------------------------------------------------- */

int oracle_q4_k_unpack_scale_min(const unsigned char *p, int s, uint8_t *scale, uint8_t *minimum)
{
    if (!p || !scale || !minimum || s < 0 || s > 7) return 0;
    if (s < 4) {
        *scale = (uint8_t)(p[s] & 63u);
        *minimum = (uint8_t)(p[s + 4] & 63u);
    } else {
        /* Low four bits live in bytes 8..11, the top two in the high bits of
         * bytes 0..3 (scales) and 4..7 (minimums). */
        *scale = (uint8_t)((p[s + 4] & 15u) | ((p[s - 4] >> 6) << 4));
        *minimum = (uint8_t)((p[s + 4] >> 4) | ((p[s] >> 6) << 4));
    }
    return 1;
}

int oracle_q6_k_unpack_value(const unsigned char *block, int n, int8_t *quantized, int8_t *scale)
{
    if (!block || !quantized || !scale || n < 0 || n > 255) return 0;
    const unsigned char *ql = block;
    const unsigned char *qh = block + 128;
    const int8_t *sc = (const int8_t *)(block + 192);
    const int g = n >> 7, l = n & 127, r = l >> 5, o = l & 31;
    const int low = (ql[64 * g + 32 * (r & 1) + o] >> (4 * (r >> 1))) & 15;
    const int high = (qh[32 * g + o] >> (2 * r)) & 3;
    *quantized = (int8_t)((low | (high << 4)) - 32);
    *scale = sc[8 * g + 2 * r + o / 16];
    return 1;
}

/* ---- block decoders ---------------------------------------------------- */

int oracle_q8_0_dequantize_block(const unsigned char *block, float *output)
{
    if (!block || !output) return 0;
    const float d = oracle_f16_to_f32(load_u16(block));
    const int8_t *qs = (const int8_t *)(block + 2);
    for (int i = 0; i < 32; ++i) output[i] = d * qs[i];
    return 1;
}

static int q5_0_value(const unsigned char *block, int i)
{
    const unsigned char *qh = block + 2;
    const unsigned char *qs = block + 6;
    const int nib = i < 16 ? (qs[i] & 15) : (qs[i - 16] >> 4);
    const int bit = (qh[i >> 3] >> (i & 7)) & 1;
    return (int)(int8_t)((nib | (bit << 4)) - 16);
}

int oracle_q5_0_dequantize_block(const unsigned char *block, float *output)
{
    if (!block || !output) return 0;
    const float d = oracle_f16_to_f32(load_u16(block));
    for (int i = 0; i < 32; ++i) output[i] = d * (int8_t)q5_0_value(block, i);
    return 1;
}

int oracle_q4_k_dequantize_block(const unsigned char *block, float *output)
{
    if (!block || !output) return 0;
    const float d = oracle_f16_to_f32(load_u16(block));
    const float dmin = oracle_f16_to_f32(load_u16(block + 2));
    const unsigned char *packed = block + 16;
    for (int s = 0; s < 8; ++s) {
        uint8_t sc, m;
        oracle_q4_k_unpack_scale_min(block + 4, s, &sc, &m);
        const float a = d * sc;
        const float b = dmin * m;
        const unsigned char *q = packed + 32 * (s >> 1);
        const int shift = 4 * (s & 1);
        for (int j = 0; j < 32; ++j) {
            const uint8_t v = (uint8_t)((q[j] >> shift) & 15);
            output[32 * s + j] = a * v - b;
        }
    }
    return 1;
}

int oracle_q6_k_dequantize_block(const unsigned char *block, float *output)
{
    if (!block || !output) return 0;
    const float d = oracle_f16_to_f32(load_u16(block + 208));
    for (int n = 0; n < 256; ++n) {
        int8_t q, sc;
        oracle_q6_k_unpack_value(block, n, &q, &sc);
        output[n] = d * sc * (int)q;
    }
    return 1;
}

/* ---- scalar block dots -------------------------------------------------- */

int oracle_q8_0_dot_f32(const unsigned char *block, const float *input, float *result)
{
    if (!block || !input || !result) return 0;
    const float d = oracle_f16_to_f32(load_u16(block));
    const int8_t *qs = (const int8_t *)(block + 2);
    float acc = 0.0f;
    for (int i = 0; i < 32; ++i) acc += d * qs[i] * input[i];
    *result = acc;
    return 1;
}

int oracle_q5_0_dot_f32(const unsigned char *block, const float *input, float *result)
{
    if (!block || !input || !result) return 0;
    const float d = oracle_f16_to_f32(load_u16(block));
    float acc = 0.0f;
    for (int i = 0; i < 32; ++i) {
        const int8_t v = (int8_t)q5_0_value(block, i);
        acc += d * v * input[i];
    }
    *result = acc;
    return 1;
}

int oracle_q4_k_dot_f32(const unsigned char *block, const float *input, float *result)
{
    if (!block || !input || !result) return 0;
    const float d = oracle_f16_to_f32(load_u16(block));
    const float dmin = oracle_f16_to_f32(load_u16(block + 2));
    const unsigned char *packed = block + 16;
    float acc = 0.0f;
    for (int s = 0; s < 8; ++s) {
        uint8_t sc, m;
        oracle_q4_k_unpack_scale_min(block + 4, s, &sc, &m);
        const float a = d * sc;
        const float b = dmin * m;
        const unsigned char *q = packed + 32 * (s >> 1);
        const float *x = input + 32 * s;
        const int shift = 4 * (s & 1);
        for (int j = 0; j < 32; ++j) {
            const float w = a * ((q[j] >> shift) & 15) - b;
            acc += w * x[j];
        }
    }
    *result = acc;
    return 1;
}

int oracle_q6_k_dot_f32(const unsigned char *block, const float *input, float *result)
{
    if (!block || !input || !result) return 0;
    const float d = oracle_f16_to_f32(load_u16(block + 208));
    const unsigned char *ql = block;
    const unsigned char *qh = block + 128;
    const int8_t *scales = (const int8_t *)(block + 192);
    float acc = 0.0f;
    /* Natural index order: group g (128), region r (32), offset o. */
    for (int g = 0; g < 2; ++g) {
        for (int r = 0; r < 4; ++r) {
            for (int o = 0; o < 32; ++o) {
                const int low = (ql[64 * g + 32 * (r & 1) + o] >> (4 * (r >> 1))) & 15;
                const int high = (qh[32 * g + o] >> (2 * r)) & 3;
                const int q = (low | (high << 4)) - 32;
                const int8_t sc = scales[8 * g + 2 * r + o / 16];
                acc += (d * sc * q) * input[128 * g + 32 * r + o];
            }
        }
    }
    *result = acc;
    return 1;
}

/* ---- whole-tensor path --------------------------------------------------- */

typedef int (*oracle_dot_fn)(const unsigned char *, const float *, float *);

static int format_of(uint32_t type, uint64_t *elements, uint64_t *bytes, oracle_dot_fn *dot)
{
    switch (type) {
    case ORACLE_TYPE_Q5_0: *elements = 32; *bytes = 22; *dot = oracle_q5_0_dot_f32; return 1;
    case ORACLE_TYPE_Q8_0: *elements = 32; *bytes = 34; *dot = oracle_q8_0_dot_f32; return 1;
    case ORACLE_TYPE_Q4_K: *elements = 256; *bytes = 144; *dot = oracle_q4_k_dot_f32; return 1;
    case ORACLE_TYPE_Q6_K: *elements = 256; *bytes = 210; *dot = oracle_q6_k_dot_f32; return 1;
    default: return 0;
    }
}

/* Layout checks shared by matvec and matmul (src/quantized_matvec.cpp:99-149). */
static int view_is_valid(const OracleView *m, uint64_t *blocks_per_row, oracle_dot_fn *dot)
{
    if (m->dimension_count != 2) return 0;
    const uint64_t cols = m->dimensions[0], rows = m->dimensions[1];
    if (cols == 0 || rows == 0 || cols > INT_MAX || rows > INT_MAX) return 0;
    uint64_t be, bb;
    if (!format_of(m->ggml_type, &be, &bb, dot)) return 0;
    if (m->block_elements != be || m->block_bytes != bb || cols % be != 0) return 0;
    const uint64_t bpr = cols / be;
    if (bpr > UINT64_MAX / rows || m->block_count != bpr * rows ||
        cols > UINT64_MAX / rows || m->element_count != cols * rows ||
        m->block_count > SIZE_MAX / bb)
        return 0;
    *blocks_per_row = bpr;
    return 1;
}

static int row_dot(const OracleView *m, oracle_dot_fn dot, uint64_t bpr,
                   const float *x, uint64_t row, float *out)
{
    float sum = 0.0f;
    for (uint64_t b = 0; b < bpr; ++b) {
        const unsigned char *blk = m->data + (row * bpr + b) * m->block_bytes;
        float part = 0.0f;
        if (!dot(blk, x + b * m->block_elements, &part)) return 0;
        sum += part;
    }
    *out = sum;
    return 1;
}

int oracle_matvec_f32(const OracleView *m, const float *input, int input_count,
                      float *output, int output_count)
{
    if (!m || !m->data || !input || !output || input_count <= 0 || output_count <= 0) return 0;
    uint64_t bpr;
    oracle_dot_fn dot;
    if (!view_is_valid(m, &bpr, &dot)) return 0;
    if ((uint64_t)input_count != m->dimensions[0] || (uint64_t)output_count != m->dimensions[1])
        return 0;
    int failed = 0;
#pragma omp parallel for schedule(static) reduction(| : failed)
    for (int r = 0; r < output_count; ++r)
        if (!row_dot(m, dot, bpr, input, (uint64_t)r, &output[r])) failed = 1;
    return !failed;
}

int oracle_matmul_f32(const OracleView *m, const float *inputs, int input_count,
                      int batch_count, float *outputs, int output_count)
{
    if (!m || !m->data || !inputs || !outputs || input_count <= 0 || output_count <= 0 ||
        batch_count <= 0)
        return 0;
    uint64_t bpr;
    oracle_dot_fn dot;
    if (!view_is_valid(m, &bpr, &dot)) return 0;
    if ((uint64_t)input_count != m->dimensions[0] || (uint64_t)output_count != m->dimensions[1])
        return 0;
    if ((size_t)batch_count > SIZE_MAX / (size_t)input_count ||
        (size_t)batch_count > SIZE_MAX / (size_t)output_count)
        return 0;
    int failed = 0;
#pragma omp parallel for schedule(static) reduction(| : failed)
    for (int r = 0; r < output_count; ++r) {
        for (int t = 0; t < batch_count; ++t) outputs[(size_t)t * output_count + r] = 0.0f;
        for (uint64_t b = 0; b < bpr && !failed; ++b) {
            const unsigned char *blk = m->data + ((uint64_t)r * bpr + b) * m->block_bytes;
            for (int t = 0; t < batch_count; ++t) {
                float part = 0.0f;
                const float *x = inputs + (size_t)t * input_count + b * m->block_elements;
                if (!dot(blk, x, &part)) { failed = 1; break; }
                outputs[(size_t)t * output_count + r] += part;
            }
        }
    }
    return !failed;
}

static int shape_ok(const OracleView *m, int first_row, int row_count, uint64_t *bpr,
                    oracle_dot_fn *dot)
{
    if (!m || !m->data || !view_is_valid(m, bpr, dot)) return 0;
    return first_row >= 0 && row_count >= 0 &&
           (uint64_t)first_row + (uint64_t)row_count <= m->dimensions[1];
}

int oracle_matvec_rows_f32(const OracleView *m, const float *input, int first_row,
                           int row_count, float *output)
{
    uint64_t bpr;
    oracle_dot_fn dot;
    if (!input || !output || !shape_ok(m, first_row, row_count, &bpr, &dot)) return 0;
    int failed = 0;
#pragma omp parallel for schedule(static) reduction(| : failed)
    for (int r = 0; r < row_count; ++r)
        if (!row_dot(m, dot, bpr, input, (uint64_t)(first_row + r), &output[r])) failed = 1;
    return !failed;
}

typedef int (*oracle_decode_fn)(const unsigned char *, float *);

static oracle_decode_fn decoder_of(uint32_t type)
{
    switch (type) {
    case ORACLE_TYPE_Q5_0: return oracle_q5_0_dequantize_block;
    case ORACLE_TYPE_Q8_0: return oracle_q8_0_dequantize_block;
    case ORACLE_TYPE_Q4_K: return oracle_q4_k_dequantize_block;
    case ORACLE_TYPE_Q6_K: return oracle_q6_k_dequantize_block;
    default: return 0;
    }
}

int oracle_dequantize_rows(const OracleView *m, int first_row, int row_count, float *output)
{
    uint64_t bpr;
    oracle_dot_fn dot;
    if (!output || !shape_ok(m, first_row, row_count, &bpr, &dot)) return 0;
    const oracle_decode_fn decode = decoder_of(m->ggml_type);
    const uint64_t cols = m->dimensions[0];
#pragma omp parallel for schedule(static)
    for (int r = 0; r < row_count; ++r) {
        const uint64_t row = (uint64_t)(first_row + r);
        for (uint64_t b = 0; b < bpr; ++b)
            decode(m->data + (row * bpr + b) * m->block_bytes,
                   output + (size_t)r * cols + b * m->block_elements);
    }
    return 1;
}

int oracle_row_stats_f64(const OracleView *m, const float *input, int first_row,
                         int row_count, double *dot_out, double *absdot_out)
{
    uint64_t bpr;
    oracle_dot_fn dot;
    if (!input || !dot_out || !absdot_out || !shape_ok(m, first_row, row_count, &bpr, &dot))
        return 0;
    const oracle_decode_fn decode = decoder_of(m->ggml_type);
    const uint64_t be = m->block_elements;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < row_count; ++r) {
        float w[256];
        double s = 0.0, a = 0.0;
        const uint64_t row = (uint64_t)(first_row + r);
        for (uint64_t b = 0; b < bpr; ++b) {
            decode(m->data + (row * bpr + b) * m->block_bytes, w);
            for (uint64_t i = 0; i < be; ++i) {
                const double p = (double)w[i] * (double)input[b * be + i];
                s += p;
                a += fabs(p);
            }
        }
        dot_out[r] = s;
        absdot_out[r] = a;
    }
    return 1;
}

int oracle_greedy_argmax(const float *logits, int vocab_size, int *token_id)
{
    if (token_id) *token_id = -1;
    if (!logits || vocab_size <= 0 || !token_id) return 0;
    int best = 0;
    for (int i = 0; i < vocab_size; ++i) {
        if (!isfinite(logits[i])) return 0;
        if (logits[i] > logits[best]) best = i; /* strict: first maximum wins */
    }
    *token_id = best;
    return 1;
}

/* ---- Decode-step element operations ----------------------------------- */

int oracle_add_f32(const float *left, const float *right, int length, float *output)
{
    /* src/tensor.cpp:11-17: null pointers and non-positive lengths fail. */
    if (!left || !right || !output || length <= 0) return 0;
    for (int i = 0; i < length; ++i) output[i] = left[i] + right[i];
    return 1;
}

int oracle_rms_norm_f32(const float *input, const float *weight, int length, float epsilon,
                        float *output)
{
    /* src/tensor.cpp:116-122: epsilon <= 0 fails (a NaN epsilon does not). */
    if (!input || !weight || !output || length <= 0 || epsilon <= 0) return 0;
    /* :124-127: sum of squares in index order, in fp32. */
    float sum_sq = 0.0f;
    for (int i = 0; i < length; ++i) {
        const float sq = input[i] * input[i];
        sum_sq += sq;
    }
    /* :129: sqrt(mean + epsilon); :131-133: (x / denom) * weight. */
    const float denom = sqrtf(sum_sq / (float)length + epsilon);
    for (int i = 0; i < length; ++i) output[i] = (input[i] / denom) * weight[i];
    return 1;
}

int oracle_swiglu_f32(const float *gate, const float *up, int length, float *output)
{
    /* src/transformer_ops.cpp:169-172: null pointers and length <= 0 fail. */
    if (!gate || !up || !output || length <= 0) return 0;
    for (int i = 0; i < length; ++i) {
        /* :163-165 silu(x) = x / (1 + exp(-x)); :175 up * silu(gate). */
        const float g = gate[i];
        const float silu = g / (1.0f + expf(-g));
        output[i] = up[i] * silu;
    }
    return 1;
}
