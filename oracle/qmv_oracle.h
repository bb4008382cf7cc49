/*
 * ORACLE — test infrastructure only.
 *
 * A plain-C restatement of the reference engine's CPU packed-weight path
 * (trungnguyen21/my-inference-engine, src/quantization.cpp scalar branches and
 * src/quantized_matvec.cpp), against which the MI355X kernels are tested.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only to check or to time a CPU baseline; the product library
 * (libqmv_hip.so) never links or calls it.
 *
 * Pinning (what fixes each function independently of this file):
 *   oracle_f16_to_f32         all 65,536 codes vs the ldexp closed form of
 *                             tests/q8_0_reference_test.cpp:48-64
 *   *_dequantize_block        reference known-answer blocks
 *                             (tests/q{8_0,5_0,4_k,6_k}_reference_test.cpp), a
 *                             float64 decoder of the documented equations
 *                             (exactness: every decode is exact in fp32 except
 *                             Q4_K's one subtraction), and the reference
 *                             itself built from source into oracle/_ref
 *   *_dot_f32, matvec/matmul  reference KATs (-6, -25, 363, 84.5; -3/5, -8,
 *                             -0.25, -16), 128-trial LCG dot-vs-dequant, the
 *                             invalid-argument table, and bit-for-bit equality
 *                             with the reference's scalar build in oracle/_ref
 *   oracle_greedy_argmax      tie/NaN cases of src/sampler.cpp:29-51 and numpy
 *                             argmax
 *   oracle_add_f32            reference KAT (tests/tensor_reference_test.cpp:
 *                             50-58), numpy's fp32 add, the reference build
 *   oracle_rms_norm_f32       reference KAT (tests/tensor_reference_test.cpp:
 *                             84-93), a float64 closed form (including inputs
 *                             small enough that epsilon dominates), the
 *                             invalid-argument table (:154-156), bit-for-bit
 *                             equality with the reference's scalar build
 *   oracle_swiglu_f32         reference KAT (tests/transformer_ops_reference_
 *                             test.cpp:95-108), a float64 closed form, bit-for-
 *                             bit equality with the reference's scalar build
 */
#ifndef QMV_ORACLE_H
#define QMV_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_TYPE_Q5_0 6u
#define ORACLE_TYPE_Q8_0 8u
#define ORACLE_TYPE_Q4_K 12u
#define ORACLE_TYPE_Q6_K 14u

/* Same layout as the reference's GgufQuantizedTensorView (src/gguf_reader.h:31-40). */
typedef struct OracleView {
    const unsigned char *data;
    uint32_t ggml_type;
    uint32_t dimension_count;
    uint64_t dimensions[4];
    uint64_t element_count;
    uint64_t block_elements;
    uint64_t block_bytes;
    uint64_t block_count;
} OracleView;

float oracle_f16_to_f32(uint16_t bits);

int oracle_q4_k_unpack_scale_min(const unsigned char *scale_and_min, int subblock,
                                 uint8_t *scale, uint8_t *minimum);
int oracle_q6_k_unpack_value(const unsigned char *block, int index,
                             int8_t *quantized, int8_t *scale);

/* Block decoders: block points at the packed bytes (any alignment). */
int oracle_q8_0_dequantize_block(const unsigned char *block, float *output);
int oracle_q5_0_dequantize_block(const unsigned char *block, float *output);
int oracle_q4_k_dequantize_block(const unsigned char *block, float *output);
int oracle_q6_k_dequantize_block(const unsigned char *block, float *output);

/* Scalar block dots (the reference's non-SIMD branches). */
int oracle_q8_0_dot_f32(const unsigned char *block, const float *input, float *result);
int oracle_q5_0_dot_f32(const unsigned char *block, const float *input, float *result);
int oracle_q4_k_dot_f32(const unsigned char *block, const float *input, float *result);
int oracle_q6_k_dot_f32(const unsigned char *block, const float *input, float *result);

/* Whole-tensor scalar path with the reference's validation. */
int oracle_matvec_f32(const OracleView *matrix, const float *input, int input_count,
                      float *output, int output_count);
int oracle_matmul_f32(const OracleView *matrix, const float *inputs, int input_count,
                      int batch_count, float *outputs, int output_count);

/* Rows [first_row, first_row+row_count) of the scalar matvec (no validation
 * beyond a consistent shape); output has row_count values. */
int oracle_matvec_rows_f32(const OracleView *matrix, const float *input,
                           int first_row, int row_count, float *output);

/* Decode rows into output[row_count, K]. */
int oracle_dequantize_rows(const OracleView *matrix, int first_row, int row_count,
                           float *output);

/* Float64 brute force for rows of one input vector: dot[r] = sum w*x and
 * absdot[r] = sum |w*x| with w from the block decoders. */
int oracle_row_stats_f64(const OracleView *matrix, const float *input,
                         int first_row, int row_count, double *dot, double *absdot);

/* sampler_greedy_sample: lowest id on ties, 0 and -1 on any non-finite logit. */
int oracle_greedy_argmax(const float *logits, int vocab_size, int *token_id);

/* Decode-step element operations between the projections. */
/* tensor_add_f32 (src/tensor.cpp:5-23): output[i] = left[i] + right[i]. */
int oracle_add_f32(const float *left, const float *right, int length, float *output);
/* tensor_rms_norm_f32 (src/tensor.cpp:99-136). */
int oracle_rms_norm_f32(const float *input, const float *weight, int length, float epsilon,
                        float *output);
/* transformer_swiglu_f32 (src/transformer_ops.cpp:163-176), out of place:
 * output[i] = up[i] * silu(gate[i]); output may equal gate. */
int oracle_swiglu_f32(const float *gate, const float *up, int length, float *output);

#ifdef __cplusplus
}
#endif

#endif
