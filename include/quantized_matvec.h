/*
 * Drop-in replacement for the reference's src/quantized_matvec.h:32-50.
 * Same names, argument meaning, C++ linkage and 1/0 return convention; the
 * implementation (quantized_matvec_hip.cpp in libqmv_hip.so) forwards to the
 * C ABI in qmv_hip.h, which runs the product on an MI355X.
 *
 * matrix->dimensions[0] is the column count K (== input_count) and
 * dimensions[1] the row count N (== output_count); both must fit in int.
 * Only Q5_0, Q8_0, Q4_K and Q6_K views are accepted, K must be a multiple of
 * the block size, and element_count/block_count/block layout must agree with
 * the shape. Returns 1 after writing every output, 0 otherwise (output
 * contents are then unspecified).
 *
 * Unlike the reference, which reads the packed bytes on every call, the
 * library keeps a device copy of each tensor it has seen, keyed by data
 * pointer, type and shape and checked against a content fingerprint (every
 * byte up to 64 KiB, sampled words beyond). The bytes must therefore stay
 * unchanged while cached: after editing them in place, or before freeing or
 * unmapping them (gguf_close), call qmv_release_tensor(data) from qmv_hip.h.
 */
#ifndef QUANTIZED_MATVEC_H
#define QUANTIZED_MATVEC_H

#include "gguf_quantized_view.h"

int quantized_tensor_matvec_f32(
    const GgufQuantizedTensorView *matrix,
    const float *input,
    int input_count,
    float *output,
    int output_count
);

/* inputs is token-major [batch_count, input_count]; outputs is
 * [batch_count, output_count]. */
int quantized_tensor_matmul_f32(
    const GgufQuantizedTensorView *matrix,
    const float *inputs,
    int input_count,
    int batch_count,
    float *outputs,
    int output_count
);

#endif
