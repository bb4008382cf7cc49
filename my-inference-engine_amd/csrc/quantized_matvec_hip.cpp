/*
 * The reference's packed-matvec entry points with their original C++
 * signatures (src/quantized_matvec.h:32-50), implemented on the MI355X C ABI.
 * Linked into libqmv_hip.so so that an engine built against the unchanged
 * quantized_matvec.h can drop src/quantized_matvec.cpp and link this library
 * instead; qwen2_weight_matvec / qwen2_weight_matmul
 * (src/qwen2_architecture.cpp:605,612,686) call it unchanged.
 */
#include "quantized_matvec.h"

#include "qmv_hip.h"

#define QMV_CXX_EXPORT __attribute__((visibility("default")))

static QmvTensorView qmv_view_of(const GgufQuantizedTensorView *v)
{
    QmvTensorView q;
    q.data = v->data;
    q.ggml_type = v->ggml_type;
    q.dimension_count = v->dimension_count;
    for (int i = 0; i < 4; ++i) q.dimensions[i] = v->dimensions[i];
    q.element_count = v->element_count;
    q.block_elements = v->block_elements;
    q.block_bytes = v->block_bytes;
    q.block_count = v->block_count;
    return q;
}

QMV_CXX_EXPORT int quantized_tensor_matvec_f32(const GgufQuantizedTensorView *matrix, const float *input,
                                               int input_count, float *output, int output_count)
{
    if (matrix == nullptr) return 0;
    const QmvTensorView q = qmv_view_of(matrix);
    return qmv_tensor_matvec_f32(&q, input, input_count, output, output_count);
}

QMV_CXX_EXPORT int quantized_tensor_matmul_f32(const GgufQuantizedTensorView *matrix, const float *inputs,
                                               int input_count, int batch_count, float *outputs,
                                               int output_count)
{
    if (matrix == nullptr) return 0;
    const QmvTensorView q = qmv_view_of(matrix);
    return qmv_tensor_matmul_f32(&q, inputs, input_count, batch_count, outputs, output_count);
}
