/*
 * ORACLE — test infrastructure only. Compiled together with the reference's
 * own src/quantization.cpp and src/quantized_matvec.cpp (straight from the
 * reference checkout, never copied) into oracle/_ref/libref_*.so, so that the
 * reference's real CPU path can be called from Python through plain C
 * symbols. Everything else in those libraries is built with hidden
 * visibility; only the ref_* forwards below are exported.
 */
#include "quantization.h"
#include "quantized_matvec.h"
#include "tensor.h"
#include "transformer_ops.h"

#include <string.h>

#define REF_EXPORT extern "C" __attribute__((visibility("default")))

REF_EXPORT int ref_f16_bits_to_f32(uint16_t bits, float *out)
{
    return f16_bits_to_f32(bits, out);
}

/* Blocks arrive as raw bytes; copy into the aligned structs the reference
 * functions take, the way src/quantized_matvec.cpp:30,43,56,69 does. */
#define REF_BLOCK_FNS(tag, Type)                                                 \
    REF_EXPORT int ref_##tag##_dequantize_block(const unsigned char *raw, float *out) \
    {                                                                            \
        Type block;                                                              \
        memcpy(&block, raw, sizeof block);                                       \
        return tag##_dequantize_block(&block, out);                              \
    }                                                                            \
    REF_EXPORT int ref_##tag##_dot_f32(const unsigned char *raw, const float *x, float *r) \
    {                                                                            \
        Type block;                                                              \
        memcpy(&block, raw, sizeof block);                                       \
        return tag##_dot_f32(&block, x, r);                                      \
    }

REF_BLOCK_FNS(q8_0, Q8_0Block)
REF_BLOCK_FNS(q5_0, Q5_0Block)
REF_BLOCK_FNS(q4_k, Q4_KBlock)
REF_BLOCK_FNS(q6_k, Q6_KBlock)

REF_EXPORT int ref_q4_k_unpack_scale_min(const uint8_t *p, int s, uint8_t *sc, uint8_t *m)
{
    return q4_k_unpack_scale_min(p, s, sc, m);
}

REF_EXPORT int ref_q6_k_unpack_value(const unsigned char *raw, int index, int8_t *q, int8_t *sc)
{
    Q6_KBlock block;
    memcpy(&block, raw, sizeof block);
    return q6_k_unpack_value(&block, index, q, sc);
}

REF_EXPORT int ref_quantized_tensor_matvec_f32(const GgufQuantizedTensorView *m, const float *x,
                                               int xn, float *y, int yn)
{
    return quantized_tensor_matvec_f32(m, x, xn, y, yn);
}

REF_EXPORT int ref_quantized_tensor_matmul_f32(const GgufQuantizedTensorView *m, const float *x,
                                               int xn, int batch, float *y, int yn)
{
    return quantized_tensor_matmul_f32(m, x, xn, batch, y, yn);
}

/* Decode-step element operations (src/tensor.cpp, src/transformer_ops.cpp). */
REF_EXPORT int ref_tensor_add_f32(const float *a, const float *b, int n, float *out)
{
    return tensor_add_f32(a, b, n, out);
}

REF_EXPORT int ref_tensor_rms_norm_f32(const float *x, const float *w, int n, float eps, float *out)
{
    return tensor_rms_norm_f32(x, w, n, eps, out);
}

/* In place on gate, as the reference defines it. */
REF_EXPORT int ref_transformer_swiglu_f32(float *gate, const float *up, int n)
{
    return transformer_swiglu_f32(gate, up, n);
}
