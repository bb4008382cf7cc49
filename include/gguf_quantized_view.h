/*
 * Minimal restatement of the reference's packed tensor view and GGML type
 * codes (src/gguf_reader.h:7-11,31-40), for building the drop-in
 * quantized_matvec.h outside the engine. Inside the engine the reference's own
 * gguf_reader.h provides the same definitions under the same include guard,
 * so only one of the two is ever seen by a translation unit.
 */
#ifndef GGUF_READER_H
#define GGUF_READER_H

#include <stddef.h>
#include <stdint.h>

#define ENGINE_GGML_TYPE_F32 0u
#define ENGINE_GGML_TYPE_Q5_0 6u
#define ENGINE_GGML_TYPE_Q8_0 8u
#define ENGINE_GGML_TYPE_Q4_K 12u
#define ENGINE_GGML_TYPE_Q6_K 14u

/* Borrowed read-only packed tensor: dimensions[0] = columns, [1] = rows. */
typedef struct GgufQuantizedTensorView {
    const unsigned char *data;
    uint32_t ggml_type;
    uint32_t dimension_count;
    uint64_t dimensions[4];
    uint64_t element_count;
    uint64_t block_elements;
    uint64_t block_bytes;
    uint64_t block_count;
} GgufQuantizedTensorView;

#endif
