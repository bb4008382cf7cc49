/*
 * GGUF packed block formats handled by the MI355X matrix-vector path.
 *
 * The byte layouts are fixed by the GGUF/ggml file format, so they must match
 * the reference engine's structs field for field:
 *   Q8_0  include/quantization.h:6-7,33-39    (34 bytes, 32 weights)
 *   Q5_0  include/quantization.h:9-10,93-100  (22 bytes, 32 weights)
 *   Q4_K  include/quantization.h:12-16,152-160 (144 bytes, 256 weights)
 *   Q6_K  include/quantization.h:18-23,236-244 (210 bytes, 256 weights)
 * Type codes follow src/gguf_reader.h:7-11.
 *
 * Decode equations (w = decoded fp32 weight, d/dmin = fp16 factors):
 *   Q8_0  w[i] = d * qs[i]                       (qs signed int8)
 *   Q5_0  w[i] = d * ((nib_i | bit_i << 4) - 16)  nib_i: low nibble of qs[i]
 *         for i < 16, high nibble of qs[i-16] otherwise; bit_i = bit i%8 of
 *         qh[i/8]
 *   Q4_K  w = (d * sc_s) * q - (dmin * m_s)      q: nibble, s = sub-block 0..7;
 *         qs[32g + j] holds weight 64g + j (low) and 64g + 32 + j (high)
 *   Q6_K  w = (d * scales[16-group]) * (q - 32), q = low4 | high2 << 4
 */
#ifndef QMV_FORMATS_H
#define QMV_FORMATS_H

#include <stdint.h>

#define QMV_GGML_TYPE_F32 0u
#define QMV_GGML_TYPE_Q5_0 6u
#define QMV_GGML_TYPE_Q8_0 8u
#define QMV_GGML_TYPE_Q4_K 12u
#define QMV_GGML_TYPE_Q6_K 14u

#define QMV_Q8_0_BLOCK_ELEMENTS 32
#define QMV_Q8_0_BLOCK_BYTES 34
#define QMV_Q5_0_BLOCK_ELEMENTS 32
#define QMV_Q5_0_BLOCK_BYTES 22
#define QMV_Q4_K_BLOCK_ELEMENTS 256
#define QMV_Q4_K_BLOCK_BYTES 144
#define QMV_Q6_K_BLOCK_ELEMENTS 256
#define QMV_Q6_K_BLOCK_BYTES 210

/* Byte offsets of the fields inside one packed block. */
#define QMV_Q8_0_OFF_D 0
#define QMV_Q8_0_OFF_QS 2
#define QMV_Q5_0_OFF_D 0
#define QMV_Q5_0_OFF_QH 2
#define QMV_Q5_0_OFF_QS 6
#define QMV_Q4_K_OFF_D 0
#define QMV_Q4_K_OFF_DMIN 2
#define QMV_Q4_K_OFF_SCALES 4
#define QMV_Q4_K_OFF_QS 16
#define QMV_Q6_K_OFF_QL 0
#define QMV_Q6_K_OFF_QH 128
#define QMV_Q6_K_OFF_SCALES 192
#define QMV_Q6_K_OFF_D 208

#endif
