/*
 * Device (HBM) layout of a packed tensor, shared by the kernels and the host
 * shim.
 *
 * Rows are grouped into tiles of 64 (one row per lane of a wavefront). Along
 * K a row is cut into units: one 256-weight super-block for Q4_K/Q6_K, four
 * consecutive 32-weight blocks (128 weights) for Q8_0/Q5_0. The bytes of one
 * (tile, unit) pair form a contiguous slab of 64 * unit_bytes bytes, split
 * into planes; plane p holds `width` bytes for each of the 64 lanes, lane l at
 * plane_offset + l * width. So the i-th 16-byte load of every lane of a wave
 * reads 1 KiB of consecutive bytes, and no byte is duplicated:
 *
 *   Q4_K  unit 144 B: plane 0 = bytes 0..15 (d, dmin, 12 scale bytes),
 *                     planes 1..8 = qs bytes 16(p-1)..16p-1      (9 x 16 B)
 *   Q6_K  unit 210 B: planes 0..7 = ql, 8..11 = qh, 12 = int8 scales (16 B
 *                     each), plane 13 = d (2 B)
 *   Q8_0  unit 136 B: planes 0..7 = qs of block p/2, half p%2 (16 B each),
 *                     plane 8 = the four d's (8 B)
 *   Q5_0  unit  88 B: planes 0..3 = qs of block p (16 B), plane 4 = the four
 *                     32-bit qh words (16 B), plane 5 = the four d's (8 B)
 *
 * Slab (t, u) starts at (t * units + u) * 64 * unit_bytes. Rows past N in the
 * last tile and blocks past K in a partial last unit are zero bytes (scale 0).
 * The total is the packed size exactly when N % 64 == 0 and K is a multiple
 * of the unit width.
 */
#ifndef QMV_LAYOUT_H
#define QMV_LAYOUT_H

#include <stdint.h>

#include "qmv_formats.h"

#define QMV_TILE_ROWS 64

enum QmvFormat { QMV_FMT_Q8_0 = 0, QMV_FMT_Q5_0 = 1, QMV_FMT_Q4_K = 2, QMV_FMT_Q6_K = 3 };

typedef struct QmvGeometry {
    int format;          /* QmvFormat */
    int block_elements;  /* 32 or 256 */
    int block_bytes;     /* 34, 22, 144, 210 */
    int blocks_per_unit; /* 4 or 1 */
    int unit_elements;   /* 128 or 256 */
    int unit_bytes;      /* per lane: 136, 88, 144, 210 */
} QmvGeometry;

static inline int qmv_geometry_of(uint32_t ggml_type, QmvGeometry *g)
{
    switch (ggml_type) {
    case QMV_GGML_TYPE_Q8_0:
        g->format = QMV_FMT_Q8_0; g->block_elements = 32; g->block_bytes = 34;
        g->blocks_per_unit = 4; g->unit_elements = 128; g->unit_bytes = 136;
        return 1;
    case QMV_GGML_TYPE_Q5_0:
        g->format = QMV_FMT_Q5_0; g->block_elements = 32; g->block_bytes = 22;
        g->blocks_per_unit = 4; g->unit_elements = 128; g->unit_bytes = 88;
        return 1;
    case QMV_GGML_TYPE_Q4_K:
        g->format = QMV_FMT_Q4_K; g->block_elements = 256; g->block_bytes = 144;
        g->blocks_per_unit = 1; g->unit_elements = 256; g->unit_bytes = 144;
        return 1;
    case QMV_GGML_TYPE_Q6_K:
        g->format = QMV_FMT_Q6_K; g->block_elements = 256; g->block_bytes = 210;
        g->blocks_per_unit = 1; g->unit_elements = 256; g->unit_bytes = 210;
        return 1;
    default:
        return 0;
    }
}

#endif
