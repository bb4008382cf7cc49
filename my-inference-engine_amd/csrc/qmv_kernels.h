/*
 * Launch interface between the host shim and the gfx950 kernels.
 */
#ifndef QMV_KERNELS_H
#define QMV_KERNELS_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmv_layout.h"

#define QMV_MAX_WAVES 8
#define QMV_MAX_JOBS 8
/* Positions per launch: the VALU kernels take up to 8, the matrix-core
 * kernels (Q4_K, Q6_K) up to 32 in blocks of 16. */
#define QMV_VALU_MAX_POSITIONS 8
#define QMV_MFMA_MAX_POSITIONS 32
/* Tiles (one per wave) per prefill workgroup. */
#define QMV_PF_TILES 4
/* Floats of split-K workspace past the last partial: the VALU kernels' last
 * split loads a batch of partials from one base pointer and may read up to
 * this far beyond its tile's (discarding what it reads there). */
#define QMV_PARTIAL_PAD 1024
/* Words between the arrival counters of consecutive tiles: one counter per
 * 128-byte line, so the atomics of different tiles do not queue on a line. */
#ifndef QMV_COUNTER_STRIDE
#define QMV_COUNTER_STRIDE 32
#endif

namespace qmv {

/* One tensor of a (possibly grouped) matvec launch. */
struct MatvecJob {
    const uint8_t *w;    /* tiled device layout */
    float *y;            /* output, y[m * ldy + row] */
    int rows;            /* N */
    int ldy;
    int tiles;           /* ceil(N / 64) */
    int splits;          /* workgroups along K per tile */
    int units_per_split; /* K-units per workgroup */
    int wg_begin;        /* first workgroup id of this job in the grid */
    int partial_offset;  /* float offset of this job's partials in the workspace */
    int counter_offset;  /* offset of this job's per-tile arrival counters */
    const float *add;    /* optional: y[m * ldy + row] += add[m * ldadd + row] */
    int ldadd;           /* 0: one vector for every position (a bias) */
};

struct MatvecParams {
    MatvecJob job[QMV_MAX_JOBS];
    int njobs;
    const float *x; /* x[m * ldx + k], shared by all jobs */
    int ldx;
    int cols;           /* K */
    int units;          /* K-units per row */
    int units_per_wave; /* contiguous K-units per wave */
    float *partials;
    unsigned *counters; /* all zero between launches; tile t at t * QMV_COUNTER_STRIDE */
    int matrix_cores; /* run this launch (Q4_K, Q6_K or Q5_0, 2 <= M <= 8) on the matrix cores */
    /* Matrix-core kernel (M <= 8): work items per unit (1 or 2; 0 = 1). A
     * tile then has units x parts items of consecutive sub-blocks, and
     * units_per_wave (1) / units_per_split count items. */
    int parts;
    int positions;    /* positions in this launch (the prefill kernel's position rows past it are padding) */
    /* Fused greedy argmax (single tensor, M = 1; result non-null): tile and
     * group candidates (argmax_words(tiles) words), group and top arrival
     * counts (argmax_counts(tiles), zero between launches) and the result. */
    uint64_t *argmax_cand;
    unsigned *argmax_count;
    int *argmax_result;
    int argmax_tiles;
    /* Fused SwiGLU (swiglu != 0; jobs 0 = gate and 1 = up, equal rows):
     * job 0's y receives up * silu(gate) and neither projection is stored.
     * Each tile's final values are published to pair_vals[2][tiles][M][64]
     * and counted in pair_count[tiles * QMV_COUNTER_STRIDE] (zero between
     * launches). */
    int swiglu;
    float *pair_vals;
    unsigned *pair_count;
    /* Paired SwiGLU (M = 1, pair_waves > 0; swiglu then 0): a workgroup runs
     * the same tile and K-range of job 0 (gate) in waves [0, pair_waves) and
     * of job 1 (up) in waves [pair_waves, 2 pair_waves), and its finisher
     * writes up * silu(gate) to job 0's y. A split publishes both sums
     * (partials [tiles][splits][2][64] at job 0's offsets), so no second
     * count per tile pair is needed. */
    int pair_waves;
    /* Prefill launches (set by launch_prefill): the splits publish their
     * partials and stop, and a second kernel (pf_reduce_kernel) sums them and
     * runs the epilogue; no arrival counts are taken. */
    int pf_deferred;
};

/* One tensor of a row-major single-position launch: `w` holds the GGUF bytes
 * of a Q4_K tensor (row r at r * sb * 144) or the planes of a Q6_K tensor
 * (row r at r * q6k_row_stride(sb), launch_rowmajor_q6k), workgroups
 * [wg_begin, next job's wg_begin) take consecutive rows. */
struct RowdotJob {
    const uint8_t *w;
    float *y;
    const float *add; /* optional: y[row] += add[row] */
    int rows;
    int wg_begin;
};

struct RowdotParams {
    RowdotJob job[QMV_MAX_JOBS];
    int njobs;
    const float *x; /* K activations, shared by all jobs */
    int sb;         /* super-blocks per row */
    /* Fused greedy argmax (QMV_ROWDOT_ARGMAX): candidate tiles as
     * MatvecParams describes, one per workgroup. */
    uint64_t *argmax_cand;
    unsigned *argmax_count;
    int *argmax_result;
    int argmax_tiles;
    /* Fused RMSNorm of the input (launch_rowgroup with norm set; rows of at
     * most 16 super-blocks): the jobs read (x / sqrt(mean(x^2) + norm_eps)) *
     * norm_w, the element rule of tensor_rms_norm_f32 (src/tensor.cpp:99-136),
     * with mean(x^2) over the K = 256 sb inputs. */
    const float *norm_w;
    float norm_eps;
    /* Q6_K (launch_rowloop_q6k): the launch's rows (its jobs' rows in job
     * order); each job's wg_begin is its first row there. */
    int groups;
};

/* Row-major epilogues. */
#define QMV_ROWDOT_STORE 0
#define QMV_ROWDOT_SWIGLU 1
#define QMV_ROWDOT_ARGMAX 2

/* Workspace of a fused argmax over `tiles` tiles (groups of 64 tiles). */
inline size_t argmax_words(size_t tiles) { return tiles + (tiles + 63) / 64; }
inline size_t argmax_counts(size_t tiles) { return (tiles + 63) / 64 + 1; }

hipError_t launch_matvec(int fmt, const MatvecParams &p, int m, int grid, int waves, hipStream_t s);
/* Row-major Q4_K launch at one position, one 64-weight group per lane.
 * Rows of at most 16 super-blocks: workgroups of QMV_ROWGROUP_WAVES waves
 * sharing the activations in LDS, each wave taking `rows` (1, 2 or 4) rows
 * per segment of `seg` lanes (16, 32 or 64), so rows * 64 / seg rows per
 * wave. Longer rows (seg = 64): a row spans the workgroup's `waves` waves,
 * `rows` rows per workgroup. norm: the fused RMSNorm of RowdotParams (rows
 * of at most 16 super-blocks; store and SwiGLU epilogues). */
#define QMV_ROWGROUP_WAVES 4
hipError_t launch_rowgroup(const RowdotParams &p, int rows, int seg, int epi, int grid, int waves, hipStream_t s,
                           bool norm = false);
/* Row-major Q6_K: bytes per row of the chunked plane layout
 * launch_rowmajor_q6k writes (210 per super-block, the row padded to 16
 * bytes). */
__host__ __device__ inline size_t q6k_row_stride(int sb) { return ((size_t)210 * sb + 15) & ~(size_t)15; }
/* Row-major Q6_K launch at one position over rows of 17 to 128
 * super-blocks: `grid` workgroups of `waves` (1 to 16) waves, one row per
 * wave, over the launch's p.groups rows (grid = ceil(p.groups / waves)).
 * epi: QMV_ROWDOT_STORE (plus the optional addends), QMV_ROWDOT_SWIGLU (jobs
 * 0 and 1 of equal rows; p.groups = their rows) or QMV_ROWDOT_ARGMAX (one
 * job, one candidate per workgroup: p.argmax_tiles = grid). */
hipError_t launch_rowloop_q6k(const RowdotParams &p, int epi, int grid, int waves, hipStream_t s);
/* The Q6_K plane layout of `rows` GGUF rows of sb super-blocks (raw, 210
 * bytes each) into out (rows * q6k_row_stride(sb) bytes; padding untouched). */
hipError_t launch_rowmajor_q6k(const uint8_t *raw, uint8_t *out, int rows, int sb, hipStream_t s);
hipError_t launch_dequant(int fmt, const uint8_t *w, float *out, int rows, int cols, int units,
                          int first_row, int row_count, hipStream_t s);
/* status (may be null): cleared to 0 if any id is outside [0, rows). */
hipError_t launch_gather(int fmt, const uint8_t *w, const int *ids, int count, float *out, int rows, int cols,
                         int units, int *status, hipStream_t s);
hipError_t launch_repack(int fmt, const uint8_t *raw, uint8_t *out, int rows, int blocks_per_row,
                         int units, int blocks_per_unit, int block_bytes, int unit_bytes, int tiles,
                         hipStream_t s);
/* Prefill launch (up to `rows` = 16 or 32 positions): grid = sum over jobs
 * of ceil(tiles / 4) tile groups x splits; for launches whose split-K finish
 * would take QMV_PF_DEFER_ROUNDS or more rounds of partial loads, followed by
 * the reduction kernel. */
hipError_t launch_prefill(int fmt, const MatvecParams &p, int rows, int grid, hipStream_t s);
/* Plain fp32 copy (n elements) as a kernel, e.g. from mapped host memory. */
hipError_t launch_copy(const float *src, float *dst, size_t n, hipStream_t s);
/* dst[0..n) = v (a fill kernel, no memset node). */
hipError_t launch_fill_u32(unsigned *dst, size_t n, unsigned v, hipStream_t s);
hipError_t launch_rms_norm(const float *x, const float *w, int n, int batch, float eps, float *out,
                           hipStream_t s);
hipError_t launch_argmax(const float *logits, int n, float *bval, int *bidx, int *bbad, int nblocks,
                         int *result, hipStream_t s);

} // namespace qmv

#endif
