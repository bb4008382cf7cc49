/*
 * Seeded synthetic packed tensors and activations for the benchmark and the
 * parity tests (libqmv_synth.so, host C++, OpenMP).
 *
 * Counter-based: block j of a tensor draws from its own SplitMix64 stream
 * keyed by (seed, j), so the bytes are identical for any thread count and on
 * any host. Normals use Box-Muller in double precision; fp16 scales are the
 * round-to-nearest-even fp16 of |N(0, sigma)|.
 *
 * Distributions (one line per format):
 *   Q8_0  d = f16|N(0,0.02)|, 32 int8 codes uniform in [-127, 127]
 *   Q5_0  d = f16|N(0,0.02)|, qh 4 and qs 16 uniform bytes
 *   Q4_K  d, dmin = f16|N(0,0.01)|, 12 uniform scale bytes (a bijection with
 *         16 uniform 6-bit scales/mins), 128 uniform nibble bytes
 *   Q6_K  ql 128 and qh 64 uniform bytes, 16 int8 scales uniform in
 *         [-64, 63], d = f16|N(0,0.001)|
 *   x     fp32 N(0,1)
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include "qmv_formats.h"

namespace {

inline uint64_t splitmix64(uint64_t &state)
{
    uint64_t z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t stream, uint64_t index)
{
    uint64_t s = seed ^ (stream * 0xD1B54A32D192ED03ull);
    uint64_t k = splitmix64(s);
    s = k ^ (index * 0xA24BAED4963EE407ull);
    return splitmix64(s);
}

inline double uniform01_open(uint64_t &state) /* (0, 1] */
{
    return ((splitmix64(state) >> 11) + 1) * (1.0 / 9007199254740992.0);
}

inline double normal(uint64_t &state)
{
    const double u1 = uniform01_open(state);
    const double u2 = uniform01_open(state);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

/* Round a non-negative finite double to binary16, nearest-even. */
uint16_t f64_to_f16_rne(double v)
{
    uint16_t sign = 0;
    if (v < 0) { sign = 0x8000; v = -v; }
    if (v == 0) return sign;
    if (v >= 65520.0) return (uint16_t)(sign | 0x7c00); /* rounds to +inf */
    int e;
    frexp(v, &e);                     /* v = f * 2^e, f in [0.5, 1) */
    int q = e - 11;                   /* quantum exponent for an 11-bit significand */
    if (q < -24) q = -24;             /* subnormal quantum 2^-24 */
    const double scaled = ldexp(v, -q); /* exact */
    double r = nearbyint(scaled);     /* default rounding mode: nearest-even */
    uint32_t m = (uint32_t)r;
    if (m >= 2048) { m >>= 1; q += 1; } /* rounding carried into a new binade */
    if (q == -24 && m < 1024) return (uint16_t)(sign | m); /* subnormal */
    const uint32_t exp5 = (uint32_t)(q + 10 + 15);
    if (exp5 >= 31) return (uint16_t)(sign | 0x7c00);
    return (uint16_t)(sign | (exp5 << 10) | (m & 1023u));
}

inline void put_u16(unsigned char *p, uint16_t v)
{
    p[0] = (unsigned char)(v & 0xff);
    p[1] = (unsigned char)(v >> 8);
}

void fill_bytes(uint64_t &state, unsigned char *dst, int n)
{
    for (int i = 0; i < n; i += 8) {
        uint64_t r = splitmix64(state);
        for (int k = 0; k < 8 && i + k < n; ++k) dst[i + k] = (unsigned char)(r >> (8 * k));
    }
}

void gen_block(uint32_t type, uint64_t &st, unsigned char *b)
{
    switch (type) {
    case QMV_GGML_TYPE_Q8_0: {
        put_u16(b, f64_to_f16_rne(fabs(0.02 * normal(st))));
        for (int i = 0; i < 32; ++i) b[2 + i] = (unsigned char)(int8_t)((int)(splitmix64(st) % 255u) - 127);
        break;
    }
    case QMV_GGML_TYPE_Q5_0: {
        put_u16(b, f64_to_f16_rne(fabs(0.02 * normal(st))));
        fill_bytes(st, b + 2, 20);
        break;
    }
    case QMV_GGML_TYPE_Q4_K: {
        put_u16(b, f64_to_f16_rne(fabs(0.01 * normal(st))));
        put_u16(b + 2, f64_to_f16_rne(fabs(0.01 * normal(st))));
        fill_bytes(st, b + 4, 140);
        break;
    }
    case QMV_GGML_TYPE_Q6_K: {
        fill_bytes(st, b, 192);
        for (int i = 0; i < 16; ++i) b[192 + i] = (unsigned char)(int8_t)((int)(splitmix64(st) & 127u) - 64);
        put_u16(b + 208, f64_to_f16_rne(fabs(0.001 * normal(st))));
        break;
    }
    default:
        break;
    }
}

int format_geometry(uint32_t type, int *elements, int *bytes)
{
    switch (type) {
    case QMV_GGML_TYPE_Q8_0: *elements = 32; *bytes = 34; return 1;
    case QMV_GGML_TYPE_Q5_0: *elements = 32; *bytes = 22; return 1;
    case QMV_GGML_TYPE_Q4_K: *elements = 256; *bytes = 144; return 1;
    case QMV_GGML_TYPE_Q6_K: *elements = 256; *bytes = 210; return 1;
    default: return 0;
    }
}

} // namespace

extern "C" {

/* Bytes of a packed rows x cols tensor, or 0 if the shape is invalid. */
uint64_t qmv_synth_tensor_bytes(uint32_t type, int rows, int cols)
{
    int be, bb;
    if (!format_geometry(type, &be, &bb) || rows <= 0 || cols <= 0 || cols % be) return 0;
    return (uint64_t)rows * (uint64_t)(cols / be) * (uint64_t)bb;
}

/* Fill out[] (qmv_synth_tensor_bytes bytes) with a row-major GGUF tensor. */
int qmv_synth_tensor(uint32_t type, int rows, int cols, uint64_t seed,
                     unsigned char *out, uint64_t out_bytes)
{
    int be, bb;
    const uint64_t need = qmv_synth_tensor_bytes(type, rows, cols);
    if (!out || need == 0 || out_bytes < need || !format_geometry(type, &be, &bb)) return 0;
    const int64_t blocks = (int64_t)(need / (uint64_t)bb);
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < blocks; ++j) {
        uint64_t st = stream_key(seed, type, (uint64_t)j);
        gen_block(type, st, out + (uint64_t)j * (uint64_t)bb);
    }
    return 1;
}

/* out[i] = float(sigma * N(0,1)) for i < n, chunked counter streams. */
int qmv_synth_normal_f32(float *out, uint64_t n, uint64_t seed, double sigma)
{
    if (!out) return 0;
    const int64_t chunks = (int64_t)((n + 255) / 256);
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < chunks; ++c) {
        uint64_t st = stream_key(seed, 0xF32u, (uint64_t)c);
        const uint64_t end = (uint64_t)(c + 1) * 256 < n ? (uint64_t)(c + 1) * 256 : n;
        for (uint64_t i = (uint64_t)c * 256; i < end; ++i) out[i] = (float)(sigma * normal(st));
    }
    return 1;
}

/* Round-to-nearest-even binary16 of v, exported for tests. */
uint16_t qmv_synth_f64_to_f16(double v)
{
    return f64_to_f16_rne(v);
}

/* 64-bit content hash (FNV-1a over 64-bit words, then a SplitMix finish). */
uint64_t qmv_synth_hash(const void *data, uint64_t n)
{
    const unsigned char *p = (const unsigned char *)data;
    uint64_t h = 0xcbf29ce484222325ull;
    uint64_t i = 0;
    for (; i + 8 <= n; i += 8) {
        uint64_t w;
        memcpy(&w, p + i, 8);
        h = (h ^ w) * 0x100000001b3ull;
    }
    for (; i < n; ++i) h = (h ^ p[i]) * 0x100000001b3ull;
    uint64_t s = h;
    return splitmix64(s);
}

} // extern "C"
