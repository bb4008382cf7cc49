/*
 * The drop-in boundary exercised from C++, the way the reference engine
 * calls it: quantized_tensor_matvec_f32 / quantized_tensor_matmul_f32 with
 * their original signatures and C++ linkage (src/quantized_matvec.h:32-50),
 * linked from libqmv_hip.so. Checked against the CPU oracle (liboracle.so,
 * test infrastructure only).
 *
 *   dropin_test --args   argument table only (no GPU needed)
 *   dropin_test          argument table, then the GPU cases
 *
 * Exit status 0 when every check holds; a failed check prints its case.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "quantized_matvec.h"

extern "C" {
/* oracle/qmv_oracle.h (the view type there has this same layout) */
int oracle_matvec_f32(const GgufQuantizedTensorView *matrix, const float *input, int input_count, float *output,
                      int output_count);
int oracle_row_stats_f64(const GgufQuantizedTensorView *matrix, const float *input, int first_row, int row_count,
                         double *dot, double *absdot);
/* include/qmv_hip.h */
int qmv_device_count(void);
}

static int g_failures = 0;

#define CHECK(cond, ...)                                                                                          \
    do {                                                                                                          \
        if (!(cond)) {                                                                                            \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__);                                                  \
            fprintf(stderr, __VA_ARGS__);                                                                         \
            fprintf(stderr, "\n");                                                                                \
            ++g_failures;                                                                                         \
        }                                                                                                         \
    } while (0)

struct Format {
    uint32_t type;
    int block_elements, block_bytes;
};
static const Format kQ5_0 = {ENGINE_GGML_TYPE_Q5_0, 32, 22};
static const Format kQ8_0 = {ENGINE_GGML_TYPE_Q8_0, 32, 34};
static const Format kQ4_K = {ENGINE_GGML_TYPE_Q4_K, 256, 144};
static const Format kQ6_K = {ENGINE_GGML_TYPE_Q6_K, 256, 210};

static GgufQuantizedTensorView make_view(const unsigned char *data, const Format &f, int rows, int cols)
{
    GgufQuantizedTensorView v;
    memset(&v, 0, sizeof v);
    v.data = data;
    v.ggml_type = f.type;
    v.dimension_count = 2;
    v.dimensions[0] = (uint64_t)cols;
    v.dimensions[1] = (uint64_t)rows;
    v.element_count = (uint64_t)rows * cols;
    v.block_elements = (uint64_t)f.block_elements;
    v.block_bytes = (uint64_t)f.block_bytes;
    v.block_count = v.element_count / (uint64_t)f.block_elements;
    return v;
}

/* SplitMix64: seeded bytes and N(0,1)-ish activations (sum of uniforms). */
struct Rng {
    uint64_t s;
    uint64_t next()
    {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    float normal()
    {
        double a = 0.0;
        for (int i = 0; i < 12; ++i) a += (double)(next() >> 11) * (1.0 / 9007199254740992.0);
        return (float)(a - 6.0);
    }
};

/* Random packed blocks whose f16 scales are small normal numbers (exponent
 * field 8..13, so no NaN/Inf), other bytes uniform. */
static std::vector<unsigned char> random_tensor(const Format &f, int rows, int cols, uint64_t seed)
{
    const size_t blocks = (size_t)rows * cols / f.block_elements;
    std::vector<unsigned char> b(blocks * f.block_bytes);
    Rng r{seed};
    for (auto &c : b) c = (unsigned char)r.next();
    for (size_t i = 0; i < blocks; ++i) {
        unsigned char *blk = &b[i * f.block_bytes];
        auto set_f16 = [&](int off) {
            const uint16_t h = (uint16_t)(((8 + r.next() % 6) << 10) | (r.next() & 0x3ff));
            memcpy(blk + off, &h, 2);
        };
        if (f.type == ENGINE_GGML_TYPE_Q6_K) {
            set_f16(208);
        } else if (f.type == ENGINE_GGML_TYPE_Q4_K) {
            set_f16(0);
            set_f16(2);
        } else {
            set_f16(0);
        }
    }
    return b;
}

static void check_args()
{
    /* src/quantized_matvec.cpp:93-149,168-191: every invalid call returns 0. */
    std::vector<unsigned char> raw(34, 0);
    float x[64] = {0}, y[4] = {7.0f, 7.0f, 7.0f, 7.0f};
    GgufQuantizedTensorView v = make_view(raw.data(), kQ8_0, 1, 32);
    CHECK(quantized_tensor_matvec_f32(nullptr, x, 32, y, 1) == 0, "null view");
    CHECK(quantized_tensor_matvec_f32(&v, nullptr, 32, y, 1) == 0, "null input");
    CHECK(quantized_tensor_matvec_f32(&v, x, 32, nullptr, 1) == 0, "null output");
    CHECK(quantized_tensor_matvec_f32(&v, x, 31, y, 1) == 0, "input_count != K");
    CHECK(quantized_tensor_matvec_f32(&v, x, 32, y, 2) == 0, "output_count != N");
    CHECK(quantized_tensor_matmul_f32(&v, x, 32, 0, y, 1) == 0, "batch_count 0");
    CHECK(quantized_tensor_matmul_f32(&v, x, 32, -1, y, 1) == 0, "batch_count -1");
    GgufQuantizedTensorView w = v;
    w.ggml_type = 99;
    CHECK(quantized_tensor_matvec_f32(&w, x, 32, y, 1) == 0, "unknown type");
    w = v;
    w.block_bytes = 35;
    CHECK(quantized_tensor_matvec_f32(&w, x, 32, y, 1) == 0, "block_bytes");
    w = v;
    w.block_count = 2;
    CHECK(quantized_tensor_matvec_f32(&w, x, 32, y, 1) == 0, "block_count");
    w = v;
    w.element_count = 31;
    CHECK(quantized_tensor_matvec_f32(&w, x, 32, y, 1) == 0, "element_count");
    /* Q4_K 4864 x 896: K is not a multiple of 256 (src/quantized_matvec.cpp:136-138). */
    std::vector<float> xb(896, 0.0f), yb(4864, -99.0f);
    GgufQuantizedTensorView q = make_view(raw.data(), kQ4_K, 4864, 896);
    q.block_count = 0;
    CHECK(quantized_tensor_matvec_f32(&q, xb.data(), 896, yb.data(), 4864) == 0, "Q4_K 4864x896");
    CHECK(yb[0] == -99.0f && yb[4863] == -99.0f, "rejected call wrote its output");
}

static void check_against_oracle(const Format &f, int rows, int cols, int batch, uint64_t seed)
{
    std::vector<unsigned char> w = random_tensor(f, rows, cols, seed);
    GgufQuantizedTensorView v = make_view(w.data(), f, rows, cols);
    std::vector<float> x((size_t)batch * cols);
    Rng r{seed ^ 0x5151};
    for (auto &e : x) e = r.normal();
    std::vector<float> y((size_t)batch * rows, NAN), y1(rows), yo(rows);
    std::vector<double> dot(rows), absdot(rows);
    const int ok = batch == 1 ? quantized_tensor_matvec_f32(&v, x.data(), cols, y.data(), rows)
                              : quantized_tensor_matmul_f32(&v, x.data(), cols, batch, y.data(), rows);
    CHECK(ok == 1, "type %u %dx%d M=%d: call failed", f.type, rows, cols, batch);
    if (ok != 1) return;
    for (int b = 0; b < batch; ++b) {
        const float *xb = &x[(size_t)b * cols];
        CHECK(oracle_matvec_f32(&v, xb, cols, yo.data(), rows) == 1, "oracle");
        CHECK(oracle_row_stats_f64(&v, xb, 0, rows, dot.data(), absdot.data()) == 1, "oracle stats");
        int bad = 0;
        for (int i = 0; i < rows; ++i) {
            const double err = fabs((double)y[(size_t)b * rows + i] - (double)yo[i]);
            if (!(err <= 1e-5 * absdot[i])) ++bad;
        }
        CHECK(bad == 0, "type %u %dx%d M=%d position %d: %d rows over 1e-5 * sum|w x|", f.type, rows, cols, batch,
              b, bad);
        if (batch > 1 && b == batch - 1) {
            /* The last position through the single-vector entry point. */
            CHECK(quantized_tensor_matvec_f32(&v, xb, cols, y1.data(), rows) == 1, "matvec of one position");
            int far = 0;
            for (int i = 0; i < rows; ++i)
                if (!(fabs((double)y1[i] - (double)yo[i]) <= 1e-5 * absdot[i])) ++far;
            CHECK(far == 0, "matvec of one position over tolerance");
        }
    }
}

int main(int argc, char **argv)
{
    const bool args_only = argc > 1 && strcmp(argv[1], "--args") == 0;
    check_args();
    if (!args_only) {
        if (qmv_device_count() <= 0) {
            fprintf(stderr, "FAIL: no HIP device visible\n");
            return 2;
        }
        check_against_oracle(kQ8_0, 896, 896, 1, 1);
        check_against_oracle(kQ5_0, 256, 1536, 8, 2);
        check_against_oracle(kQ4_K, 4864, 1024, 1, 3);
        check_against_oracle(kQ6_K, 896, 4864, 1, 4);
        check_against_oracle(kQ4_K, 1000, 1536, 8, 5);
        check_against_oracle(kQ6_K, 130, 2048, 20, 6);
        check_against_oracle(kQ4_K, 520, 3584, 40, 7);
    }
    printf("dropin_test: %s (%d failure%s)\n", g_failures ? "FAILED" : "ok", g_failures, g_failures == 1 ? "" : "s");
    return g_failures ? 1 : 0;
}
