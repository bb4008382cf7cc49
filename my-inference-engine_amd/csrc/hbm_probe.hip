/*
 * HBM probes for measurement, not part of the matvec path (libqmv_probe.so):
 *   qmv_probe_read  - read-only streaming kernel over a device buffer, the
 *                     measured read bandwidth the matvec kernels are compared
 *                     with besides the nominal 8 TB/s;
 *   qmv_probe_copy  - plain copy of a known size, used to calibrate what the
 *                     FETCH_SIZE / WRITE_SIZE counters report per byte moved.
 * Each call allocates its buffers, runs warm-up passes, times `reps` passes
 * with HIP events on its own stream, frees everything and returns 1 (0 and
 * no timing on any HIP error).
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

/* Each thread reads `per` 16-byte words at a stride of the whole grid, so
 * the grid covers exactly blocks * threads * per words (the host sizes the
 * buffer to that). One word per thread is written to keep the loads live. */
__global__ void __launch_bounds__(256) read_kernel(const uint4 *__restrict__ src, uint32_t *__restrict__ sink,
                                                   int per)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
#pragma unroll 4
    for (int k = 0; k < per; ++k, i += stride) {
        const uint4 v = src[i];
        acc ^= v.x + v.y + v.z + v.w;
    }
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

__global__ void __launch_bounds__(256) copy_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                                   size_t n)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

struct Timer {
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    bool ok = false;
    Timer()
    {
        ok = hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess &&
             hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess;
    }
    ~Timer()
    {
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        if (s) (void)hipStreamDestroy(s);
    }
};

} // namespace

extern "C" __attribute__((visibility("default"))) int qmv_probe_read(uint64_t bytes, int blocks, int reps,
                                                                     double *ms_per_pass, uint64_t *bytes_read)
{
    if (bytes < 16 || blocks <= 0 || reps <= 0 || !ms_per_pass) return 0;
    const int threads = 256;
    const size_t total = (size_t)blocks * threads;
    const int per = (int)((bytes / 16 + total - 1) / total);
    const size_t words = (size_t)per * total;
    Timer t;
    if (!t.ok) return 0;
    uint4 *src = nullptr;
    uint32_t *sink = nullptr;
    int ok = hipMalloc(&src, words * 16) == hipSuccess && hipMalloc(&sink, total * 4) == hipSuccess &&
             hipMemsetAsync(src, 1, words * 16, t.s) == hipSuccess;
    for (int r = 0; ok && r < 2; ++r) {
        hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(threads), 0, t.s, src, sink, per);
        ok = hipGetLastError() == hipSuccess;
    }
    ok = ok && hipEventRecord(t.e0, t.s) == hipSuccess;
    for (int r = 0; ok && r < reps; ++r) {
        hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(threads), 0, t.s, src, sink, per);
        ok = hipGetLastError() == hipSuccess;
    }
    float ms = 0.0f;
    ok = ok && hipEventRecord(t.e1, t.s) == hipSuccess && hipStreamSynchronize(t.s) == hipSuccess &&
         hipEventElapsedTime(&ms, t.e0, t.e1) == hipSuccess;
    if (src) (void)hipFree(src);
    if (sink) (void)hipFree(sink);
    if (!ok) return 0;
    *ms_per_pass = ms / reps;
    if (bytes_read) *bytes_read = words * 16;
    return 1;
}

extern "C" __attribute__((visibility("default"))) int qmv_probe_copy(uint64_t bytes, int reps, double *ms_per_pass)
{
    if (bytes < 16 || reps <= 0 || !ms_per_pass) return 0;
    const size_t n = bytes / 16;
    Timer t;
    if (!t.ok) return 0;
    uint4 *src = nullptr, *dst = nullptr;
    int ok = hipMalloc(&src, n * 16) == hipSuccess && hipMalloc(&dst, n * 16) == hipSuccess &&
             hipMemsetAsync(src, 1, n * 16, t.s) == hipSuccess;
    const int blocks = 2048, threads = 256;
    ok = ok && hipEventRecord(t.e0, t.s) == hipSuccess;
    for (int r = 0; ok && r < reps; ++r) {
        hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(threads), 0, t.s, src, dst, n);
        ok = hipGetLastError() == hipSuccess;
    }
    float ms = 0.0f;
    ok = ok && hipEventRecord(t.e1, t.s) == hipSuccess && hipStreamSynchronize(t.s) == hipSuccess &&
         hipEventElapsedTime(&ms, t.e0, t.e1) == hipSuccess;
    if (src) (void)hipFree(src);
    if (dst) (void)hipFree(dst);
    if (!ok) return 0;
    *ms_per_pass = ms / reps;
    return 1;
}
