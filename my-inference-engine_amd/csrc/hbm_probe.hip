/*
 * HBM probes for measurement, not part of the matvec path (libqmv_probe.so):
 *   qmv_probe_read  - read-only streaming kernel over a device buffer, the
 *                     measured read bandwidth the matvec kernels are compared
 *                     with besides the nominal 8 TB/s;
 *   qmv_probe_copy  - plain copy of a known size, used to calibrate what the
 *                     FETCH_SIZE / WRITE_SIZE counters report per byte moved;
 *   qmv_probe_read_chain - a chain of dependent read-only launches over
 *                     distinct buffers of given sizes, replayed from a HIP
 *                     graph: the streaming floor of a sequence of matvec
 *                     launches that read the same bytes (no decode, no
 *                     reduction, the same launch boundaries).
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

/* Read-only streaming of `words` 16-byte words: each thread issues PER loads
 * at a stride of the whole grid before using any (so PER loads are in
 * flight per thread), the grid covering the buffer once. */
template <int PER>
__global__ void __launch_bounds__(256) read_once_kernel(const uint4 *__restrict__ src, size_t words,
                                                        uint32_t *__restrict__ sink)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t i0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint4 v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const size_t i = i0 + k * stride;
        v[k] = i < words ? src[i] : make_uint4(0, 0, 0, 0);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int k = 0; k < PER; ++k) acc ^= v[k].x + v[k].y + v[k].z + v[k].w;
    if (acc == 0x9e3779b9u) sink[i0] = acc; /* keeps the loads live; practically never stores */
}

typedef void (*ReadOnce)(const uint4 *, size_t, uint32_t *);

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

/* Streaming floor of a launch sequence: buffer i (bytes[i] bytes, rounded up
 * to 16) is read once by launch i, the launches in order on one stream,
 * captured once into a graph and replayed `reps` times after two warm-up
 * replays. Each launch covers its buffer with workgroups of 256 threads that
 * each issue `per` (1, 2, 4 or 8) 16-byte loads before using any. Returns the
 * microseconds per replay of the whole chain. */
extern "C" __attribute__((visibility("default"))) int qmv_probe_read_chain(const uint64_t *bytes, int n, int per,
                                                                           int reps, double *us_per_chain)
{
    if (!bytes || n <= 0 || reps <= 0 || !us_per_chain) return 0;
    const void *kernel = per == 1   ? (const void *)read_once_kernel<1>
                         : per == 2 ? (const void *)read_once_kernel<2>
                         : per == 4 ? (const void *)read_once_kernel<4>
                         : per == 8 ? (const void *)read_once_kernel<8>
                                    : nullptr;
    if (!kernel) return 0;
    const int threads = 256;
    Timer t;
    if (!t.ok) return 0;
    uint4 **bufs = new uint4 *[n]();
    size_t *words = new size_t[n];
    uint32_t *sink = nullptr;
    size_t max_threads = 0;
    for (int i = 0; i < n; ++i) {
        words[i] = (bytes[i] + 15) / 16;
        const size_t g = (words[i] + (size_t)threads * per - 1) / ((size_t)threads * per);
        if (g * threads > max_threads) max_threads = g * threads;
    }
    int ok = max_threads <= 0x7fffffffull && hipMalloc(&sink, max_threads * 4) == hipSuccess;
    for (int i = 0; ok && i < n; ++i)
        ok = hipMalloc(&bufs[i], words[i] * 16) == hipSuccess &&
             hipMemsetAsync(bufs[i], 1, words[i] * 16, t.s) == hipSuccess;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    ok = ok && hipStreamSynchronize(t.s) == hipSuccess &&
         hipStreamBeginCapture(t.s, hipStreamCaptureModeThreadLocal) == hipSuccess;
    if (ok) {
        for (int i = 0; i < n; ++i) {
            const unsigned g = (unsigned)((words[i] + (size_t)threads * per - 1) / ((size_t)threads * per));
            hipLaunchKernelGGL((ReadOnce)kernel, dim3(g), dim3(threads), 0, t.s, bufs[i], words[i], sink);
        }
        ok = hipStreamEndCapture(t.s, &graph) == hipSuccess && hipGetLastError() == hipSuccess &&
             hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
    }
    for (int r = 0; ok && r < 2; ++r) ok = hipGraphLaunch(exec, t.s) == hipSuccess;
    ok = ok && hipEventRecord(t.e0, t.s) == hipSuccess;
    for (int r = 0; ok && r < reps; ++r) ok = hipGraphLaunch(exec, t.s) == hipSuccess;
    float ms = 0.0f;
    ok = ok && hipEventRecord(t.e1, t.s) == hipSuccess && hipStreamSynchronize(t.s) == hipSuccess &&
         hipEventElapsedTime(&ms, t.e0, t.e1) == hipSuccess;
    (void)hipStreamSynchronize(t.s);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    for (int i = 0; i < n; ++i)
        if (bufs[i]) (void)hipFree(bufs[i]);
    if (sink) (void)hipFree(sink);
    delete[] bufs;
    delete[] words;
    if (!ok) return 0;
    *us_per_chain = ms * 1e3 / reps;
    return 1;
}
