/*
 * Host side of libqmv_hip.so: the C ABI declared in include/qmv_hip.h.
 *
 *  - Argument validation restated from the reference's dispatch
 *    (src/quantized_matvec.cpp:93-149 for the matvec, :168-191 for the
 *    batched form); every rule runs before any HIP call, so invalid calls
 *    return 0 without touching the GPU.
 *  - A thread-safe cache of device tensors keyed by (device, host data
 *    pointer, type, shape), guarded by a sampled content fingerprint, so each
 *    packed tensor is uploaded and re-tiled once (the reference reads the same
 *    bytes from its mmap on every call).
 *  - A per-device pool of contexts (HIP stream, pinned staging, device I/O
 *    buffers) that host-pointer calls check out for their duration, from
 *    any thread (sessions call concurrently); a per-stream workspace
 *    (split-K partials, arrival counters, argmax partials).
 *  - Launch planning: tiles of 64 rows x K-units spread over waves,
 *    workgroups and K-splits.
 */
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <atomic>
#include <condition_variable>
#include <string>
#include <tuple>
#include <vector>

#include "qmv_hip.h"
#include "qmv_kernels.h"
#include "qmv_layout.h"

#define QMV_API extern "C" __attribute__((visibility("default")))

struct QmvDeviceTensor {
    int device;
    uint32_t ggml_type;
    QmvGeometry geo;
    int rows, cols;
    int blocks_per_row;
    int units, tiles;
    uint64_t packed_bytes, device_bytes;
    uint8_t *data;
    uint8_t *rowmajor; /* row-major copy (Q4_K: the GGUF bytes; Q6_K: planes), else null */
};

namespace {

/* ---- errors ----------------------------------------------------------------- */

thread_local std::string t_error;

void set_error(const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_error = buf;
}

bool hip_ok(hipError_t e, const char *what)
{
    if (e == hipSuccess) return true;
    set_error("%s failed: %s", what, hipGetErrorString(e));
    return false;
}

#define HIP_TRY(expr)                         \
    do {                                      \
        if (!hip_ok((expr), #expr)) return 0; \
    } while (0)

std::atomic<int> g_device{0};
std::atomic<int> g_fail_next{0};

/* Every device, pinned-host or stream allocation the library makes, counted
 * (qmv_allocation_count): after registration and qmv_reserve_calls, matvec
 * calls within the reserved sizes leave it unchanged. */
std::atomic<unsigned long long> g_allocations{0};

hipError_t counted_malloc(void **p, size_t bytes)
{
    g_allocations.fetch_add(1);
    return hipMalloc(p, bytes);
}

hipError_t counted_host_malloc(void **p, size_t bytes)
{
    g_allocations.fetch_add(1);
    return hipHostMalloc(p, bytes, hipHostMallocDefault);
}

/* ---- validation (src/quantized_matvec.cpp:93-149, :168-191) ------------------ */

struct Shape {
    QmvGeometry geo;
    int rows, cols, blocks_per_row;
};

bool view_layout_ok(const QmvTensorView *m, Shape *out)
{
    if (m == nullptr || m->data == nullptr) { set_error("null tensor view or data"); return false; }
    if (m->dimension_count != 2) { set_error("tensor view must be 2-D"); return false; }
    const uint64_t cols = m->dimensions[0], rows = m->dimensions[1];
    if (cols == 0 || rows == 0 || cols > INT_MAX || rows > INT_MAX) {
        set_error("tensor dimensions must be in 1..INT_MAX");
        return false;
    }
    QmvGeometry g;
    if (!qmv_geometry_of(m->ggml_type, &g)) {
        set_error("unsupported ggml type %u (need Q5_0, Q8_0, Q4_K or Q6_K)", m->ggml_type);
        return false;
    }
    if (m->block_elements != (uint64_t)g.block_elements || m->block_bytes != (uint64_t)g.block_bytes ||
        cols % (uint64_t)g.block_elements != 0) {
        set_error("block layout does not match the type or the column count");
        return false;
    }
    const uint64_t bpr = cols / (uint64_t)g.block_elements;
    if (bpr > UINT64_MAX / rows || m->block_count != bpr * rows || cols > UINT64_MAX / rows ||
        m->element_count != cols * rows || m->block_count > SIZE_MAX / (uint64_t)g.block_bytes) {
        set_error("element_count/block_count disagree with the shape");
        return false;
    }
    out->geo = g;
    out->rows = (int)rows;
    out->cols = (int)cols;
    out->blocks_per_row = (int)bpr;
    return true;
}

bool matvec_args_ok(const QmvTensorView *m, const float *in, int in_count, const float *outp, int out_count,
                    int batch, Shape *s)
{
    if (m == nullptr || in == nullptr || outp == nullptr || in_count <= 0 || out_count <= 0 || batch <= 0) {
        set_error("null pointer or non-positive count");
        return false;
    }
    if (!view_layout_ok(m, s)) return false;
    if (in_count != s->cols || out_count != s->rows) {
        set_error("input_count/output_count (%d, %d) do not match the tensor (%d cols, %d rows)", in_count,
                  out_count, s->cols, s->rows);
        return false;
    }
    if ((size_t)batch > SIZE_MAX / (size_t)in_count || (size_t)batch > SIZE_MAX / (size_t)out_count) {
        set_error("batch size overflows");
        return false;
    }
    return true;
}

/* ---- per-device / per-stream workspace --------------------------------------- */

struct Workspace {
    float *partials = nullptr;
    size_t partial_cap = 0; /* floats */
    unsigned *counters = nullptr;
    size_t counter_cap = 0;
    float *arg_val = nullptr;
    int *arg_idx = nullptr;
    int *arg_bad = nullptr;
    int *arg_result = nullptr; /* 2 ints */
    uint64_t *fused_cand = nullptr;  /* fused argmax: tile and group candidates */
    unsigned *fused_count = nullptr; /* fused argmax: arrival counts, zero between launches */
    size_t fused_cap = 0;            /* tiles */
    /* Buffers replaced by a larger one. They are never freed: a graph
     * captured earlier on this stream still launches kernels that use them
     * (every launch leaves its counters at zero, so such replays stay
     * correct). Growth is geometric, so they hold less than twice the final
     * size. */
    std::vector<void *> retired;
    std::mutex mu;
};

/* Grow the workspace; waits for work already queued on the stream. New
 * counters are zeroed on the stream the kernels run on (never inside a graph
 * capture: growth is refused there), so every launch finds them zero. */
int workspace_reserve(Workspace &ws, hipStream_t stream, size_t partials, size_t counters)
{
    if (partials <= ws.partial_cap && counters <= ws.counter_cap) return 1;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone) {
        set_error("workspace must grow during stream capture; run the call once before capturing");
        return 0;
    }
    HIP_TRY(hipStreamSynchronize(stream));
    if (partials > ws.partial_cap) {
        const size_t n = partials + partials / 2 + 4096;
        float *np = nullptr;
        HIP_TRY(counted_malloc((void **)&np, n * sizeof(float)));
        if (ws.partials) ws.retired.push_back(ws.partials);
        ws.partials = np;
        ws.partial_cap = n;
    }
    if (counters > ws.counter_cap) {
        const size_t n = counters + counters / 2 + 1024;
        unsigned *nc = nullptr;
        HIP_TRY(counted_malloc((void **)&nc, n * sizeof(unsigned)));
        if (ws.counters) ws.retired.push_back(ws.counters);
        ws.counters = nc;
        ws.counter_cap = 0;
        HIP_TRY(hipMemsetAsync(ws.counters, 0, n * sizeof(unsigned), stream));
        ws.counter_cap = n;
    }
    return 1;
}

constexpr int kArgBlocks = 512;

/* Candidate slots and counters for a fused argmax over `tiles` tiles (grown
 * outside graph capture only; counters are zeroed on the launch stream). */
int workspace_fused_argmax(Workspace &ws, hipStream_t stream, size_t tiles)
{
    if (tiles <= ws.fused_cap) return 1;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone) {
        set_error("workspace must grow during stream capture; run the call once before capturing");
        return 0;
    }
    HIP_TRY(hipStreamSynchronize(stream));
    const size_t n = tiles + tiles / 2 + 256;
    uint64_t *cand = nullptr;
    unsigned *count = nullptr;
    HIP_TRY(counted_malloc((void **)&cand, qmv::argmax_words(n) * sizeof(uint64_t)));
    if (!hip_ok(counted_malloc((void **)&count, qmv::argmax_counts(n) * sizeof(unsigned)), "hipMalloc")) {
        ws.retired.push_back(cand);
        return 0;
    }
    if (ws.fused_cand) ws.retired.push_back(ws.fused_cand);
    if (ws.fused_count) ws.retired.push_back(ws.fused_count);
    ws.fused_cand = cand;
    ws.fused_count = count;
    ws.fused_cap = 0;
    HIP_TRY(hipMemsetAsync(ws.fused_count, 0, qmv::argmax_counts(n) * sizeof(unsigned), stream));
    ws.fused_cap = n;
    return 1;
}

int workspace_argmax(Workspace &ws)
{
    if (ws.arg_result) return 1;
    HIP_TRY(counted_malloc((void **)&ws.arg_val, kArgBlocks * sizeof(float)));
    HIP_TRY(counted_malloc((void **)&ws.arg_idx, kArgBlocks * sizeof(int)));
    HIP_TRY(counted_malloc((void **)&ws.arg_bad, kArgBlocks * sizeof(int)));
    HIP_TRY(counted_malloc((void **)&ws.arg_result, 2 * sizeof(int)));
    return 1;
}

std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, std::unique_ptr<Workspace>> g_workspaces;

Workspace &workspace_for(int device, hipStream_t stream)
{
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto &slot = g_workspaces[{device, stream}];
    if (!slot) slot.reset(new Workspace());
    return *slot;
}

/* ---- pooled contexts for the host-pointer entry points --------------------------
 * A host-pointer call checks a context out of its device's pool for the
 * duration of the call: a non-blocking HIP stream with that stream's split-K
 * workspace, pinned staging for the input and the output, and device buffers.
 * Any thread may run on any context (a thread first tries the one it used
 * last), so a session may move between threads, as the reference allows
 * (include/engine_api.h:12-13). Until the first reservation
 * (qmv_reserve_calls, qmv_reserve_contexts) a pool grows when every context
 * is checked out. A reservation closes it: from then on a call that finds
 * every context checked out waits for one instead of creating another, and
 * every context holds at least the largest reservation's staging and
 * workspace, so reserved calls allocate nothing on any thread. Contexts are
 * never freed (HIP may already be torn down at process exit). */

struct CtxPool;

struct HostCtx {
    int device = -1;
    CtxPool *pool = nullptr;
    hipStream_t stream = nullptr;
    Workspace *ws = nullptr; /* the stream's split-K workspace */
    float *h_in = nullptr, *h_out = nullptr;
    size_t h_in_cap = 0, h_out_cap = 0;
    float *d_in = nullptr, *d_out = nullptr; /* d_out: dequantised rows, sampler results */
    size_t d_in_cap = 0, d_out_cap = 0;
    bool busy = false; /* checked out; guarded by the pool's mutex */
};

/* What a context holds at least: input and output staging floats, split-K
 * partial floats and counter words. */
struct CtxSizes {
    size_t nin = 0, nout = 0, partials = 0, counters = 0;
};

CtxSizes max_sizes(const CtxSizes &a, const CtxSizes &b)
{
    CtxSizes z;
    z.nin = a.nin > b.nin ? a.nin : b.nin;
    z.nout = a.nout > b.nout ? a.nout : b.nout;
    z.partials = a.partials > b.partials ? a.partials : b.partials;
    z.counters = a.counters > b.counters ? a.counters : b.counters;
    return z;
}

struct CtxPool {
    std::mutex mu;
    std::condition_variable cv;
    std::vector<HostCtx *> all;
    bool closed = false; /* reserved: wait for a context rather than create one */
    CtxSizes sizes;      /* every context of a closed pool holds at least these */
};

/* Contexts per device at most (a pool that was never reserved stops growing
 * there and waits instead). */
constexpr int kMaxContexts = 1024;

std::mutex g_pools_mu;
std::map<int, CtxPool *> g_pools; /* pools are never destroyed */

CtxPool &pool_for(int device)
{
    std::lock_guard<std::mutex> lock(g_pools_mu);
    CtxPool *&p = g_pools[device];
    if (!p) p = new CtxPool();
    return *p;
}

int grow_pinned(float **p, size_t *cap, size_t n)
{
    if (n <= *cap) return 1;
    if (*p) HIP_TRY(hipHostFree(*p));
    *p = nullptr;
    *cap = 0;
    const size_t m = n + n / 2 + 1024;
    HIP_TRY(counted_host_malloc((void **)p, m * sizeof(float)));
    *cap = m;
    return 1;
}

int grow_device(float **p, size_t *cap, size_t n)
{
    if (n <= *cap) return 1;
    if (*p) HIP_TRY(hipFree(*p));
    *p = nullptr;
    *cap = 0;
    const size_t m = n + n / 2 + 1024;
    HIP_TRY(counted_malloc((void **)p, m * sizeof(float)));
    *cap = m;
    return 1;
}

/* Grow a checked-out context to hold z (nothing is allocated if it does). */
int ctx_fit(HostCtx *c, const CtxSizes &z)
{
    if (!grow_pinned(&c->h_in, &c->h_in_cap, z.nin) || !grow_pinned(&c->h_out, &c->h_out_cap, z.nout) ||
        !grow_device(&c->d_in, &c->d_in_cap, z.nin))
        return 0;
    std::lock_guard<std::mutex> lock(c->ws->mu);
    return workspace_reserve(*c->ws, c->stream, z.partials, z.counters);
}

/* A new context on the current device, sized to z; added to the pool as
 * checked out (busy) or idle. Called with the pool's mutex held, so that a
 * reservation sees every context the pool will ever have when it closes it. */
HostCtx *ctx_create_locked(CtxPool &pool, int device, const CtxSizes &z, bool busy)
{
    if ((int)pool.all.size() >= kMaxContexts) {
        set_error("more than %d host contexts requested on device %d", kMaxContexts, device);
        return nullptr;
    }
    std::unique_ptr<HostCtx> c(new HostCtx());
    g_allocations.fetch_add(1);
    if (!hip_ok(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate")) return nullptr;
    c->device = device;
    c->pool = &pool;
    c->ws = &workspace_for(device, c->stream);
    if (!ctx_fit(c.get(), z)) return nullptr; /* the stream stays (contexts are never freed) */
    c->busy = busy;
    pool.all.push_back(c.get());
    return c.release();
}

thread_local HostCtx *t_last_ctx = nullptr;

/* Check a context of the selected device out of its pool (waits while a
 * closed pool has none free). The device is made current. */
HostCtx *ctx_acquire()
{
    const int dev = g_device.load();
    if (!hip_ok(hipSetDevice(dev), "hipSetDevice")) return nullptr;
    CtxPool &pool = pool_for(dev);
    std::unique_lock<std::mutex> lock(pool.mu);
    for (;;) {
        HostCtx *pick = nullptr;
        if (t_last_ctx != nullptr && t_last_ctx->pool == &pool && !t_last_ctx->busy) {
            pick = t_last_ctx;
        } else {
            for (HostCtx *c : pool.all)
                if (!c->busy) {
                    pick = c;
                    break;
                }
        }
        if (pick != nullptr) {
            pick->busy = true;
            t_last_ctx = pick;
            return pick;
        }
        if (!pool.closed && (int)pool.all.size() < kMaxContexts) break;
        pool.cv.wait(lock);
    }
    HostCtx *c = ctx_create_locked(pool, dev, pool.sizes, true);
    if (c != nullptr) t_last_ctx = c;
    return c;
}

void ctx_release(HostCtx *c)
{
    {
        std::lock_guard<std::mutex> lock(c->pool->mu);
        c->busy = false;
    }
    /* Every waiter re-checks: a reservation waits for one particular context. */
    c->pool->cv.notify_all();
}

/* A context checked out for one call. A call that ends early (failure) may
 * leave work queued on the stream that still reads the staging buffers, so
 * the stream is drained before the next caller gets the context. */
class CtxLease {
public:
    CtxLease() : c(ctx_acquire()) {}
    ~CtxLease()
    {
        if (c == nullptr) return;
        if (!done) (void)hipStreamSynchronize(c->stream);
        ctx_release(c);
    }
    CtxLease(const CtxLease &) = delete;
    CtxLease &operator=(const CtxLease &) = delete;
    HostCtx *const c;
    bool done = false; /* the call drained its stream */
};

/* Close the selected device's pool, raise what every context holds to at
 * least `need`, grow each existing context to that, and create contexts up to
 * `count`. Waits for contexts that are checked out. */
int pool_reserve(const CtxSizes &need, int count)
{
    const int dev = g_device.load();
    HIP_TRY(hipSetDevice(dev));
    CtxPool &pool = pool_for(dev);
    std::vector<HostCtx *> existing;
    CtxSizes z;
    {
        std::lock_guard<std::mutex> lock(pool.mu);
        pool.closed = true;
        pool.sizes = max_sizes(pool.sizes, need);
        z = pool.sizes;
        existing = pool.all;
    }
    for (HostCtx *c : existing) {
        {
            std::unique_lock<std::mutex> lock(pool.mu);
            pool.cv.wait(lock, [c] { return !c->busy; });
            c->busy = true;
        }
        const int ok = ctx_fit(c, z);
        ctx_release(c);
        if (!ok) return 0;
    }
    std::lock_guard<std::mutex> lock(pool.mu);
    while ((int)pool.all.size() < count)
        if (ctx_create_locked(pool, dev, z, false) == nullptr) return 0;
    pool.cv.notify_all();
    return 1;
}

int env_int(const char *name, int dflt)
{
    const char *v = getenv(name);
    if (!v || !*v) return dflt;
    return atoi(v);
}

/* Row-major single-position kernel for Q4_K launches (rowgroup_q4k_kernel).
 * QMV_ROWDOT = 0 turns it off at start-up and qmv_set_rowmajor at run time
 * (tensors uploaded while it is off keep no GGUF copy); QMV_ROWDOT_ROWS /
 * qmv_set_rowmajor set the rows a 64-lane row segment takes in launches of
 * at most kRowdotMaxUnits (tile, unit) pairs (1, 2 or 4; shorter rows'
 * segments take 2). Measured on MI355X in a graph of the Qwen2.5-7B decode
 * set, us per launch, q|k|v / o: tiled 6.81 / 5.80; workgroups of 4 waves
 * sharing the activations in LDS, 1, 2 or 4 rows per wave: 4.85 / 4.19,
 * 4.87 / 4.08, 5.67 / 4.51 (2 rows and per-wave activation loads: 7.1 / 5.8;
 * 2 rows with 1, 2 or 8 waves per workgroup: 5.6 / 4.7, 5.2 / 4.8,
 * 5.8 / 4.0). Larger launches of rows of at most 16 super-blocks (gate|up,
 * 2 x 18944 x 3584: 8288 pairs) take kRowdotRowsLarge = 4 rows per segment:
 * 16.5 us against 18.1 tiled (2 rows: 19.0, 8 rows: 17.7), and the decode
 * set 1.139 ms against 1.189 (8 rows: 1.189); longer rows stay tiled there. */
std::atomic<int> g_rowdot{env_int("QMV_ROWDOT", 1)};
std::atomic<int> g_rowdot_rows{env_int("QMV_ROWDOT_ROWS", 2)};

/* Super-blocks per row the row-major kernel takes: 8 waves x 64 lanes, 4
 * lanes per super-block. */
constexpr int kRowdotMaxSb = QMV_MAX_WAVES * 64 / 4;
/* Launches of up to this many tiled (64-row tile, K-unit) pairs, summed over
 * the launch's tensors, run row-major with any row length up to
 * kRowdotMaxSb (Qwen2.5-7B q|k|v: 1008, o: 784); larger ones only with rows
 * of at most kRowdotSharedSb super-blocks (one LDS copy of the activations
 * per workgroup), at kRowdotRowsLarge rows per segment. */
constexpr long long kRowdotMaxUnits = 2048;
constexpr int kRowdotSharedSb = 16;
constexpr int kRowdotRowsLarge = 4;
/* The fused SwiGLU of such launches (gate and up rows in every segment, so
 * twice the loads in flight per row) takes 2: 16.7-17.8 us against 18.0-18.4
 * at 4 and 19.1 at 1. A row's sum does not depend on the rows per segment,
 * so the fused result stays that of the plain launch's rows bit for bit. */
constexpr int kRowdotRowsLargeSwiglu = 2;
/* Q6_K rows of 17 to kRowdotMaxSb super-blocks keep a row-major copy in the
 * chunked plane layout of rowloop_q6k_kernel (q6k_row_stride bytes per row)
 * and run their single-position launches there (QMV_ROWDOT_Q6K = 0 at
 * start-up keeps them tiled): one row per wave, workgroups of
 * ceil(rows / kRowloopQ6Groups) waves (at most 16), each copying the
 * activations into LDS once. Measured on MI355X, Qwen2.5-7B down
 * (3584 x 18944), us per launch: 14.2 with 224 workgroups of 16 waves, 15.0
 * with 256 of 14, 15.7 with 512 of 7, against 14.4-14.6 tiled; loading two
 * or three slices ahead instead of one, 15.0 and 16.0. In the decode set's
 * graph the step went 1.128 -> 1.108 ms (no split-K tail before the next
 * launch), 1.095-1.101 with every wave copying its share of the
 * activations. */
std::atomic<int> g_rowdot_q6{env_int("QMV_ROWDOT_Q6K", 1)};
constexpr long long kRowloopQ6Groups = 224;

long long tiled_units(int rows, int blocks_per_row)
{
    return (long long)((rows + QMV_TILE_ROWS - 1) / QMV_TILE_ROWS) * blocks_per_row;
}

/* Whether an upload also keeps the GGUF bytes for the row-major kernel. */
bool keeps_rowmajor(const QmvGeometry &geo, int rows, int blocks_per_row)
{
    if (g_rowdot.load() == 0 || blocks_per_row > kRowdotMaxSb) return false;
    if (geo.format == QMV_FMT_Q6_K) return g_rowdot_q6.load() != 0 && blocks_per_row > kRowdotSharedSb;
    return geo.format == QMV_FMT_Q4_K &&
           (tiled_units(rows, blocks_per_row) <= kRowdotMaxUnits || blocks_per_row <= kRowdotSharedSb);
}

/* ---- upload ------------------------------------------------------------------- */

void tensor_free(QmvDeviceTensor *t)
{
    if (!t) return;
    if (t->data || t->rowmajor) {
        int cur = 0;
        const bool other = hipGetDevice(&cur) == hipSuccess && cur != t->device;
        if (!other || hipSetDevice(t->device) == hipSuccess) {
            if (t->data) (void)hipFree(t->data);
            if (t->rowmajor) (void)hipFree(t->rowmajor);
            if (other) (void)hipSetDevice(cur);
        }
    }
    delete t;
}

int tensor_upload(const QmvTensorView *m, const Shape &s, int device, hipStream_t stream, QmvDeviceTensor **out)
{
    std::unique_ptr<QmvDeviceTensor, void (*)(QmvDeviceTensor *)> t(new QmvDeviceTensor(), tensor_free);
    t->device = device;
    t->ggml_type = m->ggml_type;
    t->geo = s.geo;
    t->rows = s.rows;
    t->cols = s.cols;
    t->blocks_per_row = s.blocks_per_row;
    t->units = (s.blocks_per_row + s.geo.blocks_per_unit - 1) / s.geo.blocks_per_unit;
    t->tiles = (s.rows + QMV_TILE_ROWS - 1) / QMV_TILE_ROWS;
    t->packed_bytes = (uint64_t)s.rows * (uint64_t)s.blocks_per_row * (uint64_t)s.geo.block_bytes;
    t->device_bytes = (uint64_t)t->tiles * (uint64_t)t->units * QMV_TILE_ROWS * (uint64_t)s.geo.unit_bytes;
    t->data = nullptr;
    t->rowmajor = nullptr;

    uint8_t *raw = nullptr;
    HIP_TRY(counted_malloc((void **)&raw, t->packed_bytes));
    std::unique_ptr<uint8_t, hipError_t (*)(void *)> raw_guard(raw, hipFree);
    HIP_TRY(hipMemcpyAsync(raw, m->data, t->packed_bytes, hipMemcpyHostToDevice, stream));
    HIP_TRY(counted_malloc((void **)&t->data, t->device_bytes));
    if (t->device_bytes != t->packed_bytes) HIP_TRY(hipMemsetAsync(t->data, 0, t->device_bytes, stream));
    HIP_TRY(qmv::launch_repack(s.geo.format, raw, t->data, s.rows, s.blocks_per_row, t->units,
                               s.geo.blocks_per_unit, s.geo.block_bytes, s.geo.unit_bytes, t->tiles, stream));
    HIP_TRY(hipStreamSynchronize(stream));
    if (keeps_rowmajor(s.geo, s.rows, s.blocks_per_row)) {
        if (s.geo.format == QMV_FMT_Q6_K) {
            const uint64_t bytes = (uint64_t)s.rows * qmv::q6k_row_stride(s.blocks_per_row);
            HIP_TRY(counted_malloc((void **)&t->rowmajor, bytes));
            HIP_TRY(hipMemsetAsync(t->rowmajor, 0, bytes, stream));
            HIP_TRY(qmv::launch_rowmajor_q6k(raw, t->rowmajor, s.rows, s.blocks_per_row, stream));
            HIP_TRY(hipStreamSynchronize(stream));
            t->device_bytes += bytes;
        } else {
            t->rowmajor = raw_guard.release();
            t->device_bytes += t->packed_bytes;
        }
    }
    *out = t.release();
    return 1;
}

/* Fingerprint of the host bytes: catches a reused data pointer that now
 * holds a different tensor (the reference's views die at gguf_close). Every
 * byte of tensors up to kFullHashBytes (a few microseconds of hashing), 64
 * sampled words of larger ones, whose callers release them on change. */
constexpr uint64_t kFullHashBytes = 64u << 10;

uint64_t fingerprint(const QmvTensorView *m, uint64_t bytes)
{
    uint64_t h = 0x9E3779B97F4A7C15ull ^ bytes;
    if (bytes <= kFullHashBytes) {
        uint64_t off = 0;
        for (; off + 8 <= bytes; off += 8) {
            uint64_t w;
            memcpy(&w, m->data + off, 8);
            h = (h ^ w) * 0x100000001b3ull;
            h ^= h >> 29;
        }
        for (; off < bytes; ++off) h = (h ^ m->data[off]) * 0x100000001b3ull;
        return h;
    }
    const int samples = 64;
    for (int i = 0; i < samples; ++i) {
        uint64_t off = bytes <= 8 ? 0 : (bytes - 8) * (uint64_t)i / (uint64_t)(samples - 1);
        uint64_t w = 0;
        memcpy(&w, m->data + off, bytes < 8 ? bytes : 8);
        h = (h ^ w) * 0x100000001b3ull;
        h ^= h >> 29;
    }
    return h;
}

struct CacheEntry {
    std::shared_ptr<QmvDeviceTensor> tensor;
    uint64_t fp;
};

/* Heap-allocated and never destroyed: its entries free device memory, which
 * must not happen during static destruction (HIP may be gone by then). */
std::mutex g_cache_mu;
auto &g_cache = *new std::map<std::tuple<int, const unsigned char *, uint32_t, int, int>, CacheEntry>();

std::shared_ptr<QmvDeviceTensor> cached_tensor(const QmvTensorView *m, const Shape &s, HostCtx *c)
{
    const uint64_t bytes = (uint64_t)s.rows * (uint64_t)s.blocks_per_row * (uint64_t)s.geo.block_bytes;
    const uint64_t fp = fingerprint(m, bytes);
    const auto key = std::make_tuple(c->device, m->data, m->ggml_type, s.rows, s.cols);
    std::lock_guard<std::mutex> lock(g_cache_mu);
    auto it = g_cache.find(key);
    if (it != g_cache.end() && it->second.fp == fp) return it->second.tensor;
    QmvDeviceTensor *t = nullptr;
    if (!tensor_upload(m, s, c->device, c->stream, &t)) return nullptr;
    std::shared_ptr<QmvDeviceTensor> sp(t, tensor_free);
    g_cache[key] = CacheEntry{sp, fp};
    return sp;
}

/* ---- launch planning ------------------------------------------------------------- */

std::atomic<int> g_target_waves{env_int("QMV_TARGET_WAVES", 0)};
std::atomic<int> g_force_u{env_int("QMV_UNITS_PER_WAVE", 0)};
std::atomic<int> g_force_w{env_int("QMV_WAVES_PER_GROUP", 0)};
/* Smallest batch run on the matrix cores (Q4_K, Q6_K); above QMV_MAX_BATCH
 * turns them off (batches then run in launches of 8 on the VALU path). By default the batch from which they beat the VALU path on
 * MI355X at Qwen2.5-7B layer shapes: 7 for Q4_K, 8 for Q6_K (its code
 * assembly costs more VALU per weight on the matrix-core path). */
std::atomic<int> g_mfma_min_batch{env_int("QMV_MFMA_MIN_BATCH", 0)};
/* QMV_PAIRED_SWIGLU=0 runs the fused SwiGLU with the tile-pair count instead
 * of paired workgroups (for comparison). */
std::atomic<int> g_paired_swiglu{env_int("QMV_PAIRED_SWIGLU", 1)};
/* QMV_MFMA_PARTS = 1 or 2 forces the work items per unit of the
 * matrix-core kernel (for measurement). */
std::atomic<int> g_mfma_parts{env_int("QMV_MFMA_PARTS", 0)};
/* QMV_VALU_PARTS = 1 or 2: the same for the VALU kernels' batches. */
std::atomic<int> g_valu_parts{env_int("QMV_VALU_PARTS", 0)};

/* Q5_0 batches from this many positions run on the matrix cores (0: never).
 * Qwen2.5-1.5B q|k|v and o (Q5_0, K = 1536), us per launch, VALU / matrix
 * cores: M = 8 11.95 / 11.27 and 11.58 / 10.95; M = 5 9.37 / 9.27 and
 * 9.07 / 8.93; M = 4 8.65 / 8.71; M = 2 6.93 / 7.38. */
std::atomic<int> g_q5_mfma_min_batch{env_int("QMV_Q5_MFMA_MIN_BATCH", 5)};

/* Q8_0 batches from this many positions run on the matrix cores (0: never).
 * Q8_0 896 x 896 and 4864 x 896, us per launch, VALU / matrix cores: M = 8
 * 11.03 / 9.82 and 11.74 / 10.51; M = 4 7.97 / 7.56 and 8.34 / 8.20; M = 2
 * 6.44 / 6.25 and 6.72 / 6.95. */
std::atomic<int> g_q8_mfma_min_batch{env_int("QMV_Q8_MFMA_MIN_BATCH", 4)};

bool use_matrix_cores(int fmt, int batch)
{
    if (fmt == QMV_FMT_Q5_0 || fmt == QMV_FMT_Q8_0) {
        const int t = (fmt == QMV_FMT_Q5_0 ? g_q5_mfma_min_batch : g_q8_mfma_min_batch).load();
        return t > 0 && batch >= t && batch <= QMV_VALU_MAX_POSITIONS;
    }
    if (fmt != QMV_FMT_Q4_K && fmt != QMV_FMT_Q6_K) return false;
    const int t = g_mfma_min_batch.load();
    return batch >= (t > 0 ? t : fmt == QMV_FMT_Q4_K ? 7 : 8);
}

/* QMV_Q5_PREFILL=0 / QMV_Q8_PREFILL=0 keep Q5_0 / Q8_0 batches in launches
 * of 8 positions. */
std::atomic<int> g_q5_prefill{env_int("QMV_Q5_PREFILL", 1)};
std::atomic<int> g_q8_prefill{env_int("QMV_Q8_PREFILL", 1)};

/* Launches of 9..32 positions: the prefill kernel (all four formats). */
bool use_prefill(int fmt, int batch)
{
    if (batch <= QMV_VALU_MAX_POSITIONS) return false;
    if (fmt == QMV_FMT_Q5_0) return g_q5_prefill.load() != 0;
    if (fmt == QMV_FMT_Q8_0) return g_q8_prefill.load() != 0;
    return (fmt == QMV_FMT_Q4_K || fmt == QMV_FMT_Q6_K) && use_matrix_cores(fmt, batch);
}

struct Plan {
    int units_per_wave, waves, splits, units_per_split;
};

/* Default: one K-unit per wave and `short_waves` (4, one per SIMD; 5 for
 * large single-position launches) waves per workgroup;
 * for long rows (>= 32 K-units) at M = 1, `long_waves` = 6: down 3584 x
 * 18944 Q6_K takes 14.4 us against 15.8 at 8 and 15.1 at 4, whose 19 splits
 * need two rounds of partial loads. Batches keep 4 for long rows too (down at
 * M = 8: 42.2 us against 45 at 8 on the VALU path; 1536 x 8960 Q4_K at M = 2
 * and 4: 9-10% faster than at 8), except Q6_K on the matrix cores, which
 * takes 3 (plan_chunk). Many short workgroups keep every CU streaming until the
 * end and let the dispatcher balance the load; on MI355X this beat longer
 * waves and stream-K partitions at every decode shape measured. With
 * target_waves set, units per wave grow instead until about that many waves
 * cover the launch. */
Plan plan_for(long long total_tiles, int units, int long_waves, int short_waves, int max_u = 8)
{
    const int target = g_target_waves.load();
    const int force_u = g_force_u.load();
    const int force_w = g_force_w.load();
    int U = 1;
    if (target > 0) {
        const long long u = (total_tiles * (long long)units + target - 1) / target;
        U = (int)(u < 1 ? 1 : u > 8 ? 8 : u);
    }
    if (force_u > 0) U = force_u;
    if (U > max_u) U = max_u;
    if (U > units) U = units;
    int W = force_w > 0 ? force_w : target > 0 ? QMV_MAX_WAVES : units >= 32 ? long_waves : short_waves;
    const int need = (units + U - 1) / U;
    if (W > need) W = need;
    int S = (units + W * U - 1) / (W * U);
    /* Even splits: every split gets ceil(units / S) units. */
    const int ups = (units + S - 1) / S;
    if (force_u <= 0) U = (ups + W - 1) / W;
    if (force_w <= 0) W = (ups + U - 1) / U;
    S = (units + ups - 1) / ups;
    Plan p;
    p.units_per_wave = U;
    p.waves = W;
    p.splits = S;
    p.units_per_split = ups;
    return p;
}

/* Work items per K-unit on the matrix-core kernel (M <= 8): halves pay on
 * small launches over rows of few units, where a unit per wave leaves about
 * one wave per SIMD. Measured at M = 8 on the Qwen2.5-7B layer shapes (us per
 * launch, whole / half / quarter units): q|k|v (72 tiles x 14 units) 11.9 /
 * 10.8 / 12.4, o (56 x 14) 9.4 / 9.9 / 11.4, gate|up (592 x 14) 34.0 / 36.3 /
 * 50.8, down (56 x 74) 33.8 / 36.1 / 48.3; Qwen2.5-1.5B gate|up (280 x 6,
 * 1680 pairs) 13.4 / 12.9 (so the bound is 2048 pairs); with the current
 * finish, quarters cost 7B q|k|v 10.4 against 9.8 and 1.5B down 11.3 against
 * 9.75. More items cost more split-K partials than they gain, so quarters are
 * not built. */
int mfma_parts(int units, long long total_tiles)
{
    const int forced = g_mfma_parts.load();
    if (forced == 1 || forced == 2) return forced;
    return units < 32 && total_tiles * units <= 2048 ? 2 : 1;
}

/* Work items per K-unit on the VALU kernels for batches (M >= 2): halves.
 * Beyond 4 positions a region's activations load only after the previous
 * region's FMAs, so a unit is a long serial chain per wave; half units
 * double the waves and halve the chain. Measured (us per launch, whole /
 * half units): Qwen2.5-1.5B Q5_0 q|k|v and o at M = 8 13.7 / 11.9 and
 * 13.4 / 11.6; Qwen2.5-7B Q4_K q|k|v and o at M = 4 14.1 / 11.8 and
 * 13.3 / 11.1, at M = 2 11.0 / 9.2 and 10.4 / 8.7; the large launches
 * (gate|up, down) within 1 us either way. */
int valu_parts(int units)
{
    const int forced = g_valu_parts.load();
    if (forced == 1 || forced == 2) return forced;
    (void)units;
    return 2;
}

/* What a launch does with each tile's final rows besides storing them. */
struct Epilogue {
    const float *const *add = nullptr; /* per tensor (entries may be null): y += add */
    const int *ldadd = nullptr;        /* per tensor: 0 = one vector for all positions */
    int *argmax = nullptr;             /* one tensor, batch 1: greedy argmax of y here */
    bool swiglu = false;               /* tensors (gate, up): out[0] = up * silu(gate) */
    const float *norm_w = nullptr;     /* row-major launches only: RMSNorm of the input fused in */
    float norm_eps = 0.0f;
};

/* Prefill launches (9..32 positions): a workgroup takes QMV_PF_TILES tiles
 * and a range of K-units (units per split). Measured on MI355X at M = 32
 * (us per launch, cold): rows of fewer than 32 units take one unit per split
 * in at most 20 tile groups (Qwen2.5-7B q|k|v, 18 groups: 19.7 against 20.9
 * at two; o 18.9 against 20.0; Qwen2.5-1.5B q|k|v 14.6 against 15.4, o 13.9
 * against 15.1), five in 100 groups or more (7B gate|up, 148 groups: 48.8
 * against 58.2 at three and 61.5 at four) and two in between (1.5B gate|up,
 * 70 groups: 19.25 against 21.0 at one); long rows take two in at most 8
 * tile groups (1.5B down 1536 x 8960: 23.0 against 24.7 at three) and five
 * beyond (7B down, 14 groups: 52.7 against 57.3 at three). More splits keep
 * more CUs busy until their partials cost more than they spread.
 * units_per_wave, when forced, sets the units per split instead. */
Plan plan_prefill(long long groups, int units)
{
    const int force_u = g_force_u.load();
    int ups = force_u > 0                ? force_u
              : units >= 32              ? (groups <= 8 ? 2 : 5)
              : groups >= 100            ? 5
              : groups <= 20             ? 1
                                         : 2;
    if (ups > units) ups = units;
    Plan p;
    p.units_per_wave = ups;
    p.waves = QMV_PF_TILES;
    p.units_per_split = ups;
    p.splits = (units + ups - 1) / ups;
    return p;
}

/* One launch over `count` tensors sharing the input, for positions
 * [b0, b0 + batch) of the caller's batch (the caller's pointers are offset
 * here), planned but not enqueued: the parameters, the grid and the workspace
 * it needs. The workspace pointers are filled in by whoever owns the memory
 * (a per-stream workspace, or the fixed device scratch of the no-allocation
 * entry point). */
struct ChunkPlan {
    qmv::MatvecParams p;
    qmv::RowdotParams rp;                  /* row-major launch (rowdot): its parameters */
    bool rowdot = false;                   /* rowgroup_q4k_kernel */
    int rd_rows = 0, rd_seg = 0, rd_epi = 0; /* rows per segment, lanes per row segment, epilogue */
    bool rd_norm = false;                    /* the fused RMSNorm of the input */
    bool prefill = false, paired = false;
    int mt = 1, grid = 0, waves = 0, fmt = 0;
    size_t partials = 0, counters = 0;     /* floats / words of split-K workspace */
    size_t pair_vals = 0, pair_count = 0;  /* offsets of the SwiGLU tile-pair region */
    size_t argmax_tiles = 0;               /* fused argmax candidate slots needed (0: none) */
};

/* The Q6_K part of plan_rowdot (tensors checked there): rowloop_q6k_kernel,
 * one row per wave (SwiGLU: a gate row and its up row). */
bool plan_rowdot_q6k(QmvDeviceTensor *const *ts, int count, const float *d_in, int b0, float *const *d_out,
                     const Epilogue &epi, ChunkPlan *cp)
{
    const QmvDeviceTensor *t0 = ts[0];
    if (epi.norm_w) return false;
    if (epi.swiglu && (count != 2 || ts[1]->rows != t0->rows)) return false; /* rejected by the tiled plan */
    if (epi.argmax && (count != 1 || b0 != 0)) return false;
    const int sb = t0->blocks_per_row;
    if (sb <= kRowdotSharedSb || sb > kRowdotMaxSb) return false;
    qmv::RowdotParams &rp = cp->rp;
    memset(&rp, 0, sizeof rp);
    rp.njobs = count;
    rp.x = d_in + (size_t)b0 * t0->cols;
    rp.sb = sb;
    long long total = 0;
    for (int i = 0; i < count; ++i) {
        qmv::RowdotJob &j = rp.job[i];
        j.w = ts[i]->rowmajor;
        j.y = d_out[i] + (size_t)b0 * ts[i]->rows;
        j.rows = ts[i]->rows;
        j.wg_begin = (int)total;
        if (epi.add && epi.add[i]) j.add = epi.add[i] + (size_t)b0 * epi.ldadd[i];
        if (!epi.swiglu || i == 0) total += ts[i]->rows; /* SwiGLU: each wave takes a gate row and its up row */
    }
    if (total > INT_MAX) return false;
    rp.groups = (int)total;
    const int waves = (int)std::min<long long>(epi.swiglu ? 8 : 16, (total + kRowloopQ6Groups - 1) / kRowloopQ6Groups);
    memset(&cp->p, 0, sizeof cp->p);
    cp->rowdot = true;
    cp->rd_rows = 1;
    cp->rd_seg = 64;
    cp->rd_epi = epi.swiglu ? QMV_ROWDOT_SWIGLU : epi.argmax ? QMV_ROWDOT_ARGMAX : QMV_ROWDOT_STORE;
    cp->rd_norm = false;
    cp->prefill = cp->paired = false;
    cp->mt = 1;
    cp->grid = (int)((total + waves - 1) / waves);
    cp->waves = waves;
    cp->fmt = QMV_FMT_Q6_K;
    cp->partials = cp->counters = 0;
    cp->pair_vals = cp->pair_count = 0;
    /* Fused argmax candidates: one per workgroup. */
    cp->argmax_tiles = epi.argmax ? (size_t)cp->grid : 0;
    if (epi.argmax) {
        rp.argmax_result = epi.argmax;
        rp.argmax_tiles = cp->grid;
    }
    return true;
}

/* A single-position launch on a row-major kernel: every tensor keeps a
 * row-major copy and has the format of the first. Q4_K: rows fit 8 waves of
 * 16 super-blocks (one wave's segment in launches of more than
 * kRowdotMaxUnits pairs), and the epilogue is at most an added vector,
 * SwiGLU, the fused argmax or the fused norm. Q6_K (rows of 17 to 128
 * super-blocks): an added vector, SwiGLU or the fused argmax. */
bool plan_rowdot(QmvDeviceTensor *const *ts, int count, const float *d_in, int b0, float *const *d_out,
                 const Epilogue &epi, ChunkPlan *cp)
{
    if (g_rowdot.load() == 0 || count > QMV_MAX_JOBS) return false;
    /* A forced tiled plan (qmv_set_launch_tuning) applies to every launch. */
    if (g_target_waves.load() > 0 || g_force_u.load() > 0 || g_force_w.load() > 0) return false;
    const QmvDeviceTensor *t0 = ts[0];
    long long units = 0;
    for (int i = 0; i < count; ++i) {
        if (ts[i]->rowmajor == nullptr || ts[i]->cols != t0->cols || ts[i]->geo.format != t0->geo.format)
            return false;
        units += tiled_units(ts[i]->rows, ts[i]->blocks_per_row);
    }
    if (t0->geo.format == QMV_FMT_Q6_K) return plan_rowdot_q6k(ts, count, d_in, b0, d_out, epi, cp);
    /* Large launches: rows of at most kRowdotSharedSb super-blocks, and no
     * fused argmax (a candidate per 16-row workgroup publishes four times as
     * often as the tiled kernel's 64-row tiles: 151936 x 3584 Q4_K took 98 us
     * with the argmax against 69 tiled, 56 against 59 without it). */
    const bool large = units > kRowdotMaxUnits;
    if (large && (t0->blocks_per_row > kRowdotSharedSb || epi.argmax)) return false;
    if (epi.swiglu && (count != 2 || ts[1]->rows != t0->rows)) return false; /* rejected by the tiled plan */
    if (epi.argmax && (count != 1 || b0 != 0)) return false;
    const int sb = t0->blocks_per_row;
    if (sb > kRowdotMaxSb) return false;
    /* The fused norm needs the shared mode (every workgroup holds the whole
     * vector) and is not combined with the argmax. Large launches keep the
     * norm as a launch of its own: the fused kernel holds 64 more registers
     * per lane (the staged norm weights and the raw activations), so the
     * Qwen2.5-7B gate|up SwiGLU drops to two waves per SIMD and took 21.2 us
     * against 16.0 + 2.4 for the two launches (an LDS pass that scaled the
     * staged activations in place kept the registers but took 18.9 us). The
     * q|k|v launch gains: 5.8 us fused against 4.6 + 2.4. */
    if (epi.norm_w && (sb > kRowdotSharedSb || epi.argmax || large)) return false;
    /* Rows of at most 16 super-blocks: a segment of 16, 32 or 64 lanes per
     * row, QMV_ROWGROUP_WAVES waves sharing the activations; longer rows span
     * ceil(sb / 16) waves. */
    const int seg = sb <= 4 ? 16 : sb <= 8 ? 32 : 64;
    const bool split = sb > 16;
    const int waves = split ? (4 * sb + 63) / 64 : QMV_ROWGROUP_WAVES;
    const int want = large ? (epi.swiglu ? kRowdotRowsLargeSwiglu : kRowdotRowsLarge) : g_rowdot_rows.load();
    const int R = seg < 64 ? 2 : want == 1 || want == 4 ? want : 2;
    const int wg_rows = split ? R : QMV_ROWGROUP_WAVES * R * (64 / seg);
    qmv::RowdotParams &rp = cp->rp;
    memset(&rp, 0, sizeof rp);
    rp.njobs = count;
    rp.x = d_in + (size_t)b0 * t0->cols;
    rp.sb = sb;
    rp.norm_w = epi.norm_w;
    rp.norm_eps = epi.norm_eps;
    long long wg = 0;
    for (int i = 0; i < count; ++i) {
        qmv::RowdotJob &j = rp.job[i];
        j.w = ts[i]->rowmajor;
        j.y = d_out[i] + (size_t)b0 * ts[i]->rows;
        j.rows = ts[i]->rows;
        j.wg_begin = (int)wg;
        if (epi.add && epi.add[i]) j.add = epi.add[i] + (size_t)b0 * epi.ldadd[i];
        if (!epi.swiglu || i == 0) wg += (ts[i]->rows + wg_rows - 1) / wg_rows; /* SwiGLU: both jobs in each workgroup */
    }
    /* Fused argmax candidates: one per workgroup. */
    const long long cand = wg;
    if (cand > INT_MAX) return false;
    memset(&cp->p, 0, sizeof cp->p);
    cp->rowdot = true;
    cp->rd_rows = R;
    cp->rd_seg = seg;
    cp->rd_epi = epi.swiglu ? QMV_ROWDOT_SWIGLU : epi.argmax ? QMV_ROWDOT_ARGMAX : QMV_ROWDOT_STORE;
    cp->rd_norm = epi.norm_w != nullptr;
    if (epi.argmax) {
        rp.argmax_result = epi.argmax;
        rp.argmax_tiles = (int)cand;
    }
    cp->prefill = cp->paired = false;
    cp->mt = 1;
    cp->grid = (int)wg;
    cp->waves = waves;
    cp->fmt = t0->geo.format;
    cp->partials = cp->counters = 0;
    cp->pair_vals = cp->pair_count = 0;
    cp->argmax_tiles = epi.argmax ? (size_t)cand : 0;
    return true;
}

int plan_chunk(QmvDeviceTensor *const *ts, int count, const float *d_in, int b0, int batch, float *const *d_out,
               const Epilogue &epi, ChunkPlan *cp)
{
    const QmvDeviceTensor *t0 = ts[0];
    cp->rowdot = false;
    if (batch == 1 && plan_rowdot(ts, count, d_in, b0, d_out, epi, cp)) return 1;
    if (epi.norm_w) {
        set_error("internal: a fused RMSNorm reached the tiled planner");
        return 0;
    }
    const bool mfma = use_matrix_cores(t0->geo.format, batch);
    /* Up to 8 positions: the matvec kernels for exactly `batch` positions.
     * More: the prefill kernel, 16 or 32 position rows with the batch in the
     * first. */
    const bool prefill = batch > QMV_VALU_MAX_POSITIONS;
    if (prefill && !use_prefill(t0->geo.format, batch)) {
        set_error("more than 8 positions per launch need the matrix-core path");
        return 0;
    }
    const int mt = !prefill ? batch : batch <= 16 ? 16 : QMV_MFMA_MAX_POSITIONS;
    long long total_tiles = 0, total_groups = 0;
    for (int i = 0; i < count; ++i) {
        total_tiles += ts[i]->tiles;
        total_groups += (ts[i]->tiles + QMV_PF_TILES - 1) / QMV_PF_TILES;
    }
    const int parts = prefill ? 1 : mfma ? mfma_parts(t0->units, total_tiles) : batch >= 2 ? valu_parts(t0->units) : 1;
    /* Single-position launches of many units (the vocabulary projection:
     * 33236) run several rounds of resident waves; five waves per workgroup
     * (three splits of 14 units instead of four) measured 80.9 us against
     * 84.8-86.8 at four for 151936 x 3584 Q6_K, while four stays best for
     * the decode-step launches (o 3584 x 3584: 6.0 against 6.6 us). */
    /* Single-position launches of 2049..16384 units over rows of fewer than
     * 32 units (Qwen2.5-7B gate|up: 592 tiles x 14 units) take two waves per
     * workgroup, so a tile's 14 units fill 14 wave slots (7 splits) instead
     * of 16 (four splits of 4, 4, 4 and 2): the launch then needs 8288 slots
     * where 8192 fit at once, not 9472. gate|up 18.1-18.2 us against
     * 18.65-19.05 at four waves (17.97 at eight, 18.2 at three), and the fused
     * SwiGLU, paired in workgroups of 2 x 2 waves, 18.1 against 18.3-18.5. */
    /* Small single-position launches over rows of at most 8 units take each
     * tile in one workgroup, with no split-K tail: Q8_0 896 x 896 (7 units)
     * 4.80 us against 5.18-5.24 us in two splits. Longer rows keep the
     * splits (Q6_K 896 x 4864, 19 units: 6.1 us at 4 waves, 7.4 at 7). */
    /* Matrix-core launches over rows of fewer than 32 units take the waves
     * per workgroup that leave no wave idle in a tile's last split: three if
     * three divides the tile's work items, else four if four does, else two
     * if two does, else four. Measured at M = 8 (us per launch):
     * Qwen2.5-1.5B q|k|v (24 items) 7.47 at three against 7.86 at four and
     * 7.99 at two, o (24) 7.18 against 7.55, gate|up (12) 12.24 against
     * 12.7-13.1 (12.2-12.3 at two); Qwen2.5-7B q|k|v (28) 9.9 at four
     * against 10.8 at three and 10.2 at two, gate|up (14) 32.8-33.0 at two
     * against 34.1 at four. Long rows (32 units or more) on the matrix
     * cores take three waves for Q6_K (7B down, 74 items: 29.6 us against
     * 30.4 at four or two) and four for the other formats (1.5B Q4_K down,
     * 35 items: 10.0 against 11.5 at three). */
    const int items = t0->units * parts;
    const int long_batch_waves = mfma && t0->geo.format == QMV_FMT_Q6_K ? 3 : 4;
    const int mfma_waves = items % 3 == 0 ? 3 : items % 4 == 0 ? 4 : items % 2 == 0 ? 2 : 4;
    const bool one_split = batch == 1 && t0->units <= QMV_MAX_WAVES && total_tiles * t0->units <= 2048;
    const int short_waves = one_split                                       ? t0->units
                            : batch == 1 && total_tiles * t0->units > 16384 ? 5
                            : mfma                                          ? mfma_waves
                            : batch == 1 && total_tiles * t0->units > 2048  ? 2
                                                                            : 4;
    const Plan plan = prefill ? plan_prefill(total_groups, t0->units)
                              : plan_for(total_tiles, t0->units * parts, batch == 1 ? 6 : long_batch_waves, short_waves,
                                         mfma || parts > 1 ? 1 : 8);

    qmv::MatvecParams &p = cp->p;
    memset(&p, 0, sizeof p);
    p.njobs = count;
    p.x = d_in + (size_t)b0 * t0->cols;
    p.ldx = t0->cols;
    p.cols = t0->cols;
    p.units = t0->units;
    p.units_per_wave = plan.units_per_wave;
    p.parts = parts;
    if ((mfma || parts > 1) && !prefill && plan.units_per_wave != 1) {
        set_error("launch planned with more than one work item per wave");
        return 0;
    }
    p.positions = batch;
    /* Fused SwiGLU at M = 1 with one unit per wave: one workgroup per
     * (tile, split) of both projections (finish_paired), when the two halves
     * fit a workgroup. */
    const bool paired = epi.swiglu && count == 2 && batch == 1 && !prefill && !mfma &&
                        plan.units_per_wave == 1 && 2 * plan.waves <= QMV_MAX_WAVES &&
                        ts[0]->rows == ts[1]->rows && g_paired_swiglu.load() != 0;
    size_t partials = 0, counters = 0;
    long long wg = 0;
    for (int i = 0; i < count; ++i) {
        qmv::MatvecJob &j = p.job[i];
        j.w = ts[i]->data;
        j.y = d_out[i] + (size_t)b0 * ts[i]->rows;
        j.rows = ts[i]->rows;
        j.ldy = ts[i]->rows;
        j.tiles = ts[i]->tiles;
        j.splits = plan.splits;
        j.units_per_split = plan.units_per_split;
        j.wg_begin = (int)wg;
        j.partial_offset = (int)partials;
        j.counter_offset = (int)counters;
        if (epi.add && epi.add[i]) {
            j.add = epi.add[i] + (size_t)b0 * epi.ldadd[i];
            j.ldadd = epi.ldadd[i];
        }
        if (paired) {
            if (i == 0) { /* two sums per split, one count per tile, in job 0's regions */
                if (plan.splits > 1) {
                    partials += (size_t)ts[0]->tiles * plan.splits * 2 * 64;
                    counters += (size_t)ts[0]->tiles * QMV_COUNTER_STRIDE;
                }
                wg += (long long)ts[0]->tiles * plan.splits;
            }
            continue;
        }
        if (plan.splits > 1) {
            partials += (size_t)ts[i]->tiles * plan.splits * mt * 64;
            counters += (size_t)ts[i]->tiles * QMV_COUNTER_STRIDE;
        }
        wg += (long long)(prefill ? (ts[i]->tiles + QMV_PF_TILES - 1) / QMV_PF_TILES : ts[i]->tiles) * plan.splits;
    }
    if (paired) p.pair_waves = plan.waves;
    /* Fused SwiGLU otherwise: both projections' final tiles, then one count
     * per tile pair, after the split-K partials and counters. */
    cp->pair_vals = partials;
    cp->pair_count = counters;
    if (epi.swiglu && !paired) {
        if (count != 2 || ts[0]->rows != ts[1]->rows) {
            set_error("fused SwiGLU takes two tensors (gate, up) with equal rows");
            return 0;
        }
        partials += (size_t)2 * t0->tiles * mt * 64;
        counters += (size_t)t0->tiles * QMV_COUNTER_STRIDE;
        p.swiglu = 1;
    }
    if (wg > INT_MAX || partials > (size_t)INT_MAX || counters > (size_t)INT_MAX) {
        set_error("launch too large");
        return 0;
    }
    p.matrix_cores = mfma;
    cp->argmax_tiles = 0;
    if (epi.argmax) {
        if (count != 1 || batch != 1 || b0 != 0 || epi.swiglu) {
            set_error("fused argmax takes one tensor and one position");
            return 0;
        }
        p.argmax_result = epi.argmax;
        p.argmax_tiles = t0->tiles;
        cp->argmax_tiles = (size_t)t0->tiles;
    }
    cp->prefill = prefill;
    cp->paired = paired;
    cp->mt = mt;
    cp->grid = (int)wg;
    cp->waves = paired ? 2 * plan.waves : plan.waves;
    cp->fmt = t0->geo.format;
    cp->partials = partials ? partials + QMV_PARTIAL_PAD : 0; /* padding past the last partial */
    cp->counters = counters;
    return 1;
}

/* Point the plan at its split-K workspace: partials[cp.partials] floats and
 * counters[cp.counters] words (zero between launches). */
void bind_workspace(ChunkPlan &cp, float *partials, unsigned *counters)
{
    cp.p.partials = partials;
    cp.p.counters = counters;
    if (cp.p.swiglu) {
        cp.p.pair_vals = partials + cp.pair_vals;
        cp.p.pair_count = counters + cp.pair_count;
    }
}

int enqueue_chunk(const ChunkPlan &cp, hipStream_t stream)
{
    if (cp.rowdot && cp.fmt == QMV_FMT_Q6_K)
        HIP_TRY(qmv::launch_rowloop_q6k(cp.rp, cp.rd_epi, cp.grid, cp.waves, stream));
    else if (cp.rowdot)
        HIP_TRY(qmv::launch_rowgroup(cp.rp, cp.rd_rows, cp.rd_seg, cp.rd_epi, cp.grid, cp.waves, stream, cp.rd_norm));
    else if (cp.prefill)
        HIP_TRY(qmv::launch_prefill(cp.fmt, cp.p, cp.mt, cp.grid, stream));
    else
        HIP_TRY(qmv::launch_matvec(cp.fmt, cp.p, cp.mt, cp.grid, cp.waves, stream));
    return 1;
}

/* Plan a launch and enqueue it on the stream's own workspace (grown here if
 * needed, outside graph capture only). */
int launch_chunk(QmvDeviceTensor *const *ts, int count, const float *d_in, int b0, int batch,
                 float *const *d_out, hipStream_t stream, Workspace &ws, const Epilogue &epi)
{
    ChunkPlan cp;
    if (!plan_chunk(ts, count, d_in, b0, batch, d_out, epi, &cp)) return 0;
    std::lock_guard<std::mutex> lock(ws.mu);
    if (!workspace_reserve(ws, stream, cp.partials, cp.counters)) return 0;
    bind_workspace(cp, ws.partials, ws.counters);
    if (cp.argmax_tiles) {
        if (!workspace_fused_argmax(ws, stream, cp.argmax_tiles)) return 0;
        cp.p.argmax_cand = cp.rp.argmax_cand = ws.fused_cand;
        cp.p.argmax_count = cp.rp.argmax_count = ws.fused_count;
    }
    return enqueue_chunk(cp, stream);
}

/* Positions per launch for the remaining `batch` positions of a call: up to
 * 32 where the prefill kernel takes them, else 8. */
int chunk_positions(int fmt, int batch)
{
    const int wide = batch < QMV_MFMA_MAX_POSITIONS ? batch : QMV_MFMA_MAX_POSITIONS;
    return use_prefill(fmt, wide) ? QMV_MFMA_MAX_POSITIONS : QMV_VALU_MAX_POSITIONS;
}

/* Positions of the launch that starts at position b0 of a `batch`-position
 * call. The chunk size is chosen again for every launch from the positions
 * left, so a tail that the prefill kernel does not take (for instance below
 * a raised matrix-core threshold) runs in launches of at most 8. */
int next_chunk(int fmt, int batch, int b0)
{
    const int left = batch - b0;
    const int chunk = chunk_positions(fmt, left);
    return left < chunk ? left : chunk;
}

/* Enqueue a batch of any size as launches of up to chunk_positions(). */
int launch_group(QmvDeviceTensor *const *ts, int count, const float *d_in, int batch, float *const *d_out,
                 hipStream_t stream, Workspace &ws, const Epilogue &epi = Epilogue())
{
    for (int b0 = 0; b0 < batch;) {
        const int nb = next_chunk(ts[0]->geo.format, batch, b0);
        if (!launch_chunk(ts, count, d_in, b0, nb, d_out, stream, ws, epi)) return 0;
        b0 += nb;
    }
    return 1;
}

int host_matmul(const QmvTensorView *m, const float *in, int in_count, int batch, float *out, int out_count)
{
    Shape s;
    if (!matvec_args_ok(m, in, in_count, out, out_count, batch, &s)) return 0;
    CtxLease lease;
    HostCtx *c = lease.c;
    if (!c) return 0;
    std::shared_ptr<QmvDeviceTensor> t = cached_tensor(m, s, c);
    if (!t) return 0;
    const size_t nin = (size_t)batch * (size_t)in_count, nout = (size_t)batch * (size_t)out_count;
    if (!grow_pinned(&c->h_in, &c->h_in_cap, nin) || !grow_pinned(&c->h_out, &c->h_out_cap, nout) ||
        !grow_device(&c->d_in, &c->d_in_cap, nin))
        return 0;
    memcpy(c->h_in, in, nin * sizeof(float));
    /* The input reaches HBM by an asynchronous copy, or for 32 KB and more by
     * a copy kernel reading the pinned buffer (faster there: 75 KB in
     * ~5 us less on MI355X); the kernels write the output straight into the
     * pinned buffer, which saves the device-to-host copy (gate 18944 rows:
     * 36 -> 28 us per call). */
    if (nin * sizeof(float) >= (32u << 10)) {
        float *hin = nullptr;
        HIP_TRY(hipHostGetDevicePointer((void **)&hin, c->h_in, 0));
        HIP_TRY(qmv::launch_copy(hin, c->d_in, nin, c->stream));
    } else {
        HIP_TRY(hipMemcpyAsync(c->d_in, c->h_in, nin * sizeof(float), hipMemcpyHostToDevice, c->stream));
    }
    QmvDeviceTensor *tp = t.get();
    float *hout = nullptr;
    HIP_TRY(hipHostGetDevicePointer((void **)&hout, c->h_out, 0));
    if (!launch_group(&tp, 1, c->d_in, batch, &hout, c->stream, *c->ws)) return 0;
    HIP_TRY(hipStreamSynchronize(c->stream));
    lease.done = true;
    int armed = g_fail_next.load();
    while (armed > 0 && !g_fail_next.compare_exchange_weak(armed, armed - 1)) {
    }
    if (armed > 0) {
        set_error("failure injected by qmv_debug_fail_next_calls");
        return 0;
    }
    memcpy(out, c->h_out, nout * sizeof(float));
    return 1;
}

} // namespace

/* ---- C ABI ------------------------------------------------------------------------ */

QMV_API int qmv_tensor_matvec_f32(const QmvTensorView *matrix, const float *input, int input_count,
                                  float *output, int output_count)
{
    return host_matmul(matrix, input, input_count, 1, output, output_count);
}

QMV_API int qmv_tensor_matmul_f32(const QmvTensorView *matrix, const float *inputs, int input_count,
                                  int batch_count, float *outputs, int output_count)
{
    return host_matmul(matrix, inputs, input_count, batch_count, outputs, output_count);
}

QMV_API int qmv_register_tensor(const QmvTensorView *matrix)
{
    Shape s;
    if (!view_layout_ok(matrix, &s)) return 0;
    CtxLease lease;
    if (!lease.c) return 0;
    return cached_tensor(matrix, s, lease.c) ? 1 : 0;
}

/* Pre-size everything a host-pointer call on this tensor needs, for batches
 * of 1..max_batch positions, in every context of the device's pool: the
 * upload, the input and output staging, and the split-K workspace of every
 * launch such a call makes (launches carry at most QMV_MFMA_MAX_POSITIONS
 * positions, and a launch's needs depend only on its own position count).
 * The pool gets a context if it has none, and is closed. */
QMV_API int qmv_reserve_calls(const QmvTensorView *matrix, int max_batch)
{
    Shape s;
    if (!view_layout_ok(matrix, &s)) return 0;
    if (max_batch <= 0 || (size_t)max_batch > SIZE_MAX / 4 / (size_t)(s.cols > s.rows ? s.cols : s.rows)) {
        set_error("max_batch must be positive and its staging addressable");
        return 0;
    }
    std::shared_ptr<QmvDeviceTensor> t;
    {
        CtxLease lease;
        if (!lease.c) return 0;
        t = cached_tensor(matrix, s, lease.c);
        if (!t) return 0;
    }
    CtxSizes need;
    need.nin = (size_t)max_batch * (size_t)s.cols;
    need.nout = (size_t)max_batch * (size_t)s.rows;
    QmvDeviceTensor *tp = t.get();
    float dummy = 0.0f; /* planning only: no launch is made, nothing is dereferenced */
    float *out = &dummy;
    const int widest = max_batch < QMV_MFMA_MAX_POSITIONS ? max_batch : QMV_MFMA_MAX_POSITIONS;
    for (int nb = 1; nb <= widest; ++nb) {
        if (nb > QMV_VALU_MAX_POSITIONS && !use_prefill(tp->geo.format, nb)) continue;
        ChunkPlan cp;
        if (!plan_chunk(&tp, 1, &dummy, 0, nb, &out, Epilogue(), &cp)) return 0;
        if (cp.partials > need.partials) need.partials = cp.partials;
        if (cp.counters > need.counters) need.counters = cp.counters;
    }
    return pool_reserve(need, 1);
}

/* Give the device's pool at least `count` contexts, each sized like the
 * reservations so far (and grown by later ones), and close it. */
QMV_API int qmv_reserve_contexts(int count)
{
    if (count <= 0 || count > kMaxContexts) {
        set_error("context count must be in 1..%d", kMaxContexts);
        return 0;
    }
    return pool_reserve(CtxSizes(), count);
}

QMV_API unsigned long long qmv_allocation_count(void)
{
    return g_allocations.load();
}

QMV_API int qmv_release_tensor(const unsigned char *data)
{
    std::lock_guard<std::mutex> lock(g_cache_mu);
    int n = 0;
    for (auto it = g_cache.begin(); it != g_cache.end();) {
        if (std::get<1>(it->first) == data) {
            it = g_cache.erase(it);
            ++n;
        } else {
            ++it;
        }
    }
    return n;
}

QMV_API void qmv_release_all(void)
{
    std::lock_guard<std::mutex> lock(g_cache_mu);
    g_cache.clear();
}

QMV_API int qmv_dequantize_rows_f32(const QmvTensorView *matrix, int first_row, int row_count, float *output)
{
    Shape s;
    if (output == nullptr || !view_layout_ok(matrix, &s)) {
        if (output == nullptr) set_error("null output");
        return 0;
    }
    if (first_row < 0 || row_count <= 0 || (long long)first_row + row_count > s.rows) {
        set_error("row range outside the tensor");
        return 0;
    }
    CtxLease lease;
    HostCtx *c = lease.c;
    if (!c) return 0;
    std::shared_ptr<QmvDeviceTensor> t = cached_tensor(matrix, s, c);
    if (!t) return 0;
    const size_t n = (size_t)row_count * (size_t)s.cols;
    if (!grow_device(&c->d_out, &c->d_out_cap, n)) return 0;
    HIP_TRY(qmv::launch_dequant(t->geo.format, t->data, c->d_out, t->rows, t->cols, t->units, first_row, row_count,
                                c->stream));
    HIP_TRY(hipMemcpyAsync(output, c->d_out, n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    lease.done = true;
    return 1;
}

/* Address ranges of device buffers, for the no-overlap rules. */
static bool overlap(const void *a, size_t abytes, const void *b, size_t bbytes)
{
    const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
    return a0 < b0 + bbytes && b0 < a0 + abytes;
}

QMV_API int qmv_device_rms_norm_f32(const float *d_input, const float *d_weight, int length, int batch_count,
                                    float epsilon, float *d_output, void *stream)
{
    /* src/tensor.cpp:116-122: null pointers, length <= 0 and epsilon <= 0
     * fail (so a NaN epsilon is accepted, as there). */
    if (d_input == nullptr || d_weight == nullptr || d_output == nullptr || length <= 0 || batch_count <= 0 ||
        epsilon <= 0) {
        set_error("invalid RMSNorm arguments");
        return 0;
    }
    const size_t bytes = (size_t)batch_count * length * sizeof(float);
    if ((d_output != d_input && overlap(d_output, bytes, d_input, bytes)) ||
        overlap(d_output, bytes, d_weight, (size_t)length * sizeof(float))) {
        set_error("RMSNorm output overlaps the weight or part of the input");
        return 0;
    }
    HIP_TRY(hipSetDevice(g_device.load()));
    HIP_TRY(qmv::launch_rms_norm(d_input, d_weight, length, batch_count, epsilon, d_output, (hipStream_t)stream));
    return 1;
}

QMV_API int qmv_device_greedy_argmax_f32(const float *d_logits, int vocab_size, int *d_result, void *stream)
{
    if (d_logits == nullptr || d_result == nullptr || vocab_size <= 0) {
        set_error("invalid argmax arguments");
        return 0;
    }
    int dev = g_device.load();
    HIP_TRY(hipSetDevice(dev));
    hipStream_t s = (hipStream_t)stream;
    Workspace &ws = workspace_for(dev, s);
    std::lock_guard<std::mutex> lock(ws.mu);
    if (!workspace_argmax(ws)) return 0;
    int blocks = (vocab_size + 4095) / 4096;
    blocks = blocks < 1 ? 1 : blocks > kArgBlocks ? kArgBlocks : blocks;
    HIP_TRY(qmv::launch_argmax(d_logits, vocab_size, ws.arg_val, ws.arg_idx, ws.arg_bad, blocks, d_result, s));
    return 1;
}

QMV_API int qmv_greedy_sample_f32(const float *logits, int vocab_size, int *token_id)
{
    if (token_id) *token_id = -1;
    if (logits == nullptr || token_id == nullptr || vocab_size <= 0) {
        set_error("invalid greedy sampler arguments");
        return 0;
    }
    CtxLease lease;
    HostCtx *c = lease.c;
    if (!c) return 0;
    const size_t n = (size_t)vocab_size;
    if (!grow_device(&c->d_in, &c->d_in_cap, n) || !grow_device(&c->d_out, &c->d_out_cap, 2) ||
        !grow_pinned(&c->h_out, &c->h_out_cap, 2))
        return 0;
    HIP_TRY(hipMemcpyAsync(c->d_in, logits, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
    int *d_res = (int *)c->d_out;
    if (!qmv_device_greedy_argmax_f32(c->d_in, vocab_size, d_res, c->stream)) return 0;
    HIP_TRY(hipMemcpyAsync(c->h_out, d_res, 2 * sizeof(int), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    lease.done = true;
    int res[2];
    memcpy(res, c->h_out, sizeof res);
    if (res[1] != 1) {
        set_error("greedy sampler received a non-finite logit");
        return 0;
    }
    *token_id = res[0];
    return 1;
}

QMV_API int qmv_device_tensor_create(const QmvTensorView *matrix, qmv_device_tensor *out_tensor)
{
    if (out_tensor == nullptr) {
        set_error("null output handle");
        return 0;
    }
    *out_tensor = nullptr;
    Shape s;
    if (!view_layout_ok(matrix, &s)) return 0;
    CtxLease lease;
    HostCtx *c = lease.c;
    if (!c) return 0;
    QmvDeviceTensor *t = nullptr;
    if (!tensor_upload(matrix, s, c->device, c->stream, &t)) return 0;
    lease.done = true; /* the upload synchronised its stream */
    *out_tensor = t;
    return 1;
}

QMV_API void qmv_device_tensor_destroy(qmv_device_tensor tensor)
{
    tensor_free(tensor);
}

QMV_API int qmv_device_tensor_info(qmv_device_tensor t, int *rows, int *columns, uint32_t *ggml_type,
                                   uint64_t *packed_bytes, uint64_t *device_bytes)
{
    if (t == nullptr) {
        set_error("null tensor");
        return 0;
    }
    if (rows) *rows = t->rows;
    if (columns) *columns = t->cols;
    if (ggml_type) *ggml_type = t->ggml_type;
    if (packed_bytes) *packed_bytes = t->packed_bytes;
    if (device_bytes) *device_bytes = t->device_bytes;
    return 1;
}

/* Shared checks of the grouped device matvec: same type, column count and
 * device; outputs overlap neither the input nor each other (every workgroup
 * reads the whole input while others write their rows). */
static int group_args_ok(const qmv_device_tensor *tensors, int count, const float *d_inputs, int batch_count,
                         float *const *d_outputs)
{
    if (tensors == nullptr || d_inputs == nullptr || d_outputs == nullptr || count <= 0 ||
        count > QMV_MAX_GROUP || batch_count <= 0 || batch_count > QMV_MAX_BATCH) {
        set_error("invalid group matvec arguments");
        return 0;
    }
    for (int i = 0; i < count; ++i) {
        if (tensors[i] == nullptr || d_outputs[i] == nullptr) {
            set_error("null tensor or output in group");
            return 0;
        }
        if (tensors[i]->ggml_type != tensors[0]->ggml_type || tensors[i]->cols != tensors[0]->cols ||
            tensors[i]->device != tensors[0]->device) {
            set_error("grouped tensors must share type, column count and device");
            return 0;
        }
    }
    const size_t in_bytes = (size_t)batch_count * tensors[0]->cols * sizeof(float);
    for (int i = 0; i < count; ++i) {
        const size_t out_bytes = (size_t)batch_count * tensors[i]->rows * sizeof(float);
        if (overlap(d_outputs[i], out_bytes, d_inputs, in_bytes)) {
            set_error("output overlaps the input");
            return 0;
        }
        for (int j = 0; j < i; ++j)
            if (overlap(d_outputs[i], out_bytes, d_outputs[j], (size_t)batch_count * tensors[j]->rows * 4)) {
                set_error("outputs overlap each other");
                return 0;
            }
    }
    return 1;
}

QMV_API int qmv_device_matvec_group_f32(const qmv_device_tensor *tensors, int count, const float *d_inputs,
                                        int batch_count, float *const *d_outputs, void *stream)
{
    if (!group_args_ok(tensors, count, d_inputs, batch_count, d_outputs)) return 0;
    HIP_TRY(hipSetDevice(tensors[0]->device));
    hipStream_t s = (hipStream_t)stream;
    Workspace &ws = workspace_for(tensors[0]->device, s);
    return launch_group(const_cast<QmvDeviceTensor *const *>(tensors), count, d_inputs, batch_count, d_outputs, s,
                        ws);
}

/* ---- no-allocation grouped matvec ----------------------------------------------
 * The split-K workspace of these launches is a fixed device array: counters
 * in its first QMV_NOALLOC_COUNTER_BYTES, partials in the rest. In host code
 * the name `scratch` is only a stand-in for the array; its device address
 * comes from hipGetSymbolAddress, once per device with that device current,
 * and only that address is passed to kernels. Every call on a device shares
 * its array: calls that overlap on one device race. */
static __device__ __align__(256) unsigned char scratch[QMV_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchDevices];

/* Device address of this device's scratch array (the device is current). */
int scratch_address(int device, void **out)
{
    if (device < 0 || device >= kScratchDevices) {
        set_error("device %d out of range for the no-allocation scratch", device);
        return 0;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device] == nullptr) {
        void *p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (p == nullptr) {
            set_error("hipGetSymbolAddress returned no address for the scratch array");
            return 0;
        }
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return 1;
}

} // namespace

QMV_API int qmv_device_matvec_group_noalloc_f32(const qmv_device_tensor *tensors, int count, const float *d_inputs,
                                                int batch_count, float *const *d_outputs, void *stream)
{
    if (!group_args_ok(tensors, count, d_inputs, batch_count, d_outputs)) return 0;
    const int dev = tensors[0]->device;
    HIP_TRY(hipSetDevice(dev));
    void *base = nullptr;
    if (!scratch_address(dev, &base)) return 0;
    unsigned *counters = (unsigned *)base;
    float *partials = (float *)((unsigned char *)base + QMV_NOALLOC_COUNTER_BYTES);
    const size_t counter_cap = QMV_NOALLOC_COUNTER_BYTES / sizeof(unsigned);
    const size_t partial_cap = (QMV_NOALLOC_SCRATCH_BYTES - QMV_NOALLOC_COUNTER_BYTES) / sizeof(float);
    QmvDeviceTensor *const *ts = const_cast<QmvDeviceTensor *const *>(tensors);
    const int fmt = ts[0]->geo.format;
    /* Every launch is planned and checked before the first is enqueued, so a
     * call that does not fit launches nothing. */
    for (int b0 = 0; b0 < batch_count;) {
        const int nb = next_chunk(fmt, batch_count, b0);
        ChunkPlan cp;
        if (!plan_chunk(ts, count, d_inputs, b0, nb, d_outputs, Epilogue(), &cp)) return 0;
        if (cp.partials > partial_cap || cp.counters > counter_cap) {
            set_error("launch needs %zu partial floats and %zu counters; the no-allocation scratch holds %zu and "
                      "%zu (use qmv_device_matvec_group_f32)",
                      cp.partials, cp.counters, partial_cap, counter_cap);
            return 0;
        }
        b0 += nb;
    }
    hipStream_t s = (hipStream_t)stream;
    for (int b0 = 0; b0 < batch_count;) {
        const int nb = next_chunk(fmt, batch_count, b0);
        ChunkPlan cp;
        if (!plan_chunk(ts, count, d_inputs, b0, nb, d_outputs, Epilogue(), &cp)) return 0;
        bind_workspace(cp, partials, counters);
        /* The counters must be zero when the launch starts. Completed
         * launches leave them zero; the fill (a kernel, not a memset node, so
         * the call can be captured) also covers an interrupted earlier one. */
        HIP_TRY(qmv::launch_fill_u32(counters, cp.counters, 0u, s));
        if (!enqueue_chunk(cp, s)) return 0;
        b0 += nb;
    }
    return 1;
}

QMV_API int qmv_device_matvec_f32(qmv_device_tensor tensor, const float *d_inputs, int batch_count,
                                  float *d_outputs, void *stream)
{
    return qmv_device_matvec_group_f32(&tensor, 1, d_inputs, batch_count, &d_outputs, stream);
}

/* The addend rules of qmv_device_matvec_add_group_f32 (include/qmv_hip.h). */
static int addend_args_ok(const qmv_device_tensor *tensors, int count, int batch_count,
                          const float *const *d_addends, const int *addend_strides, float *const *d_outputs)
{
    if (d_addends == nullptr || addend_strides == nullptr) {
        set_error("invalid addend arguments");
        return 0;
    }
    for (int i = 0; i < count; ++i) {
        if (d_addends[i] == nullptr) continue;
        const int n = tensors[i]->rows, ld = addend_strides[i];
        if (ld != 0 && ld < n) {
            set_error("addend stride must be 0 or at least the row count");
            return 0;
        }
        const size_t add_bytes = ((size_t)(batch_count - 1) * ld + n) * sizeof(float);
        const bool in_place = d_addends[i] == d_outputs[i] && ld == n;
        for (int j = 0; j < count; ++j) {
            if (j == i && in_place) continue;
            if (overlap(d_addends[i], add_bytes, d_outputs[j], (size_t)batch_count * tensors[j]->rows * 4)) {
                set_error("addend overlaps an output (only an addend that is its own output, stride = rows, may)");
                return 0;
            }
        }
    }
    return 1;
}

QMV_API int qmv_device_matvec_add_group_f32(const qmv_device_tensor *tensors, int count, const float *d_inputs,
                                            int batch_count, const float *const *d_addends,
                                            const int *addend_strides, float *const *d_outputs, void *stream)
{
    if (!group_args_ok(tensors, count, d_inputs, batch_count, d_outputs)) return 0;
    if (!addend_args_ok(tensors, count, batch_count, d_addends, addend_strides, d_outputs)) return 0;
    HIP_TRY(hipSetDevice(tensors[0]->device));
    hipStream_t s = (hipStream_t)stream;
    Workspace &ws = workspace_for(tensors[0]->device, s);
    Epilogue epi;
    epi.add = d_addends;
    epi.ldadd = addend_strides;
    return launch_group(const_cast<QmvDeviceTensor *const *>(tensors), count, d_inputs, batch_count, d_outputs, s,
                        ws, epi);
}

QMV_API int qmv_device_matvec_swiglu_f32(qmv_device_tensor gate, qmv_device_tensor up, const float *d_inputs,
                                         int batch_count, float *d_outputs, void *stream)
{
    if (gate == nullptr || up == nullptr) {
        set_error("invalid fused SwiGLU arguments");
        return 0;
    }
    if (!group_args_ok(&gate, 1, d_inputs, batch_count, &d_outputs)) return 0;
    if (up->ggml_type != gate->ggml_type || up->cols != gate->cols || up->rows != gate->rows ||
        up->device != gate->device) {
        set_error("gate and up must share type, shape and device");
        return 0;
    }
    HIP_TRY(hipSetDevice(gate->device));
    hipStream_t s = (hipStream_t)stream;
    Workspace &ws = workspace_for(gate->device, s);
    QmvDeviceTensor *const pair[2] = {gate, up};
    float *const outs[2] = {d_outputs, d_outputs}; /* only job 0's output is written */
    Epilogue epi;
    epi.swiglu = true;
    return launch_group(pair, 2, d_inputs, batch_count, outs, s, ws, epi);
}

/* RMSNorm of the input followed by a grouped launch. The norm runs inside
 * the row-major launch where that launch takes the call (one position, Q4_K
 * rows of at most 16 super-blocks: each workgroup holds the whole input);
 * otherwise a norm launch writes d_normed and the group reads it. */
static int norm_then_group(QmvDeviceTensor *const *ts, int count, const float *d_in, const float *d_w, float eps,
                           int batch, float *const *d_out, float *d_normed, hipStream_t s, Workspace &ws,
                           Epilogue epi)
{
    if (batch == 1) {
        epi.norm_w = d_w;
        epi.norm_eps = eps;
        ChunkPlan cp;
        if (plan_rowdot(ts, count, d_in, 0, d_out, epi, &cp)) return enqueue_chunk(cp, s);
        epi.norm_w = nullptr;
    }
    HIP_TRY(qmv::launch_rms_norm(d_in, d_w, ts[0]->cols, batch, eps, d_normed, s));
    return launch_group(ts, count, d_normed, batch, d_out, s, ws, epi);
}

/* The norm arguments of the fused entry points: those of
 * qmv_device_rms_norm_f32, and d_normed clear of the input, the weights and
 * every output. */
static int norm_args_ok(const float *d_input, const float *d_norm_weight, float epsilon, int cols, int batch_count,
                        float *d_normed, float *const *d_outputs, const int *out_rows, int nout)
{
    if (d_norm_weight == nullptr || d_normed == nullptr || epsilon <= 0) {
        set_error("invalid RMSNorm arguments");
        return 0;
    }
    const size_t bytes = (size_t)batch_count * cols * sizeof(float);
    if (overlap(d_normed, bytes, d_input, bytes) || overlap(d_normed, bytes, d_norm_weight, (size_t)cols * 4)) {
        set_error("d_normed overlaps the input or the norm weights");
        return 0;
    }
    for (int i = 0; i < nout; ++i)
        if (overlap(d_normed, bytes, d_outputs[i], (size_t)batch_count * out_rows[i] * 4)) {
            set_error("d_normed overlaps an output");
            return 0;
        }
    return 1;
}

QMV_API int qmv_device_rms_norm_matvec_add_group_f32(const qmv_device_tensor *tensors, int count,
                                                     const float *d_input, const float *d_norm_weight,
                                                     float epsilon, int batch_count, const float *const *d_addends,
                                                     const int *addend_strides, float *const *d_outputs,
                                                     float *d_normed, void *stream)
{
    if (!group_args_ok(tensors, count, d_input, batch_count, d_outputs)) return 0;
    if (d_addends != nullptr && !addend_args_ok(tensors, count, batch_count, d_addends, addend_strides, d_outputs))
        return 0;
    int rows[QMV_MAX_GROUP];
    for (int i = 0; i < count; ++i) rows[i] = tensors[i]->rows;
    if (!norm_args_ok(d_input, d_norm_weight, epsilon, tensors[0]->cols, batch_count, d_normed, d_outputs, rows,
                      count))
        return 0;
    HIP_TRY(hipSetDevice(tensors[0]->device));
    hipStream_t s = (hipStream_t)stream;
    Workspace &ws = workspace_for(tensors[0]->device, s);
    Epilogue epi;
    if (d_addends != nullptr) {
        epi.add = d_addends;
        epi.ldadd = addend_strides;
    }
    return norm_then_group(const_cast<QmvDeviceTensor *const *>(tensors), count, d_input, d_norm_weight, epsilon,
                           batch_count, d_outputs, d_normed, s, ws, epi);
}

QMV_API int qmv_device_rms_norm_matvec_swiglu_f32(qmv_device_tensor gate, qmv_device_tensor up,
                                                  const float *d_input, const float *d_norm_weight, float epsilon,
                                                  int batch_count, float *d_output, float *d_normed, void *stream)
{
    if (gate == nullptr || up == nullptr) {
        set_error("invalid fused SwiGLU arguments");
        return 0;
    }
    if (!group_args_ok(&gate, 1, d_input, batch_count, &d_output)) return 0;
    if (up->ggml_type != gate->ggml_type || up->cols != gate->cols || up->rows != gate->rows ||
        up->device != gate->device) {
        set_error("gate and up must share type, shape and device");
        return 0;
    }
    const int rows[1] = {gate->rows};
    if (!norm_args_ok(d_input, d_norm_weight, epsilon, gate->cols, batch_count, d_normed, &d_output, rows, 1))
        return 0;
    HIP_TRY(hipSetDevice(gate->device));
    hipStream_t s = (hipStream_t)stream;
    Workspace &ws = workspace_for(gate->device, s);
    QmvDeviceTensor *const pair[2] = {gate, up};
    float *const outs[2] = {d_output, d_output}; /* only job 0's output is written */
    Epilogue epi;
    epi.swiglu = true;
    return norm_then_group(pair, 2, d_input, d_norm_weight, epsilon, batch_count, outs, d_normed, s, ws, epi);
}

QMV_API int qmv_device_matvec_argmax_f32(qmv_device_tensor tensor, const float *d_input, float *d_logits,
                                         int *d_result, void *stream)
{
    if (tensor == nullptr || d_input == nullptr || d_logits == nullptr || d_result == nullptr) {
        set_error("invalid fused argmax arguments");
        return 0;
    }
    HIP_TRY(hipSetDevice(tensor->device));
    hipStream_t s = (hipStream_t)stream;
    Workspace &ws = workspace_for(tensor->device, s);
    Epilogue epi;
    epi.argmax = d_result;
    return launch_group(&tensor, 1, d_input, 1, &d_logits, s, ws, epi);
}

QMV_API int qmv_device_embed_rows_f32(qmv_device_tensor t, const int *d_token_ids, int count, float *d_output,
                                      int *d_status, void *stream)
{
    if (t == nullptr || d_token_ids == nullptr || d_output == nullptr || count <= 0 || count > 65535) {
        set_error("invalid embedding gather arguments");
        return 0;
    }
    HIP_TRY(hipSetDevice(t->device));
    hipStream_t s = (hipStream_t)stream;
    /* The status starts at 1 (a fill kernel, so the call can be captured)
     * and the gather clears it on an out-of-range id. */
    if (d_status != nullptr) HIP_TRY(qmv::launch_fill_u32((unsigned *)d_status, 1, 1u, s));
    HIP_TRY(qmv::launch_gather(t->geo.format, t->data, d_token_ids, count, d_output, t->rows, t->cols, t->units,
                               d_status, s));
    return 1;
}

QMV_API int qmv_device_dequantize_f32(qmv_device_tensor t, int first_row, int row_count, float *d_output,
                                      void *stream)
{
    if (t == nullptr || d_output == nullptr || first_row < 0 || row_count <= 0 ||
        (long long)first_row + row_count > t->rows) {
        set_error("invalid dequantize arguments");
        return 0;
    }
    HIP_TRY(hipSetDevice(t->device));
    HIP_TRY(qmv::launch_dequant(t->geo.format, t->data, d_output, t->rows, t->cols, t->units, first_row, row_count,
                                (hipStream_t)stream));
    return 1;
}

QMV_API const char *qmv_last_error(void)
{
    return t_error.c_str();
}

QMV_API int qmv_set_device(int ordinal)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || ordinal < 0 || ordinal >= n) {
        set_error("device %d not available", ordinal);
        return 0;
    }
    g_device.store(ordinal);
    return 1;
}

QMV_API int qmv_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

QMV_API void qmv_set_launch_tuning(int target_waves, int units_per_wave, int waves_per_group,
                                   int mfma_min_batch)
{
    g_mfma_min_batch.store(mfma_min_batch > 0 ? mfma_min_batch : 0);
    g_target_waves.store(target_waves > 0 ? target_waves : 0);
    g_force_u.store(units_per_wave > 0 ? units_per_wave : 0);
    g_force_w.store(waves_per_group > 0 && waves_per_group <= QMV_MAX_WAVES ? waves_per_group : 0);
}

QMV_API void qmv_set_rowmajor(int enable, int rows)
{
    g_rowdot.store(enable != 0 ? 1 : 0);
    g_rowdot_rows.store(rows == 1 || rows == 2 || rows == 4 ? rows : 2);
}

QMV_API void qmv_debug_fail_next_calls(int count)
{
    g_fail_next.store(count > 0 ? count : 0);
}
