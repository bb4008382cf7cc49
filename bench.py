"""Benchmark: Qwen2.5-7B-shaped decode-step projection set on one MI355X.

One step = every packed-weight projection of one decode step of a 28-layer
Qwen2.5-7B-shaped Q4_K_M model with synthetic weights resident in HBM:
per layer q,o 3584x3584, k,v 512x3584, gate,up 18944x3584 (Q4_K) and down
3584x18944 (Q6_K); 4,160,593,920 packed weight bytes. A layer issues 4
launches, the grouping a real decode step's data dependencies allow:
{q,k,v} (one shared input), {o}, {gate,up} (one shared input), {down}. The
112 launches of a step are captured once in a HIP graph and replayed.

Prints one JSON line: value = packed weight bytes / wall time per step
(GB/s) over the timed graph replays, the roofline of the dominant kernel
(its launches of one step captured in a graph of their own and replayed
between two HIP events on the stream the kernels run on, over the same
resident weights), the HBM traffic per
launch from the committed rocprofv3 counter summary when it covers this
kernel and workload, and the CPU baseline (the reference's own x86 build,
AVX2 + OpenMP, on a bounded sample). `extra` adds the same set at M=8 and at
M=32 (a prefill chunk of 32 positions per pass over the weights), the
per-step p10/p50/p90, eager (ungraphed) launch time, a measured streaming
read bandwidth, the vocabulary projection with greedy sampling, the same
layers as a device-resident decode step with its element operations
(biases, residuals, RMSNorm, SwiGLU), and the small Qwen2.5-0.5B/1.5B
configurations (cold and warm).
"""
import argparse
import ctypes
import importlib
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "weight-stream GB/s and % of HBM peak; µs per decode-step matvec set (1 GPU)"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3  # MI355X vector fp32 (the reference's arithmetic: fp32 FMA)


def batch_roofline(weight_bytes, flops, seconds):
    """Both bounds of a configuration: packed weight bytes over the HBM peak
    and the product's fp32 arithmetic (2 x positions x rows x columns flops)
    over the fp32 vector peak; `bound` names the larger fraction. The
    matrix-core and prefill paths compute the same exact products from three
    bf16 limbs per activation, so this fp32 figure is the algorithmic rate,
    not the matrix-core issue rate."""
    gbs = weight_bytes / seconds / 1e9
    tflops = flops / seconds / 1e12
    hbm, fp32 = gbs / HBM_PEAK_GBS, tflops / FP32_PEAK_TFLOPS
    return {"bound": "hbm" if hbm >= fp32 else "fp32", "frac": round(max(hbm, fp32), 4),
            "hbm": {"achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(hbm, 4)},
            "fp32": {"achieved": round(tflops, 2), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(fp32, 4)}}
LAYERS, HIDDEN, INTER, KV = 28, 3584, 18944, 512
Q4_K, Q6_K = 12, 14


def layer_shapes():
    # (name, type, rows, cols)
    return [("q", Q4_K, HIDDEN, HIDDEN), ("k", Q4_K, KV, HIDDEN), ("v", Q4_K, KV, HIDDEN),
            ("o", Q4_K, HIDDEN, HIDDEN), ("gate", Q4_K, INTER, HIDDEN), ("up", Q4_K, INTER, HIDDEN),
            ("down", Q6_K, HIDDEN, INTER)]


def _cpu_layer(qmv, host_layer, batch):
    import oracle

    views, xs, ys, nbytes = [], [], [], 0
    for name, t, rows, cols, raw in host_layer:
        views.append((oracle.view(raw, t, rows, cols), rows, cols))
        xs.append(qmv.synth_normal(batch * cols, seed=7000 + cols))
        ys.append(np.empty(batch * rows, dtype=np.float32))
        nbytes += raw.size
    return views, xs, ys, nbytes


def _time_cpu(fn, views, xs, ys, batch, seconds):
    """Median seconds per pass over layer 0's seven matvecs, ~`seconds` of passes."""
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 3 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        for (v, rows, cols), x, y in zip(views, xs, ys):
            assert fn(ctypes.byref(v), x.ctypes.data, cols, batch, y.ctypes.data, rows) == 1
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


_HOST_CPUS = None


def host_cpus():
    """CPUs this process may run on, the physical cores among them (distinct
    package/core pairs) and the CPU model name, from the kernel's view. Taken
    once, before the OpenMP runtime binds the main thread to one place
    (OMP_PROC_BIND), after which the thread's own affinity is that place."""
    global _HOST_CPUS
    if _HOST_CPUS is not None:
        return _HOST_CPUS
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        try:
            base = f"/sys/devices/system/cpu/cpu{c}/topology/"
            cores.add((open(base + "physical_package_id").read().strip(), open(base + "core_id").read().strip()))
        except OSError:
            cores.add(("?", str(c)))
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    _HOST_CPUS = (len(cpus), len(cores), model)
    return _HOST_CPUS


def cpu_threads():
    """Threads for the CPU baseline: OMP_NUM_THREADS where the environment
    sets it (a shared machine's CPU share for this job), else every physical
    core this process may use."""
    env = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return env if env > 0 else host_cpus()[1]


def cpu_baseline(qmv, host_layer, batch, seconds):
    """Time the reference's CPU path (its own sources, x86 Release flags with
    AVX2/FMA/F16C and OpenMP) on layer 0's seven matvecs for ~`seconds`, with
    the thread count applied to the OpenMP runtime that runs it and read back
    from it."""
    import oracle

    kind = "reference"
    lib = oracle.ref_lib("avx2")
    if lib is None:
        kind, lib = "port", oracle.lib()
    fn = lib.ref_quantized_tensor_matmul_f32 if kind == "reference" else lib.oracle_matmul_f32
    gomp = ctypes.CDLL("libgomp.so.1")  # the runtime the library already loaded
    threads = cpu_threads()
    gomp.omp_set_num_threads(threads)
    applied = gomp.omp_get_max_threads()
    views, xs, ys, nbytes = _cpu_layer(qmv, host_layer, batch)
    med, reps = _time_cpu(fn, views, xs, ys, batch, seconds)
    ncpu, ncores, model = host_cpus()
    env = {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OMP_PROC_BIND", "OMP_PLACES")}
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": applied, "kind": kind,
            "sample": f"layer 0 of the set (7 matvecs, {nbytes} packed bytes, M={batch}), "
                      f"{reps} repetitions, median {med * 1e3:.1f} ms "
                      f"({'oracle/_ref/libref_avx2.so: -O3 -mavx2 -mfma -mf16c -fopenmp' if kind == 'reference' else 'oracle/liboracle.so scalar port'}, "
                      f"omp_get_max_threads()={applied})",
            "host": {"nproc": ncpu, "physical_cores": ncores, "cpu_model": model,
                     "omp_get_max_threads": applied, "env": env}}


def cpu_variants(qmv, host_layer, batch, seconds):
    """The other CPU figures on the same layer: the reference's AVX2 build on
    one thread, and the scalar restatement (oracle, -O2 with no SIMD flags) on
    all threads; GB/s each."""
    import oracle

    views, xs, ys, nbytes = _cpu_layer(qmv, host_layer, batch)
    out = {}
    ref = oracle.ref_lib("avx2")
    if ref is not None:
        gomp = ctypes.CDLL("libgomp.so.1")
        before = gomp.omp_get_max_threads()
        gomp.omp_set_num_threads(1)
        try:
            med, _ = _time_cpu(ref.ref_quantized_tensor_matmul_f32, views, xs, ys, batch, seconds)
        finally:
            gomp.omp_set_num_threads(before)
        out["reference_avx2_1_thread_gbs"] = round(nbytes / med / 1e9, 3)
    med, _ = _time_cpu(oracle.lib().oracle_matmul_f32, views, xs, ys, batch, seconds)
    out["scalar_port_all_threads_gbs"] = round(nbytes / med / 1e9, 3)
    return out


# Single-position Q4_K launches of at most this many (64-row tile, 256-weight
# unit) pairs run on the row-major kernel at QMV_ROWDOT_ROWS rows per row
# segment, larger ones over rows of at most 16 super-blocks at 4; Q6_K rows
# of 17 to 128 super-blocks run on the row-loop kernel (the library's policy,
# including its QMV_ROWDOT / QMV_ROWDOT_ROWS / QMV_ROWDOT_Q6K switches read
# at start-up).
ROWDOT_MAX_UNITS = 2048
ROWDOT_SHARED_SB = 16


def kernel_name(fmt, M, tiled_units=None, cols=None):
    """The kernel a Q4_K / Q6_K launch of M positions over `tiled_units`
    (tile, unit) pairs of rows of `cols` columns runs (default tuning)."""
    if M > 8:
        return "prefill_kernel<%s,%d>" % (fmt, 1 if M <= 16 else 2)
    if M >= (7 if fmt == "Q4_K" else 8):
        return "matvec_mfma_kernel<%s,%d>" % (fmt, M)
    rowdot = os.environ.get("QMV_ROWDOT", "1") != "0"
    if fmt == "Q6_K" and M == 1 and cols is not None and rowdot and os.environ.get("QMV_ROWDOT_Q6K", "1") != "0":
        sb = cols // 256
        if ROWDOT_SHARED_SB < sb <= 128:
            return "rowloop_q6k_kernel<%d,2>" % (-(-sb // 16))
    if fmt == "Q4_K" and M == 1 and tiled_units is not None and rowdot:
        if tiled_units <= ROWDOT_MAX_UNITS:
            rows = os.environ.get("QMV_ROWDOT_ROWS", "2")
            return "rowgroup_q4k_kernel<%s,64,0,false>" % (rows if rows in ("1", "2", "4") else "2")
        if cols is not None and cols // 256 <= ROWDOT_SHARED_SB:
            return "rowgroup_q4k_kernel<4,64,0,false>"
    return "matvec_kernel<%s,%d>" % (fmt, M)


def build_launches(lib, layers, acts, outs, M):
    """One step = 4 launches per layer, arguments prepared once: (kernel name,
    algorithmic bytes, callable(stream), launch shape)."""
    grp_fn = lib.qmv_device_matvec_group_f32
    one_fn = lib.qmv_device_matvec_f32
    launches = []
    for layer in range(LAYERS):
        T, A, O = layers[layer], acts[layer], outs[layer]

        def grp(names, x, T=T, O=O):
            hs = (ctypes.c_void_p * len(names))(*[T[n].handle.value for n in names])
            ps = (ctypes.c_void_p * len(names))(*[O[n].ptr for n in names])
            n, xp = len(names), x.ptr
            return lambda s: grp_fn(hs, n, xp, M, ps, s)

        def one(name, x, T=T, O=O):
            h, xp, yp = T[name].handle, x.ptr, O[name].ptr
            return lambda s: one_fn(h, xp, M, yp, s)

        def algo(names, cols):
            w = sum(T[n].packed_bytes for n in names)
            return w + 4 * M * cols + 4 * M * sum(T[n].rows for n in names)

        def kern(fmt, names, cols):
            return kernel_name(fmt, M, sum(-(-T[n].rows // 64) * (cols // 256) for n in names), cols)

        launches.append((kern("Q4_K", ["q", "k", "v"], HIDDEN), algo(["q", "k", "v"], HIDDEN),
                         grp(["q", "k", "v"], A["attn"]), "qkv"))
        launches.append((kern("Q4_K", ["o"], HIDDEN), algo(["o"], HIDDEN), one("o", A["o"]), "o"))
        launches.append((kern("Q4_K", ["gate", "up"], HIDDEN), algo(["gate", "up"], HIDDEN),
                         grp(["gate", "up"], A["ffn"]), "gate_up"))
        launches.append((kern("Q6_K", ["down"], INTER), algo(["down"], INTER), one("down", A["down"]), "down"))
    return launches


def run_set(qmv, hip, stream, launches, steps, warmup, use_graph):
    """Warm up, then time `steps` steps (graph replays unless use_graph is
    False) between two stream synchronisations; events between steps give
    the per-step spread."""
    sp = stream.handle

    def step():
        for launch in launches:
            if launch[2](sp) != 1:
                raise RuntimeError(qmv.last_error())

    for _ in range(max(1, warmup)):
        step()
    stream.synchronize()
    graph = None
    if use_graph:
        graph = hip.Graph(stream)
        graph.begin()
        step()
        graph.end()
        for _ in range(warmup):
            graph.replay()
        stream.synchronize()
    marks = [hip.Event() for _ in range(steps + 1)]
    t0 = time.perf_counter()
    for i in range(steps):
        marks[i].record(stream)
        graph.replay() if graph is not None else step()
    marks[steps].record(stream)
    stream.synchronize()
    elapsed = time.perf_counter() - t0
    per_step = sorted(marks[i].elapsed_ms(marks[i + 1]) for i in range(steps))
    eager = None
    if graph is not None:
        reps = max(3, steps // 5)
        t0 = time.perf_counter()
        for _ in range(reps):
            step()
        stream.synchronize()
        eager = (time.perf_counter() - t0) / reps
    for m in marks:
        m.destroy()
    if graph is not None:
        graph.destroy()
    q = lambda f: per_step[min(len(per_step) - 1, int(f * len(per_step)))]
    return {"elapsed": elapsed, "ms_per_step": elapsed / steps * 1e3, "p10": q(0.1), "p50": q(0.5),
            "p90": q(0.9), "eager_ms": eager * 1e3 if eager else None, "graph": graph is not None}


def launch_profile(hip, stream, launches, passes, use_graph, key=0):
    """Average duration per launch of each kernel (key 0) or launch shape
    (key 3): the group's own launches of one step, in step order, captured in
    a HIP graph and replayed `passes` times between two HIP events on the
    launch stream (no event between launches, so dispatch overhead is
    counted as in the timed replays). Returns {group: [algorithmic bytes, ms,
    launches]} over all passes."""
    per_kernel = {}
    sp = stream.handle
    for name in sorted({launch[key] for launch in launches}):
        mine = [(launch[1], launch[2]) for launch in launches if launch[key] == name]
        run = lambda: [fn(sp) for _, fn in mine]
        graph = None
        if use_graph:
            graph = hip.Graph(stream)
            graph.begin()
            run()
            graph.end()
            graph.replay()
        else:
            run()
        stream.synchronize()
        e0, e1 = hip.Event(), hip.Event()
        e0.record(stream)
        for _ in range(passes):
            graph.replay() if graph is not None else run()
        e1.record(stream)
        stream.synchronize()
        per_kernel[name] = [passes * sum(b for b, _ in mine), e0.elapsed_ms(e1), passes * len(mine)]
        e0.destroy()
        e1.destroy()
        if graph is not None:
            graph.destroy()
    return per_kernel


def streaming_floor(probe, hip, stream, launches, passes, main_run, no_graph):
    """Streaming floors in the same run: each launch shape's launches of one
    step (and the whole step) as dependent read-only launches over distinct
    buffers of the same byte counts, replayed from a graph
    (probe.read_chain_us), against the matvec launches of that shape timed
    the same way (launch_profile by shape)."""
    shapes = launch_profile(hip, stream, launches, passes, not no_graph, key=3)
    out = {"method": "graph of dependent read-only launches over distinct buffers of each launch's "
                     "algorithmic bytes, each read once (fastest of 1/2/4/8 loads in flight per thread), "
                     "same run",
           "floor_us": {}, "kernel_us": {}, "kernel_to_floor": {}}
    for shape, (nbytes, ms, count) in shapes.items():
        sizes = [launch[1] for launch in launches if launch[3] == shape]
        floor = probe.read_chain_us(sizes) / len(sizes)
        us = ms / count * 1e3
        out["floor_us"][shape] = round(floor, 3)
        out["kernel_us"][shape] = round(us, 3)
        out["kernel_to_floor"][shape] = round(us / floor, 3)
    set_floor = probe.read_chain_us([launch[1] for launch in launches]) / 1e3
    out["set_floor_ms"] = round(set_floor, 4)
    out["set_to_floor"] = round(main_run["ms_per_step"] / set_floor, 3)
    return out


def vocab_bench(qmv, hip, stream, reps):
    """Vocabulary projection 151936 x 3584 Q6_K at M=1 followed by greedy
    sampling: the matvec alone, matvec + separate device argmax, and the
    fused launch; each from graph replays between two HIP events."""
    rows, cols = 151936, 3584
    raw = qmv.synth_tensor(Q6_K, rows, cols, seed=77)
    nbytes = raw.size
    dt = qmv.DeviceTensor(qmv.make_view(raw, Q6_K, rows, cols))
    del raw
    dx = hip.DeviceBuffer.from_array(qmv.synth_normal(cols, seed=78))
    dl = hip.DeviceBuffer(4 * rows)
    res = hip.DeviceBuffer(8)
    sp = stream.handle
    variants = {
        "matvec": lambda: dt.matvec(dx.ptr, 1, dl.ptr, sp),
        "matvec_then_argmax": lambda: (dt.matvec(dx.ptr, 1, dl.ptr, sp),
                                       qmv.device_greedy_argmax(dl.ptr, rows, res.ptr, sp)),
        "fused_matvec_argmax": lambda: qmv.device_matvec_argmax(dt, dx.ptr, dl.ptr, res.ptr, sp),
    }
    out = {"shape": f"{rows}x{cols} Q6_K", "packed_bytes": nbytes}
    for name, fn in variants.items():
        fn()
        stream.synchronize()
        g = hip.Graph(stream)
        g.begin()
        fn()
        g.end()
        g.replay()
        stream.synchronize()
        e0, e1 = hip.Event(), hip.Event()
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
        stream.synchronize()
        us = e0.elapsed_ms(e1) / reps * 1e3
        out[name + "_us"] = round(us, 2)
        e0.destroy()
        e1.destroy()
        g.destroy()
    out["matvec_gbs"] = round(nbytes / (out["matvec_us"] * 1e-6) / 1e9, 1)
    dt.close()
    return out


def graph_us(hip, stream, fns, reps):
    """Capture fns (each enqueues on `stream`) once; µs per replay between two
    HIP events on the stream."""
    for fn in fns:
        fn()
    stream.synchronize()
    g = hip.Graph(stream)
    g.begin()
    for fn in fns:
        fn()
    g.end()
    g.replay()
    stream.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(stream)
    for _ in range(reps):
        g.replay()
    e1.record(stream)
    stream.synchronize()
    us = e0.elapsed_ms(e1) / reps * 1e3
    e0.destroy()
    e1.destroy()
    g.destroy()
    return us


def decode_ops_bench(qmv, hip, stream, layers, reps):
    """The same 28 layers as a device-resident decode step: the projections
    with the element operations between them on device buffers (RMSNorm ->
    q/k/v + bias -> o + residual -> RMSNorm -> gate/up SwiGLU -> down +
    residual; RoPE and attention are not on this path, so o reads the query
    rows). 6 launches per layer, captured once and replayed between two HIP
    events; then each kind of launch alone (its 28 or 56 launches of a step
    in one graph) for the time per launch; then the same step with the norms
    fused into the projections after them (4 launches per layer)."""
    D = hip.DeviceBuffer
    rng = np.random.default_rng(90)
    vec = lambda n, s: D.from_array((s * rng.standard_normal(n)).astype(np.float32))
    x = D.from_array(qmv.synth_normal(HIDDEN, seed=91))
    w_attn, w_ffn = D.from_array(np.ones(HIDDEN, np.float32)), D.from_array(np.ones(HIDDEN, np.float32))
    bq, bk, bv = vec(HIDDEN, 0.1), vec(KV, 0.1), vec(KV, 0.1)
    h, q, k, v, act = D(4 * HIDDEN), D(4 * HIDDEN), D(4 * KV), D(4 * KV), D(4 * INTER)
    sp = stream.handle
    eps = 1e-6
    ops = []  # (kind, fn) in step order
    for T in layers:
        ops += [
            ("rms_norm", lambda: qmv.device_rms_norm(x.ptr, w_attn.ptr, HIDDEN, 1, eps, h.ptr, sp)),
            ("qkv_bias", lambda T=T: qmv.device_matvec_add_group(
                [T["q"], T["k"], T["v"]], h.ptr, 1, [bq.ptr, bk.ptr, bv.ptr], [0, 0, 0], [q.ptr, k.ptr, v.ptr], sp)),
            ("o_residual", lambda T=T: qmv.device_matvec_add_group([T["o"]], q.ptr, 1, [x.ptr], [HIDDEN], [x.ptr],
                                                                   sp)),
            ("rms_norm", lambda: qmv.device_rms_norm(x.ptr, w_ffn.ptr, HIDDEN, 1, eps, h.ptr, sp)),
            ("gate_up_swiglu", lambda T=T: qmv.device_matvec_swiglu(T["gate"], T["up"], h.ptr, 1, act.ptr, sp)),
            ("down_residual", lambda T=T: qmv.device_matvec_add_group([T["down"]], act.ptr, 1, [x.ptr], [HIDDEN],
                                                                      [x.ptr], sp)),
        ]
    out = {"ms_per_step": round(graph_us(hip, stream, [fn for _, fn in ops], reps) / 1e3, 4),
           "launches_per_step": len(ops)}
    out["residual_finite"] = bool(np.isfinite(x.to_array(np.float32, (HIDDEN,))).all())
    per = {}
    for kind in dict.fromkeys(k for k, _ in ops):
        fns = [fn for k, fn in ops if k == kind]
        per[kind] = round(graph_us(hip, stream, fns, reps) / len(fns), 2)
    out["us_per_launch"] = per
    # The same step through the fused norm entry points
    # (qmv_device_rms_norm_matvec_add_group_f32 / _swiglu_f32): 4 calls per
    # layer; the library fuses the attention norm into the q/k/v launch and
    # keeps the FFN norm as a launch of its own before the large gate/up
    # launch, so 5 launches per layer.
    fused = []
    for T in layers:
        fused += [
            ("norm_qkv_bias", lambda T=T: qmv.device_rms_norm_matvec_add_group(
                [T["q"], T["k"], T["v"]], x.ptr, w_attn.ptr, eps, 1, [bq.ptr, bk.ptr, bv.ptr], [0, 0, 0],
                [q.ptr, k.ptr, v.ptr], h.ptr, sp)),
            ("o_residual", lambda T=T: qmv.device_matvec_add_group([T["o"]], q.ptr, 1, [x.ptr], [HIDDEN], [x.ptr],
                                                                   sp)),
            ("norm_gate_up_swiglu", lambda T=T: qmv.device_rms_norm_matvec_swiglu(
                T["gate"], T["up"], x.ptr, w_ffn.ptr, eps, 1, act.ptr, h.ptr, sp)),
            ("down_residual", lambda T=T: qmv.device_matvec_add_group([T["down"]], act.ptr, 1, [x.ptr], [HIDDEN],
                                                                      [x.ptr], sp)),
        ]
    fo = {"ms_per_step": round(graph_us(hip, stream, [fn for _, fn in fused], reps) / 1e3, 4),
          "calls_per_step": len(fused)}
    fo["residual_finite"] = bool(np.isfinite(x.to_array(np.float32, (HIDDEN,))).all())
    per = {}
    for kind in ("norm_qkv_bias", "norm_gate_up_swiglu"):
        fns = [fn for k, fn in fused if k == kind]
        per[kind] = round(graph_us(hip, stream, fns, reps) / len(fns), 2)
    fo["us_per_launch"] = per
    out["fused_norms"] = fo
    return out


def small_configs_bench(qmv, hip, stream, reps):
    """The small reference configurations, latency- and launch-bound:
    Q8_0 896x896 (Qwen2.5-0.5B q_proj) and Q6_K 896x4864 (its FFN down; the
    Q4_K 4864x896 gate/up shape is not a valid Q4_K tensor and is rejected,
    as by the reference) at M=1, and one Qwen2.5-1.5B layer set at M=8 (q|k|v
    Q5_0 1536/256/256x1536, o Q5_0 1536x1536, gate|up Q4_K 8960x1536, down
    Q4_K 1536x8960) as its four launches, also at 32 positions. Cold: graph
    replays cycling through enough copies to exceed 1 GB (twice the Infinity
    Cache); warm: one copy."""
    Q5_0, Q8_0 = 6, 8
    D = hip.DeviceBuffer
    sp = stream.handle
    cases = {
        "q8_0_896x896_m1": (1, [[("a", Q8_0, 896, 896)]]),
        "q6_k_896x4864_m1": (1, [[("a", Q6_K, 896, 4864)]]),
        "qwen2_1_5b_layer_set_m8": (8, [[("q", Q5_0, 1536, 1536), ("k", Q5_0, 256, 1536), ("v", Q5_0, 256, 1536)],
                                        [("o", Q5_0, 1536, 1536)],
                                        [("gate", Q4_K, 8960, 1536), ("up", Q4_K, 8960, 1536)],
                                        [("down", Q4_K, 1536, 8960)]]),
    }
    # The same layer set as one prefill chunk of 32 positions (the reference
    # prefills in chunks of 8, src/qwen2_internal.h:7).
    cases["qwen2_1_5b_layer_set_m32"] = (32, cases["qwen2_1_5b_layer_set_m8"][1])
    out = {}
    for name, (m, groups) in cases.items():
        raws = {t[0]: qmv.synth_tensor(t[1], t[2], t[3], seed=900 + i)
                for i, t in enumerate(x for g in groups for x in g)}
        nbytes = sum(r.size for r in raws.values())
        flops = 2 * m * sum(t[2] * t[3] for g in groups for t in g)
        copies = max(2, -(-(1 << 30) // nbytes))
        sets = [{t[0]: qmv.DeviceTensor(qmv.make_view(raws[t[0]], t[1], t[2], t[3])) for g in groups for t in g}
                for _ in range(copies)]
        xs = [D.from_array(qmv.synth_normal(m * g[0][3], seed=950 + j)) for j, g in enumerate(groups)]
        ys = [[D(4 * m * t[2]) for t in g] for g in groups]

        def launches(ts):
            return [lambda g=g, x=x, y=y: qmv.device_matvec_group([ts[t[0]] for t in g], x.ptr, m,
                                                                  [b.ptr for b in y], sp)
                    for g, x, y in zip(groups, xs, ys)]

        cold = graph_us(hip, stream, [fn for ts in sets for fn in launches(ts)], reps) / copies
        # Warm: the first copy's launches repeated as many times in one graph.
        warm = graph_us(hip, stream, launches(sets[0]) * copies, reps) / copies
        out[name] = {"packed_bytes": nbytes, "launches": len(groups), "positions": m, "copies_cold": copies,
                     "cold_us": round(cold, 2), "warm_us": round(warm, 2),
                     "cold_weight_gbs": round(nbytes / (cold * 1e-6) / 1e9, 1),
                     "roofline_cold": batch_roofline(nbytes, flops, cold * 1e-6)}
        for ts in sets:
            for d in ts.values():
                d.close()
    return out


def committed_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (FETCH_SIZE and WRITE_SIZE passes, each scaled by a copy-kernel
    calibration), if it was taken on this kernel and workload."""
    path = os.path.join(ROOT, "profiles", "roofline_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("kernel") != kernel or t.get("workload") != workload:
        return None
    return int(t["fetch_bytes_per_launch"] + t["write_bytes_per_launch"])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=1, help="positions per matvec (1 = decode, <= 32)")
    ap.add_argument("--profile-passes", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the M=8 set and the read probe")
    args = ap.parse_args()
    # Thread placement for the CPU baseline, set before any library starts
    # the OpenMP runtime (it reads these once).
    host_cpus()
    os.environ.setdefault("OMP_PROC_BIND", "close")
    os.environ.setdefault("OMP_PLACES", "cores")
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this path has no multi-GPU mode); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    if not 1 <= args.batch <= 32:
        print("--batch must be in 1..32", file=sys.stderr)
        sys.exit(2)

    qmv = importlib.import_module("my-inference-engine_amd")
    hip = importlib.import_module("my-inference-engine_amd.hip_runtime")
    lib = qmv.hip_lib()
    assert lib.qmv_device_count() > 0, "no GPU"
    assert lib.qmv_set_device(0) == 1
    hip.check(hip.rt().hipSetDevice(0), "hipSetDevice")
    stream = hip.Stream()
    M = args.batch
    MX = 32  # activation rows per layer: the M = 32 prefill leg reads all of them

    # ---- weights: generated per layer on the host, uploaded, host copy dropped
    t0 = time.time()
    layers, host_layer0, total_bytes = [], None, 0
    for layer in range(LAYERS):
        tensors = {}
        keep = []
        for j, (name, t, rows, cols) in enumerate(layer_shapes()):
            raw = qmv.synth_tensor(t, rows, cols, seed=1000 * layer + j)
            total_bytes += raw.size
            tensors[name] = qmv.DeviceTensor(qmv.make_view(raw, t, rows, cols))
            if layer == 0:
                keep.append((name, t, rows, cols, raw))
        if layer == 0:
            host_layer0 = keep
        layers.append(tensors)
    upload_s = time.time() - t0

    # ---- activations (fp32 N(0,1), token-major [MX, K] per layer) and
    # outputs, resident in HBM; an M-position set reads the first M rows
    acts, outs = [], []
    for layer in range(LAYERS):
        a = {k: hip.DeviceBuffer.from_array(qmv.synth_normal(MX * c, seed=50000 + 10 * layer + i))
             for i, (k, c) in enumerate((("attn", HIDDEN), ("o", HIDDEN), ("ffn", HIDDEN), ("down", INTER)))}
        o = {name: hip.DeviceBuffer(4 * MX * rows) for name, _, rows, _ in layer_shapes()}
        acts.append(a)
        outs.append(o)
    hip.synchronize()

    set_weights = LAYERS * sum(rows * cols for _, _, rows, cols in layer_shapes())  # rows x columns
    launches = build_launches(lib, layers, acts, outs, M)
    main_run = run_set(qmv, hip, stream, launches, args.steps, args.warmup, not args.no_graph)
    passes = max(1, args.profile_passes)
    per_kernel = launch_profile(hip, stream, launches, passes, not args.no_graph)

    value = total_bytes / (main_run["elapsed"] / args.steps) / 1e9
    dname, (dbytes, dms, dcount) = max(per_kernel.items(), key=lambda kv: kv[1][1])
    achieved = (dbytes / dcount) / (dms / dcount * 1e-3) / 1e9
    kernels = {k: {"launches_per_step": v[2] // passes,
                   "avg_bytes": v[0] // v[2], "avg_us": round(v[1] / v[2] * 1e3, 3),
                   "gbs": round((v[0] / v[2]) / (v[1] / v[2] * 1e-3) / 1e9, 1)} for k, v in per_kernel.items()}
    workload = (f"Qwen2.5-7B-shaped decode-step projection set, M={M}: 28 layers x "
                "{q,o 3584x3584; k,v 512x3584; gate,up 18944x3584 Q4_K; down 3584x18944 Q6_K}")

    extra = {"per_step_ms_p10_p50_p90": [round(main_run[k], 4) for k in ("p10", "p50", "p90")],
             "eager_ms_per_step": round(main_run["eager_ms"], 4) if main_run["eager_ms"] else None,
             "kernel_sum_ms_per_step": round(sum(v[1] for v in per_kernel.values()) / passes, 4),
             "kernels": kernels, "upload_s": round(upload_s, 2)}
    if not args.no_extra:
        for mb in (8, 32):
            if mb == M:
                continue
            lb = build_launches(lib, layers, acts, outs, mb)
            rb = run_set(qmv, hip, stream, lb, max(5, args.steps // 5), 2, not args.no_graph)
            extra[f"m{mb}_set"] = {"ms_per_step": round(rb["ms_per_step"], 4),
                                   "weight_gbs": round(total_bytes / (rb["elapsed"] / max(5, args.steps // 5)) / 1e9,
                                                       1),
                                   "positions_per_s": round(mb / (rb["ms_per_step"] * 1e-3), 1),
                                   "roofline": batch_roofline(total_bytes, 2 * mb * set_weights,
                                                              rb["ms_per_step"] * 1e-3)}
        extra["vocab_projection"] = vocab_bench(qmv, hip, stream, max(10, args.steps // 2))
        if M == 1:
            ops = decode_ops_bench(qmv, hip, stream, layers, max(10, args.steps // 2))
            ops["projection_set_ms"] = round(main_run["ms_per_step"], 4)
            ops["element_ops_overhead_ms"] = round(ops["ms_per_step"] - main_run["ms_per_step"], 4)
            extra["decode_step_with_element_ops"] = ops
        extra["small_configs"] = small_configs_bench(qmv, hip, stream, max(5, args.steps // 10))
        probe = importlib.import_module("my-inference-engine_amd.probe")
        extra["streaming_floor"] = streaming_floor(probe, hip, stream, launches, passes, main_run, args.no_graph)
        extra["hbm_read_probe"] = probe.read_bandwidth(1 << 30, 512, 10)
        extra["hbm_fraction_of_read_probe"] = round(value / extra["hbm_read_probe"]["gbs"], 4)

    # ---- the drop-in host-pointer API (host x in, host y out, weights cached
    # in HBM after the first call): PCIe-inclusive time per call, never `value`
    host_api = {}
    for name, t, rows, cols, raw in host_layer0 if not args.no_extra else []:
        if name not in ("o", "gate", "down"):
            continue
        v = qmv.make_view(raw, t, rows, cols)
        x = qmv.synth_normal(cols, seed=7000 + cols)
        y = np.empty(rows, dtype=np.float32)
        if qmv.quantized_tensor_matvec_f32(v, x, cols, y, rows) != 1:
            raise RuntimeError(qmv.last_error())
        reps = 50
        t0 = time.perf_counter()
        for _ in range(reps):
            qmv.quantized_tensor_matvec_f32(v, x, cols, y, rows)
        host_api[name] = round((time.perf_counter() - t0) / reps * 1e6, 1)
        qmv.release_tensor(v.data)
    if host_api:
        extra["host_api_us_per_call"] = host_api

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(qmv, host_layer0, M, args.cpu_seconds)
        if not args.no_extra:
            extra["cpu_variants"] = cpu_variants(qmv, host_layer0, M, min(3.0, args.cpu_seconds))

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_run["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded Q4_K/Q6_K weights (d,dmin ~ |N(0,0.01)|, Q6_K d ~ |N(0,0.001)|), fp32 N(0,1) activations",
        "config": {"workload": workload, "batch": M, "layers": LAYERS, "packed_weight_bytes": total_bytes,
                   "launches_per_step": len(launches), "hip_graph": main_run["graph"]},
        "us_per_set": round(main_run["ms_per_step"] * 1e3, 1),
        "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": committed_traffic(dname, workload),
                     "kernel": dname, "bytes_per_launch": dbytes // dcount,
                     "avg_launch_us": round(dms / dcount * 1e3, 3)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
