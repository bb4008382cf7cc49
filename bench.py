"""Benchmark: Qwen2.5-7B-shaped decode-step projection set on one MI355X.

One step = every packed-weight projection of one decode step of a 28-layer
Qwen2.5-7B-shaped Q4_K_M model with synthetic weights resident in HBM:
per layer q,o 3584x3584, k,v 512x3584, gate,up 18944x3584 (Q4_K) and down
3584x18944 (Q6_K); 4,160,593,920 packed weight bytes. A layer issues 4
launches, the grouping a real decode step's data dependencies allow:
{q,k,v} (one shared input), {o}, {gate,up} (one shared input), {down}. The
112 launches of a step are captured once in a HIP graph and replayed.

Prints one JSON line: value = packed weight bytes / wall time per step
(GB/s), the roofline of the dominant kernel (HIP events around each launch
of a separate profiling pass over the same resident weights), and the CPU
baseline (the reference's own x86 build, AVX2 + OpenMP, on a bounded sample).
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
LAYERS, HIDDEN, INTER, KV = 28, 3584, 18944, 512
Q4_K, Q6_K = 12, 14


def layer_shapes():
    # (name, type, rows, cols)
    return [("q", Q4_K, HIDDEN, HIDDEN), ("k", Q4_K, KV, HIDDEN), ("v", Q4_K, KV, HIDDEN),
            ("o", Q4_K, HIDDEN, HIDDEN), ("gate", Q4_K, INTER, HIDDEN), ("up", Q4_K, INTER, HIDDEN),
            ("down", Q6_K, HIDDEN, INTER)]


def cpu_baseline(qmv, host_layer, batch, seconds):
    """Time the reference's CPU path (its own sources, x86 Release flags with
    AVX2/FMA/F16C and OpenMP) on layer 0's seven matvecs for ~`seconds`."""
    import oracle

    kind = "reference"
    lib = oracle.ref_lib("avx2")
    if lib is None:
        kind, lib = "port", oracle.lib()
    fn = lib.ref_quantized_tensor_matmul_f32 if kind == "reference" else lib.oracle_matmul_f32
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
    views, xs, ys, nbytes = [], [], [], 0
    for name, t, rows, cols, raw in host_layer:
        v = oracle.view(raw, t, rows, cols)
        x = qmv.synth_normal(batch * cols, seed=7000 + cols)
        views.append((v, rows, cols))
        xs.append(x)
        ys.append(np.empty(batch * rows, dtype=np.float32))
        nbytes += raw.size
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 3 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        for (v, rows, cols), x, y in zip(views, xs, ys):
            assert fn(ctypes.byref(v), x.ctypes.data, cols, batch, y.ctypes.data, rows) == 1
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": f"layer 0 of the set (7 matvecs, {nbytes} packed bytes, M={batch}), "
                      f"{len(times)} repetitions, median {med * 1e3:.1f} ms "
                      f"({'oracle/_ref/libref_avx2.so: -O3 -mavx2 -mfma -mf16c -fopenmp' if kind == 'reference' else 'oracle/liboracle.so scalar port'}, "
                      f"OMP_NUM_THREADS={threads})"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=1, help="positions per matvec (1 = decode, <= 8)")
    ap.add_argument("--profile-passes", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this path has no multi-GPU mode); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    qmv = importlib.import_module("my-inference-engine_amd")
    hip = importlib.import_module("my-inference-engine_amd.hip_runtime")
    lib = qmv.hip_lib()
    assert lib.qmv_device_count() > 0, "no GPU"
    assert lib.qmv_set_device(0) == 1
    hip.check(hip.rt().hipSetDevice(0), "hipSetDevice")
    stream = hip.Stream()
    sp = stream.handle
    M = args.batch

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

    # ---- activations (fp32 N(0,1), per layer) and outputs, resident in HBM
    acts, outs = [], []
    for layer in range(LAYERS):
        a = {k: hip.DeviceBuffer.from_array(qmv.synth_normal(M * c, seed=50000 + 10 * layer + i))
             for i, (k, c) in enumerate((("attn", HIDDEN), ("o", HIDDEN), ("ffn", HIDDEN), ("down", INTER)))}
        o = {name: hip.DeviceBuffer(4 * M * rows) for name, _, rows, _ in layer_shapes()}
        acts.append(a)
        outs.append(o)
    hip.synchronize()

    # ---- one step = 4 launches per layer, arguments prepared once
    grp_fn = lib.qmv_device_matvec_group_f32
    one_fn = lib.qmv_device_matvec_f32
    launches = []  # (kernel name, algorithmic bytes, callable(stream))
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

        kq, k6 = "matvec_kernel<Q4_K,%d>" % M, "matvec_kernel<Q6_K,%d>" % M
        launches.append((kq, algo(["q", "k", "v"], HIDDEN), grp(["q", "k", "v"], A["attn"])))
        launches.append((kq, algo(["o"], HIDDEN), one("o", A["o"])))
        launches.append((kq, algo(["gate", "up"], HIDDEN), grp(["gate", "up"], A["ffn"])))
        launches.append((k6, algo(["down"], INTER), one("down", A["down"])))

    def step(s):
        for _, _, fn in launches:
            if fn(s) != 1:
                raise RuntimeError(qmv.last_error())

    for _ in range(max(1, args.warmup)):
        step(sp)
    stream.synchronize()

    graph = None
    if not args.no_graph:
        graph = hip.Graph(stream)
        graph.begin()
        step(sp)
        graph.end()
        for _ in range(args.warmup):
            graph.replay()
        stream.synchronize()

    t_a = time.perf_counter()
    for _ in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            step(sp)
    stream.synchronize()
    elapsed = time.perf_counter() - t_a

    eager_elapsed = None
    if graph is not None:
        reps = max(3, args.steps // 5)
        t_a = time.perf_counter()
        for _ in range(reps):
            step(sp)
        stream.synchronize()
        eager_elapsed = (time.perf_counter() - t_a) / reps

    # ---- profiling pass: HIP events around every launch, on the bench stream
    per_kernel = {}
    kernel_sum = []
    evs = [(hip.Event(), hip.Event()) for _ in launches]
    for _ in range(args.profile_passes):
        for (name, nbytes, fn), (e0, e1) in zip(launches, evs):
            e0.record(stream)
            fn(sp)
            e1.record(stream)
        stream.synchronize()
        tot = 0.0
        for (name, nbytes, _), (e0, e1) in zip(launches, evs):
            ms = e0.elapsed_ms(e1)
            tot += ms
            d = per_kernel.setdefault(name, [0, 0.0, 0])
            d[0] += nbytes
            d[1] += ms
            d[2] += 1
        kernel_sum.append(tot)

    ms_per_step = elapsed / args.steps * 1e3
    value = total_bytes / (elapsed / args.steps) / 1e9
    dominant = max(per_kernel.items(), key=lambda kv: kv[1][1])
    dname, (dbytes, dms, dcount) = dominant
    achieved = (dbytes / dcount) / (dms / dcount * 1e-3) / 1e9
    kernels = {k: {"launches_per_step": v[2] // args.profile_passes,
                   "avg_bytes": v[0] // v[2], "avg_us": round(v[1] / v[2] * 1e3, 3),
                   "gbs": round((v[0] / v[2]) / (v[1] / v[2] * 1e-3) / 1e9, 1)} for k, v in per_kernel.items()}

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(qmv, host_layer0, M, args.cpu_seconds)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded Q4_K/Q6_K weights (d,dmin ~ |N(0,0.01)|, Q6_K d ~ |N(0,0.001)|), fp32 N(0,1) activations",
        "config": {"workload": f"Qwen2.5-7B-shaped decode-step projection set, M={M}: 28 layers x "
                               "{q,o 3584x3584; k,v 512x3584; gate,up 18944x3584 Q4_K; down 3584x18944 Q6_K}",
                   "batch": M, "layers": LAYERS, "packed_weight_bytes": total_bytes,
                   "launches_per_step": len(launches), "hip_graph": graph is not None},
        "us_per_set": round(ms_per_step * 1e3, 1),
        "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": dname,
                     "bytes_per_launch": dbytes // dcount, "avg_launch_us": round(dms / dcount * 1e3, 3)},
        "cpu_baseline": cpu,
        "extra": {"eager_ms_per_step": round(eager_elapsed * 1e3, 4) if eager_elapsed else None,
                  "kernel_sum_ms_per_step": round(statistics.median(kernel_sum), 4),
                  "kernels": kernels, "upload_s": round(upload_s, 2)},
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
