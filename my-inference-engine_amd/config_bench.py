"""Per-configuration benchmark of the packed matvec on one GPU.

The GPU counterpart of the reference's synthetic benchmark CLI
(tests/quantized_matvec_benchmark.cpp:57-99, which times one shape per
format on the CPU): each named configuration below is synthesised with the
seeded generators, uploaded once, and its launches are timed with HIP events
around `reps` eager repetitions after two warm-up repetitions (no graph, so a
profiler sees plain dispatches). Small configurations cycle through enough
copies of their weights to exceed 1 GiB, twice the 256 MB Infinity Cache, so
every repetition reads HBM.

Configurations:
  c1     Q8_0 896x896, one position (Qwen2.5-0.5B q_proj)
  c2     Q6_K 896x4864, one position (its FFN down); the Q4_K 4864x896
         gate/up shape is not a valid Q4_K tensor and is only checked to be
         rejected, as the reference rejects it
  c3     Qwen2.5-1.5B layer set, 8 positions: q|k|v Q5_0 1536/256/256x1536,
         o Q5_0 1536x1536, gate|up Q4_K 8960x1536, down Q4_K 1536x8960
  c4     vocabulary projection Q6_K 151936x3584, one position, then the fused
         projection + greedy argmax
  c5m8   Qwen2.5-7B-shaped decode-step set (28 layers, 4 launches each), 8
         positions per launch
  c5m32  the same set at 32 positions per launch (one prefill chunk of 32)

Usage: python3 my-inference-engine_amd/config_bench.py [--config c1,c2,...|all] [--reps N]
Prints one JSON object per configuration.
"""
import argparse
import importlib
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

Q5_0, Q8_0, Q4_K, Q6_K = 6, 8, 12, 14
NAMES = {Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}


def configs():
    l15 = [[("q", Q5_0, 1536, 1536), ("k", Q5_0, 256, 1536), ("v", Q5_0, 256, 1536)], [("o", Q5_0, 1536, 1536)],
           [("gate", Q4_K, 8960, 1536), ("up", Q4_K, 8960, 1536)], [("down", Q4_K, 1536, 8960)]]
    l7 = [[("q", Q4_K, 3584, 3584), ("k", Q4_K, 512, 3584), ("v", Q4_K, 512, 3584)], [("o", Q4_K, 3584, 3584)],
          [("gate", Q4_K, 18944, 3584), ("up", Q4_K, 18944, 3584)], [("down", Q6_K, 3584, 18944)]]
    return {
        "c1": (1, 1, [[("q", Q8_0, 896, 896)]]),
        "c2": (1, 1, [[("down", Q6_K, 896, 4864)]]),
        "c3": (8, 1, l15),
        "c4": (1, 1, [[("output", Q6_K, 151936, 3584)]]),
        "c5m8": (8, 28, l7),
        "c5m32": (32, 28, l7),
    }


def run_config(qmv, hip, name, reps):
    positions, layers, groups = configs()[name]
    D = hip.DeviceBuffer
    stream = hip.Stream()
    sp = stream.handle
    seed = 0 if name == "c1" else 100 * (1 + list(configs()).index(name))
    raws = {}
    for li in range(layers):
        for g in groups:
            for tname, t, rows, cols in g:
                raws[(li, tname)] = qmv.synth_tensor(t, rows, cols, seed=seed)
                seed += 1
    nbytes = sum(r.size for r in raws.values())
    copies = 1 if nbytes >= (1 << 30) else -(-(1 << 30) // nbytes)
    sets = [{k: qmv.DeviceTensor(qmv.make_view(raws[k], t, rows, cols))
             for li in range(layers) for g in groups for (tname, t, rows, cols) in g for k in [(li, tname)]}
            for _ in range(copies)]
    del raws
    xs = [[D.from_array(qmv.synth_normal(positions * g[0][3], seed=7000 + 10 * li + j)) for j, g in enumerate(groups)]
          for li in range(layers)]
    ys = [[[D(4 * positions * r) for _, _, r, _ in g] for g in groups] for _ in range(layers)]

    def one_pass(ts):
        for li in range(layers):
            for j, g in enumerate(groups):
                qmv.device_matvec_group([ts[(li, tname)] for tname, _, _, _ in g], xs[li][j].ptr, positions,
                                        [y.ptr for y in ys[li][j]], sp)

    for c in range(min(2, copies)):
        one_pass(sets[c])
    stream.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(stream)
    for i in range(reps):
        one_pass(sets[i % copies])
    e1.record(stream)
    stream.synchronize()
    us = e0.elapsed_ms(e1) / reps * 1e3
    flops = 2 * positions * layers * sum(r * c for g in groups for _, _, r, c in g)
    out = {"config": name, "positions": positions, "layers": layers, "launches_per_pass": layers * len(groups),
           "packed_bytes": nbytes, "copies": copies, "reps": reps, "us_per_pass": round(us, 2),
           "weight_gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "fp32_tflops": round(flops / (us * 1e-6) / 1e12, 2)}
    if name == "c4":
        ts = sets[0]
        res = D(8)
        logits = ys[0][0][0]
        qmv.device_matvec_argmax(ts[(0, "output")], xs[0][0].ptr, logits.ptr, res.ptr, sp)
        stream.synchronize()
        e0.record(stream)
        for _ in range(reps):
            qmv.device_matvec_argmax(ts[(0, "output")], xs[0][0].ptr, logits.ptr, res.ptr, sp)
        e1.record(stream)
        stream.synchronize()
        out["fused_argmax_us"] = round(e0.elapsed_ms(e1) / reps * 1e3, 2)
    if name == "c2":
        import numpy as np
        raw = qmv.synth_tensor(Q4_K, 4864, 1024, seed=1)  # bytes only: the view claims 896 columns
        v = qmv.make_view(raw, Q4_K, 4864, 896)
        y = np.empty(4864, dtype=np.float32)
        out["q4_k_4864x896_rejected"] = qmv.quantized_tensor_matvec_f32(v, np.zeros(896, np.float32), 896, y, 4864) == 0
    e0.destroy()
    e1.destroy()
    for ts in sets:
        for d in ts.values():
            d.close()
    stream.destroy()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="all", help="comma-separated names, or all")
    ap.add_argument("--reps", type=int, default=50)
    args = ap.parse_args()
    names = list(configs()) if args.config == "all" else args.config.split(",")
    for n in names:
        if n not in configs():
            print(f"unknown configuration {n}; choose from {', '.join(configs())}", file=sys.stderr)
            sys.exit(2)
    qmv = importlib.import_module("my-inference-engine_amd")
    hip = importlib.import_module("my-inference-engine_amd.hip_runtime")
    if qmv.hip_lib().qmv_device_count() <= 0 or qmv.hip_lib().qmv_set_device(0) != 1:
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    for n in names:
        print(f"config {n}: running", file=sys.stderr, flush=True)
        print(json.dumps(run_config(qmv, hip, n, max(1, args.reps))), flush=True)


if __name__ == "__main__":
    main()
