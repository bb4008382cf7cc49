"""HBM probes (libqmv_probe.so): measured streaming-read bandwidth, and a
plain copy of known size for calibrating rocprofv3's FETCH_SIZE / WRITE_SIZE.

    python3 my-inference-engine_amd/probe.py read [--mib 1024] [--blocks 512]
    python3 my-inference-engine_amd/probe.py copy [--mib 512] [--reps 1]

read_chain_us() (used by bench.py) gives the streaming floor of a sequence
of launches.

Each prints one JSON line. Measurement tooling only; the matvec path does not
use it.
"""
import argparse
import ctypes
import json
import os

CSRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc")
PROBE_LIB_PATH = os.path.join(CSRC, "libqmv_probe.so")
_lib = None


def probe_lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(PROBE_LIB_PATH):
            raise RuntimeError(f"{PROBE_LIB_PATH} is missing: run __graft_entry__.build()")
        lib = ctypes.CDLL(PROBE_LIB_PATH)
        lib.qmv_probe_read.restype = ctypes.c_int
        lib.qmv_probe_read.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                       ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_uint64)]
        lib.qmv_probe_copy.restype = ctypes.c_int
        lib.qmv_probe_copy.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
        lib.qmv_probe_read_chain.restype = ctypes.c_int
        lib.qmv_probe_read_chain.argtypes = [ctypes.POINTER(ctypes.c_uint64), ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
        _lib = lib
    return _lib


def read_bandwidth(nbytes: int = 1 << 30, blocks: int = 512, reps: int = 10) -> dict:
    """Streaming read of one buffer larger than the 256 MB MALL, `reps` passes."""
    ms, got = ctypes.c_double(), ctypes.c_uint64()
    if probe_lib().qmv_probe_read(nbytes, blocks, reps, ctypes.byref(ms), ctypes.byref(got)) != 1:
        raise RuntimeError("qmv_probe_read failed")
    return {"probe": "read", "bytes": got.value, "blocks": blocks, "threads": 256, "reps": reps,
            "us_per_pass": round(ms.value * 1e3, 3), "gbs": round(got.value / (ms.value * 1e-3) / 1e9, 1)}


def copy_pass(nbytes: int = 512 << 20, reps: int = 1) -> dict:
    ms = ctypes.c_double()
    if probe_lib().qmv_probe_copy(nbytes, reps, ctypes.byref(ms)) != 1:
        raise RuntimeError("qmv_probe_copy failed")
    return {"probe": "copy", "bytes_read": nbytes, "bytes_written": nbytes, "reps": reps,
            "us_per_pass": round(ms.value * 1e3, 3), "gbs": round(2 * nbytes / (ms.value * 1e-3) / 1e9, 1)}


def read_chain_us(sizes, reps: int = 20, pers=(1, 2, 4, 8)) -> float:
    """Streaming floor of a launch sequence: microseconds per replay of a
    graph of dependent read-only launches over distinct buffers of `sizes`
    bytes, each read once by threads that issue `per` 16-byte loads at once
    (the fastest of the `pers` tried)."""
    arr = (ctypes.c_uint64 * len(sizes))(*sizes)
    best = None
    for per in pers:
        us = ctypes.c_double()
        if probe_lib().qmv_probe_read_chain(arr, len(sizes), per, reps, ctypes.byref(us)) != 1:
            raise RuntimeError("qmv_probe_read_chain failed")
        best = us.value if best is None else min(best, us.value)
    return best


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("kind", choices=["read", "copy"])
    ap.add_argument("--mib", type=int, default=None)
    ap.add_argument("--blocks", type=int, default=512)
    ap.add_argument("--reps", type=int, default=None)
    a = ap.parse_args()
    if a.kind == "read":
        r = read_bandwidth((a.mib or 1024) << 20, a.blocks, a.reps or 10)
    else:
        r = copy_pass((a.mib or 512) << 20, a.reps or 1)
    print(json.dumps(r), flush=True)


if __name__ == "__main__":
    main()
