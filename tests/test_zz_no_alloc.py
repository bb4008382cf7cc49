"""The no-allocation grouped matvec (qmv_device_matvec_group_noalloc_f32)
against the allocating one it varies (qmv_device_matvec_group_f32), through
the C ABI: the same launches, so the outputs must be bit-identical.

Covered: two calls in a row with the second smaller (the scratch array keeps
the first call's contents), a grouped launch, prefill-sized and single
position launches, the largest single-position shape (151936 x 3584), a call
too large for the scratch (rejected, nothing written), graph capture with
replays, and no allocation by any of these calls.
"""
import ctypes

import numpy as np
import pytest

import _blocks as B

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def hip(qmv):
    import importlib
    return importlib.import_module("my-inference-engine_amd.hip_runtime")


def _tensors(qmv, t, shapes, cols, seed):
    raws = [qmv.synth_tensor(t, r, cols, seed=seed + i) for i, r in enumerate(shapes)]
    return [qmv.DeviceTensor(qmv.make_view(raw, t, r, cols)) for raw, r in zip(raws, shapes)]


def _run_both(qmv, hip, dts, batch, seed, stream):
    """Outputs of the allocating and the no-allocation call, same inputs."""
    cols = dts[0].cols
    x = qmv.synth_normal(batch * cols, seed=seed)
    dx = hip.DeviceBuffer.from_array(x)
    ref = [hip.DeviceBuffer(4 * batch * d.rows) for d in dts]
    got = [hip.DeviceBuffer(4 * batch * d.rows) for d in dts]
    for g in got:
        g.fill(0xFF)
    qmv.device_matvec_group(dts, dx.ptr, batch, [r.ptr for r in ref], stream.handle)
    stream.synchronize()
    before = qmv.allocation_count()
    qmv.device_matvec_group_noalloc(dts, dx.ptr, batch, [g.ptr for g in got], stream.handle)
    stream.synchronize()
    assert qmv.allocation_count() == before, "the no-allocation call allocated"
    out = []
    for d, r, g in zip(dts, ref, got):
        a = r.to_array(np.float32, (batch * d.rows,))
        b = g.to_array(np.float32, (batch * d.rows,))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{d.rows}x{d.cols} M={batch}"
        out.append(b)
    return out


def test_two_calls_second_smaller(qmv, gpu, hip):
    """A grouped 8-position call, then a single-position call on smaller
    tensors, then a 32-position prefill call and a 3-position call."""
    with hip.Stream() as stream:
        qkv = _tensors(qmv, B.Q4_K, [3584, 512, 512], 3584, seed=500)
        log("noalloc: Q4_K q|k|v 3584x3584 + 2x512x3584, M=8")
        _run_both(qmv, hip, qkv, 8, seed=501, stream=stream)
        small = _tensors(qmv, B.Q4_K, [512, 512], 3584, seed=510)
        log("noalloc: Q4_K 2x512x3584, M=2")
        _run_both(qmv, hip, small, 2, seed=511, stream=stream)
        gate = _tensors(qmv, B.Q4_K, [18944], 3584, seed=520)
        log("noalloc: Q4_K 18944x3584, M=32")
        _run_both(qmv, hip, gate, 32, seed=521, stream=stream)
        q8 = _tensors(qmv, B.Q8_0, [896], 896, seed=530)
        log("noalloc: Q8_0 896x896, M=3")
        _run_both(qmv, hip, q8, 3, seed=531, stream=stream)
        for d in qkv + small + gate + q8:
            d.close()


@pytest.mark.parametrize("t,rows,cols,batch", [(B.Q6_K, 3584, 18944, 1), (B.Q6_K, 1000, 3584, 1),
                                               (B.Q5_0, 1536, 1536, 6), (B.Q6_K, 896, 4864, 20),
                                               (B.Q4_K, 1000, 2304, 2)])
def test_formats_and_batches(qmv, gpu, hip, t, rows, cols, batch):
    """Q6_K 3584 x 18944 at one position runs row-major (no scratch); Q6_K
    1000 x 3584 (14 K-units, tiled) splits K at one position; Q6_K 896 x 4864
    at 20 positions splits K 19 ways and finishes in the prefill reduction
    kernel, whose partials live in the scratch array too."""
    with hip.Stream() as stream:
        dts = _tensors(qmv, t, [rows], cols, seed=rows + batch)
        log(f"noalloc: {B.NAMES[t]} {rows}x{cols}, M={batch}")
        _run_both(qmv, hip, dts, batch, seed=batch + 7, stream=stream)
        dts[0].close()


def test_vocab_shape_and_oversized_call(qmv, gpu, hip):
    """151936 x 3584 Q6_K fits for one position; at 32 positions its split-K
    partials (2374 tiles x 3 splits x 32 position rows x 64 floats, 58 MB)
    exceed the scratch, so the call fails and writes nothing."""
    rows, cols, big = 151936, 3584, 32
    with hip.Stream() as stream:
        dts = _tensors(qmv, B.Q6_K, [rows], cols, seed=540)
        log("noalloc: Q6_K 151936x3584, M=1")
        _run_both(qmv, hip, dts, 1, seed=541, stream=stream)
        x = qmv.synth_normal(big * cols, seed=542)
        dx = hip.DeviceBuffer.from_array(x)
        dy = hip.DeviceBuffer(4 * big * rows)
        dy.fill(0x7F)
        log(f"noalloc: Q6_K 151936x3584, M={big} (must be rejected)")
        h = (ctypes.c_void_p * 1)(dts[0].handle)
        o = (ctypes.c_void_p * 1)(dy.ptr)
        assert qmv.hip_lib().qmv_device_matvec_group_noalloc_f32(h, 1, dx.ptr, big, o, stream.handle) == 0
        assert "scratch" in qmv.last_error()
        stream.synchronize()
        assert np.all(dy.to_array(np.uint8, (4 * big * rows,)) == 0x7F)
        dts[0].close()


@pytest.mark.parametrize("t,rows,cols,batch", [(B.Q6_K, 1000, 3584, 1), (B.Q4_K, 3584, 3584, 8),
                                               (B.Q4_K, 3584, 3584, 1), (B.Q6_K, 896, 4864, 1)])
def test_graph_capture_and_replays(qmv, gpu, hip, t, rows, cols, batch):
    """The call captured into a graph replays to the eager bits, with eager
    work between replays. Q6_K 1000 x 3584 at one position (14 K-units,
    tiled, in splits) and Q4_K 3584 x 3584 at 8 positions split K, so their
    counters live in the scratch array and are cleared by a fill-kernel node;
    Q4_K 3584 x 3584 and Q6_K 896 x 4864 at one position run row-major with
    no split."""
    with hip.Stream() as stream:
        dts = _tensors(qmv, t, [rows], cols, seed=550 + batch)
        x = qmv.synth_normal(batch * cols, seed=551)
        dx = hip.DeviceBuffer.from_array(x)
        dy = hip.DeviceBuffer(4 * batch * rows)
        log(f"noalloc graph: {B.NAMES[t]} {rows}x{cols}, M={batch}")
        eager = _run_both(qmv, hip, dts, batch, seed=551, stream=stream)[0]
        with hip.Graph(stream) as g:
            g.begin()
            qmv.device_matvec_group_noalloc(dts, dx.ptr, batch, [dy.ptr], stream.handle)
            g.end()
            for i in range(4):
                dy.fill(0)
                g.replay()
                stream.synchronize()
                got = dy.to_array(np.float32, (batch * rows,))
                assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), i
                qmv.device_matvec_group_noalloc(dts, dx.ptr, batch, [dy.ptr], stream.handle)
                stream.synchronize()
        dts[0].close()
