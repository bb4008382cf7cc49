"""GPU checks of the allocation contract and of workspace lifetime.

* After qmv_reserve_calls, host-pointer matvec/matmul calls of 1..32
  positions allocate nothing (the reference's contracts: the matvec itself
  allocates nothing, src/quantized_matvec.h:24, and a forward pass allocates
  nothing after state init, include/engine.h:84-85), and still match the
  oracle within the row tolerance.
* A graph captured on a stream keeps working after a larger eager call on the
  same stream has grown that stream's workspace.
* Small tensors are fingerprinted over every byte, so a one-block edit in
  place is seen.
"""
import numpy as np
import pytest

import _blocks as B

pytestmark = pytest.mark.gpu

TOL = 1e-5


def log(msg):
    print(msg, flush=True)


def check_rows(y, y_ref, absdot, what):
    err = np.abs(np.asarray(y, np.float64) - np.asarray(y_ref, np.float64))
    bad = err > TOL * np.asarray(absdot, np.float64)
    assert not bad.any(), f"{what}: {int(bad.sum())} rows over tolerance"


@pytest.fixture(scope="module")
def hip(qmv):
    import importlib
    return importlib.import_module("my-inference-engine_amd.hip_runtime")


SHAPES = [(B.Q4_K, 3584, 3584), (B.Q6_K, 896, 4864), (B.Q8_0, 896, 896), (B.Q5_0, 1536, 1536),
          (B.Q4_K, 1000, 2304)]


def test_reserved_calls_allocate_nothing(qmv, oracle, gpu):
    tensors = []
    for i, (t, rows, cols) in enumerate(SHAPES):
        raw = qmv.synth_tensor(t, rows, cols, seed=300 + i)
        v = qmv.make_view(raw, t, rows, cols)
        qmv.reserve_calls(v, 32)
        tensors.append((t, rows, cols, raw, v))
    before = qmv.allocation_count()
    log(f"allocations after reserve: {before}")
    for t, rows, cols, raw, v in tensors:
        x = qmv.synth_normal(32 * cols, seed=rows + cols).reshape(32, cols)
        for m in range(1, 33):
            y = qmv.matvec(v, x[:m] if m > 1 else x[0]).reshape(m, rows)
            if m in (1, 2, 7, 8, 9, 16, 17, 27, 32):
                y_ref = oracle.matvec(raw, t, rows, cols, x[:m] if m > 1 else x[0]).reshape(m, rows)
                for b in (0, m - 1):
                    _, absdot = oracle.row_stats(raw, t, rows, cols, x[b])
                    check_rows(y[b], y_ref[b], absdot, f"{B.NAMES[t]} {rows}x{cols} M={m} pos {b}")
        assert qmv.allocation_count() == before, f"{B.NAMES[t]} {rows}x{cols} allocated after reserve"
        log(f"{B.NAMES[t]} {rows}x{cols}: M=1..32, no allocation")
    for *_, v in tensors:
        qmv.release_tensor(v.data)


def test_reserve_rejects_bad_arguments(qmv, gpu):
    raw = qmv.synth_tensor(B.Q8_0, 64, 256, seed=1)
    v = qmv.make_view(raw, B.Q8_0, 64, 256)
    assert qmv.hip_lib().qmv_reserve_calls(v, 0) == 0
    bad = qmv.make_view(raw, B.Q8_0, 64, 256)
    bad.block_bytes = 33
    assert qmv.hip_lib().qmv_reserve_calls(bad, 4) == 0


def test_graph_survives_workspace_growth(qmv, gpu, hip):
    """Capture an M = 1 launch on a fresh stream, then run a 32-position
    launch of a larger tensor eagerly on the same stream (its workspace grows),
    then replay: the replays still match the eager M = 1 bits."""
    small = qmv.synth_tensor(B.Q4_K, 3584, 3584, seed=71)
    big = qmv.synth_tensor(B.Q4_K, 18944, 3584, seed=72)
    ds = qmv.DeviceTensor(qmv.make_view(small, B.Q4_K, 3584, 3584))
    db = qmv.DeviceTensor(qmv.make_view(big, B.Q4_K, 18944, 3584))
    x = qmv.synth_normal(32 * 3584, seed=73)
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(4 * 3584)
    dbig = hip.DeviceBuffer(4 * 18944 * 32)
    with hip.Stream() as stream:
        ds.matvec(dx.ptr, 1, dy.ptr, stream.handle)
        stream.synchronize()
        eager = dy.to_array(np.float32, (3584,))
        with hip.Graph(stream) as g:
            g.begin()
            ds.matvec(dx.ptr, 1, dy.ptr, stream.handle)
            g.end()
            before = qmv.allocation_count()
            db.matvec(dx.ptr, 32, dbig.ptr, stream.handle)
            stream.synchronize()
            assert qmv.allocation_count() > before, "the large call was expected to grow the workspace"
            for i in range(4):
                dy.fill(0)
                g.replay()
                stream.synchronize()
                assert np.array_equal(dy.to_array(np.float32, (3584,)).view(np.uint32), eager.view(np.uint32)), i
                db.matvec(dx.ptr, 32, dbig.ptr, stream.handle)
                stream.synchronize()
    ds.close()
    db.close()


def test_small_tensor_edit_in_place_is_seen(qmv, gpu):
    """A tensor of at most 64 KiB is fingerprinted over every byte: changing
    one block's scale in place gives the new product without a release."""
    t, rows, cols = B.Q8_0, 64, 512
    buf = qmv.synth_tensor(t, rows, cols, seed=5)
    assert buf.nbytes <= 64 << 10
    v = qmv.make_view(buf, t, rows, cols)
    x = qmv.synth_normal(cols, seed=6)
    y1 = qmv.matvec(v, x)
    blk = 37 * (cols // 32) + 3  # row 37, block 3
    off = blk * 34
    buf[off:off + 2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    y2 = qmv.matvec(v, x)
    changed = np.nonzero(y1 != y2)[0].tolist()
    assert changed == [37], changed
    qmv.release_tensor(v.data)
