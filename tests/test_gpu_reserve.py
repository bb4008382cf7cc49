"""GPU checks of the allocation contract and of workspace lifetime.

* After qmv_reserve_calls, host-pointer matvec/matmul calls of 1..32
  positions allocate nothing (the reference's contracts: the matvec itself
  allocates nothing, src/quantized_matvec.h:24, and a forward pass allocates
  nothing after state init, include/engine.h:84-85), and still match the
  oracle within the row tolerance.
* That holds on every OS thread, not only the one that reserved: a session
  may be created on one thread and run on others (include/engine_api.h:12-13;
  the Go server's cgo calls, server/engine/engine.go:181,238, land on
  whatever thread the Go runtime picks). Calls from new threads, from the
  reserving thread, and from several threads at once (waiting for a pooled
  context, or on the declared number of contexts) allocate nothing.
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


THREAD_SHAPES = [(B.Q4_K, 3584, 3584), (B.Q6_K, 896, 4864), (B.Q5_0, 1536, 1536), (B.Q8_0, 896, 896)]
THREAD_BATCHES = (1, 2, 5, 8, 9, 16, 32)


def _thread_cases(qmv, oracle):
    """Reserved views with their inputs (32 positions) and oracle rows."""
    cases = []
    for i, (t, rows, cols) in enumerate(THREAD_SHAPES):
        raw = qmv.synth_tensor(t, rows, cols, seed=700 + i)
        v = qmv.make_view(raw, t, rows, cols)
        x = qmv.synth_normal(32 * cols, seed=710 + i).reshape(32, cols)
        y_ref = np.asarray(oracle.matvec(raw, t, rows, cols, x), np.float64).reshape(32, rows)
        absdot = np.stack([oracle.row_stats(raw, t, rows, cols, x[b])[1] for b in range(32)])
        cases.append((t, rows, cols, raw, v, x, y_ref, absdot))
    return cases


def _run_cases(qmv, cases, tag, errors):
    """Every case at every batch in THREAD_BATCHES; failures go to errors."""
    try:
        for t, rows, cols, raw, v, x, y_ref, absdot in cases:
            for m in THREAD_BATCHES:
                y = qmv.matvec(v, x[:m] if m > 1 else x[0]).reshape(m, rows)
                err = np.abs(y.astype(np.float64) - y_ref[:m])
                bad = err > TOL * absdot[:m]
                if bad.any():
                    errors.append(f"{tag}: {B.NAMES[t]} {rows}x{cols} M={m}: {int(bad.sum())} rows over tolerance")
    except Exception as e:  # noqa: BLE001 - reported by the main thread
        errors.append(f"{tag}: {e!r}")


def _in_threads(qmv, cases, tags):
    import threading
    errors = []
    threads = [threading.Thread(target=_run_cases, args=(qmv, cases, tag, errors)) for tag in tags]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors


def test_reservation_holds_on_every_thread(qmv, oracle, gpu):
    """Reserve on this thread (A); then calls of 1..32 positions from new
    threads B and C one after the other, from A, from 4 threads at once (the
    pool may hold fewer contexts: callers wait, they do not allocate), and,
    after declaring 4 concurrent callers, from 4 threads at once again. The
    allocation count stays put except for the declaration itself."""
    cases = _thread_cases(qmv, oracle)
    for _, _, _, _, v, *_ in cases:
        qmv.reserve_calls(v, 32)
    before = qmv.allocation_count()
    log(f"allocations after reserve on thread A: {before}")
    _in_threads(qmv, cases, ["B"])
    _in_threads(qmv, cases, ["C"])
    log("threads B and C: M=1..32, within tolerance")
    errors = []
    _run_cases(qmv, cases, "A", errors)
    assert not errors, errors
    _in_threads(qmv, cases, ["D0", "D1", "D2", "D3"])
    assert qmv.allocation_count() == before, "a call on another thread allocated after the reservation"
    log("thread A and 4 concurrent threads: no allocation")
    qmv.reserve_contexts(4)
    declared = qmv.allocation_count()
    _in_threads(qmv, cases, ["E0", "E1", "E2", "E3"])
    _in_threads(qmv, cases, ["F0", "F1", "F2", "F3", "F4", "F5"])
    assert qmv.allocation_count() == declared, "concurrent calls allocated after declaring 4 callers"
    log("4 declared contexts: 4 and 6 concurrent threads, no allocation")
    for _, _, _, _, v, *_ in cases:
        qmv.release_tensor(v.data)


def test_reserve_rejects_bad_arguments(qmv, gpu):
    raw = qmv.synth_tensor(B.Q8_0, 64, 256, seed=1)
    v = qmv.make_view(raw, B.Q8_0, 64, 256)
    assert qmv.hip_lib().qmv_reserve_calls(v, 0) == 0
    bad = qmv.make_view(raw, B.Q8_0, 64, 256)
    bad.block_bytes = 33
    assert qmv.hip_lib().qmv_reserve_calls(bad, 4) == 0
    assert qmv.hip_lib().qmv_reserve_contexts(0) == 0
    assert qmv.hip_lib().qmv_reserve_contexts(1025) == 0


def test_graph_survives_workspace_growth(qmv, gpu, hip):
    """Capture a split-K launch (Q6_K 3584 x 18944 at M = 1, uploaded with the
    row-major kernels off so it runs tiled: 56 tiles in 13 K-splits) on a
    fresh stream, then run a 32-position launch of the same tensor eagerly on
    that stream (its workspace grows past the captured one), then replay:
    the replays still match the eager M = 1 bits."""
    rows, cols = 3584, 18944
    big = qmv.synth_tensor(B.Q6_K, rows, cols, seed=72)
    qmv.set_rowmajor(False, 2)
    try:
        db = qmv.DeviceTensor(qmv.make_view(big, B.Q6_K, rows, cols))
    finally:
        qmv.set_rowmajor(True, 2)
    x = qmv.synth_normal(32 * cols, seed=73)
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(4 * rows)
    dbig = hip.DeviceBuffer(4 * rows * 32)
    with hip.Stream() as stream:
        first = qmv.allocation_count()
        db.matvec(dx.ptr, 1, dy.ptr, stream.handle)
        stream.synchronize()
        assert qmv.allocation_count() > first, "the M = 1 launch was expected to use the stream's workspace"
        eager = dy.to_array(np.float32, (rows,))
        with hip.Graph(stream) as g:
            g.begin()
            db.matvec(dx.ptr, 1, dy.ptr, stream.handle)
            g.end()
            before = qmv.allocation_count()
            db.matvec(dx.ptr, 32, dbig.ptr, stream.handle)
            stream.synchronize()
            assert qmv.allocation_count() > before, "the 32-position call was expected to grow the workspace"
            for i in range(4):
                dy.fill(0)
                g.replay()
                stream.synchronize()
                assert np.array_equal(dy.to_array(np.float32, (rows,)).view(np.uint32), eager.view(np.uint32)), i
                db.matvec(dx.ptr, 32, dbig.ptr, stream.handle)
                stream.synchronize()
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
