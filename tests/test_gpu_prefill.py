"""GPU parity of prefill batches of more than 8 positions (the reference
prefills in chunks of QWEN2_PREFILL_CHUNK_SIZE = 8, src/qwen2_internal.h:7,
through quantized_tensor_matmul_f32, src/quantized_matvec.cpp:164-224).
Q4_K and Q6_K batches of 9..32 positions run as one launch of the prefill
kernel (four tiles per workgroup sharing activations staged in LDS, two
position blocks of 16 per decoded code tile); larger batches and the other
formats run as consecutive launches.

Bars: every row of every position within 1e-5 * sum |w x| of the oracle;
and, because a position's arithmetic in the prefill kernel does not depend
on the other positions of its launch, a launch is bit-identical to the same
positions run in smaller prefill launches.
"""
import os

import numpy as np
import pytest

import _blocks as B

pytestmark = pytest.mark.gpu

TOL = 1e-5


def log(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def hip(qmv):
    import importlib
    return importlib.import_module("my-inference-engine_amd.hip_runtime")


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _check(oracle, raw, t, rows, cols, x, y, what):
    worst = 0.0
    for b in range(x.shape[0]):
        y_ref = oracle.matvec(raw, t, rows, cols, x[b])
        _, absdot = oracle.row_stats(raw, t, rows, cols, x[b])
        err = np.abs(y[b].astype(np.float64) - y_ref)
        assert (err <= TOL * absdot).all(), f"{what}: position {b}"
        worst = max(worst, float(np.max(err / np.maximum(absdot, 1e-300))))
    log(f"{what}: worst err/sum|wx| {worst:.2e}")


@pytest.mark.parametrize("t", [B.Q4_K, B.Q6_K, B.Q8_0, B.Q5_0])
@pytest.mark.parametrize("batch", [9, 16, 17, 32, 33, 40])
def test_prefill_batches_match_oracle(qmv, oracle, gpu, t, batch):
    rows = 200
    cols = 5 * B.BLOCK_ELEMENTS[t] if t in (B.Q4_K, B.Q6_K) else 7 * 32 + 512
    raw = qmv.synth_tensor(t, rows, cols, seed=300 + batch)
    x = qmv.synth_normal(batch * cols, seed=301 + batch).reshape(batch, cols)
    v = qmv.make_view(raw, t, rows, cols)
    y = qmv.matvec(v, x)
    _check(oracle, raw, t, rows, cols, x, y, f"type {t} {rows}x{cols} B={batch}")
    qmv.release_tensor(v.data)


@pytest.mark.parametrize("t,rows,cols", [(B.Q4_K, 18944, 3584), (B.Q6_K, 3584, 18944), (B.Q4_K, 3584, 3584),
                                         (B.Q4_K, 512, 3584), (B.Q4_K, 8960, 1536), (B.Q5_0, 1536, 1536),
                                         (B.Q5_0, 256, 1536), (B.Q8_0, 896, 896), (B.Q8_0, 4864, 896)])
def test_prefill_32_at_layer_shapes(qmv, oracle, gpu, t, rows, cols):
    batch = 32
    raw = qmv.synth_tensor(t, rows, cols, seed=310)
    x = qmv.synth_normal(batch * cols, seed=311).reshape(batch, cols)
    v = qmv.make_view(raw, t, rows, cols)
    y = qmv.matvec(v, x)
    _check(oracle, raw, t, rows, cols, x, y, f"type {t} {rows}x{cols} B=32")
    qmv.release_tensor(v.data)


@pytest.mark.parametrize("t,rows,cols", [(B.Q8_0, 896, 4864), (B.Q5_0, 1536, 8960), (B.Q8_0, 200, 32 * 131),
                                         (B.Q5_0, 130, 32 * 133)])
@pytest.mark.parametrize("batch", [16, 27, 32])
def test_prefill_long_rows_q5_q8(qmv, oracle, gpu, t, rows, cols, batch):
    """Q8_0 / Q5_0 prefill launches over rows of 32 or more four-block units
    (K >= 4096), where the plan takes two units per split for launches of at
    most 8 tile groups and five otherwise; two shapes end in a partial last
    unit (131 and 133 blocks). The first two shapes split K 19 and 35 ways, so
    their launches finish in the reduction kernel (pf_reduce_kernel) at every
    batch here, 16 position rows included."""
    raw = qmv.synth_tensor(t, rows, cols, seed=340 + batch)
    x = qmv.synth_normal(batch * cols, seed=341 + batch).reshape(batch, cols)
    v = qmv.make_view(raw, t, rows, cols)
    y = qmv.matvec(v, x)
    _check(oracle, raw, t, rows, cols, x, y, f"type {t} {rows}x{cols} B={batch}")
    qmv.release_tensor(v.data)


@pytest.mark.parametrize("t", [B.Q4_K, B.Q6_K, B.Q5_0, B.Q8_0])
@pytest.mark.parametrize("batch,parts", [(32, [16, 16]), (27, [9, 18]), (24, [12, 12]), (30, [10, 10, 10])])
def test_prefill_positions_independent(qmv, gpu, hip, t, batch, parts):
    """One prefill launch of `batch` positions against the same positions in
    smaller prefill launches (each of 9 or more positions), on device
    buffers: bit-identical, since a position's arithmetic does not depend on
    the other positions of its launch."""
    knob = {B.Q5_0: "QMV_Q5_PREFILL", B.Q8_0: "QMV_Q8_PREFILL"}.get(t)
    if knob and os.environ.get(knob) == "0":
        pytest.skip(f"{knob}=0 runs these batches in launches of at most 8 positions")
    rows, cols = 1000, 3584
    raw = qmv.synth_tensor(t, rows, cols, seed=320)
    dt = qmv.DeviceTensor(qmv.make_view(raw, t, rows, cols))
    x = qmv.synth_normal(batch * cols, seed=321)
    dx = hip.DeviceBuffer.from_array(x)
    wide = hip.DeviceBuffer(4 * batch * rows)
    narrow = hip.DeviceBuffer(4 * batch * rows)
    s = hip.Stream()
    dt.matvec(dx.ptr, batch, wide.ptr, s.handle)
    b0 = 0
    for n in parts:
        dt.matvec(dx.ptr + 4 * b0 * cols, n, narrow.ptr + 4 * b0 * rows, s.handle)
        b0 += n
    s.synchronize()
    assert np.array_equal(_bits(wide.to_array(np.float32, (batch, rows))),
                          _bits(narrow.to_array(np.float32, (batch, rows))))
    dt.close()


@pytest.mark.parametrize("cols,batch", [(3584, 27), (1024, 27), (7936, 12), (3584, 12)],
                         ids=["32rows-reduction-kernel", "32rows-in-kernel", "16rows-reduction-kernel",
                              "16rows-in-kernel"])
def test_prefill_epilogues(qmv, oracle, gpu, hip, cols, batch):
    """Bias addend and fused SwiGLU on prefill launches (the positions past
    the batch inside the kernel's position blocks are never stored), for both
    split-K finishes: in the reduction kernel (pf_reduce_kernel) where the
    in-kernel finish would take 5 or more rounds of partial loads (K = 3584:
    14 splits at 32 position rows, 7 rounds; K = 7936: 31 splits at 16, 8
    rounds), and inside the prefill kernel with its SwiGLU pair protocol
    otherwise (K = 1024: 4 splits; K = 3584 at 16 position rows: 4 rounds)."""
    t, rows = B.Q4_K, 1000
    raw_g = qmv.synth_tensor(t, rows, cols, seed=330)
    raw_u = qmv.synth_tensor(t, rows, cols, seed=331)
    dg = qmv.DeviceTensor(qmv.make_view(raw_g, t, rows, cols))
    du = qmv.DeviceTensor(qmv.make_view(raw_u, t, rows, cols))
    x = qmv.synth_normal(batch * cols, seed=332).reshape(batch, cols)
    dx = hip.DeviceBuffer.from_array(x)
    s = hip.Stream()
    g, u = hip.DeviceBuffer(4 * (batch + 5) * rows), hip.DeviceBuffer(4 * batch * rows)
    g.fill(0x7f)  # sentinel rows past the batch must survive
    qmv.device_matvec_group([dg, du], dx.ptr, batch, [g.ptr, u.ptr], s.handle)
    s.synchronize()
    gate = g.to_array(np.float32, (batch + 5, rows))
    assert np.all(_bits(gate[batch:]) == 0x7f7f7f7f)
    gate, up = gate[:batch], u.to_array(np.float32, (batch, rows))
    _check(oracle, raw_g, t, rows, cols, x, gate, f"gate B={batch}")
    bias = np.random.default_rng(333).standard_normal(rows).astype(np.float32)
    db = hip.DeviceBuffer.from_array(bias)
    out = hip.DeviceBuffer(4 * batch * rows)
    qmv.device_matvec_add_group([dg], dx.ptr, batch, [db.ptr], [0], [out.ptr], s.handle)
    act = hip.DeviceBuffer(4 * batch * rows)
    qmv.device_matvec_swiglu(dg, du, dx.ptr, batch, act.ptr, s.handle)
    s.synchronize()
    assert np.array_equal(_bits(out.to_array(np.float32, (batch, rows))), _bits(gate + bias[None, :]))
    got = act.to_array(np.float32, (batch, rows))
    for b in range(batch):
        ok, ref = oracle.swiglu(gate[b], up[b])
        assert ok == 1
        assert (np.abs(got[b].astype(np.float64) - ref) <= 4 * 2.0 ** -23 * np.abs(ref) + 1e-30).all(), b
    dg.close()
    du.close()


@pytest.mark.parametrize("t", [B.Q4_K, B.Q6_K])
@pytest.mark.parametrize("batch", [27, 32])
def test_prefill_group_of_unequal_tensors(qmv, oracle, gpu, hip, t, batch):
    """A grouped launch of three tensors of unequal rows (17, 2 and 1 tiles,
    the last two partial) over K = 3584 (14 splits): its partials finish in
    the reduction kernel, which finds each thread's tensor from the tile
    counts. Every tensor within the row bar of the oracle and bit-identical
    to the same tensor launched alone."""
    rows, cols = [1030, 100, 7], 3584
    raws = [qmv.synth_tensor(t, r, cols, seed=380 + i) for i, r in enumerate(rows)]
    dts = [qmv.DeviceTensor(qmv.make_view(raw, t, r, cols)) for raw, r in zip(raws, rows)]
    x = qmv.synth_normal(batch * cols, seed=383).reshape(batch, cols)
    dx = hip.DeviceBuffer.from_array(x)
    s = hip.Stream()
    grouped = [hip.DeviceBuffer(4 * batch * r) for r in rows]
    alone = [hip.DeviceBuffer(4 * batch * r) for r in rows]
    qmv.device_matvec_group(dts, dx.ptr, batch, [y.ptr for y in grouped], s.handle)
    for dt, y in zip(dts, alone):
        dt.matvec(dx.ptr, batch, y.ptr, s.handle)
    s.synchronize()
    for raw, r, yg, ya in zip(raws, rows, grouped, alone):
        a = yg.to_array(np.float32, (batch, r))
        assert np.array_equal(_bits(a), _bits(ya.to_array(np.float32, (batch, r)))), f"{r} rows"
        _check(oracle, raw, t, r, cols, x, a, f"type {t} group member {r}x{cols} B={batch}")
    for dt in dts:
        dt.close()


def test_prefill_graph_replay(qmv, gpu, hip):
    t, rows, cols, batch = B.Q6_K, 3584, 18944, 32
    raw = qmv.synth_tensor(t, rows, cols, seed=340)
    dt = qmv.DeviceTensor(qmv.make_view(raw, t, rows, cols))
    dx = hip.DeviceBuffer.from_array(qmv.synth_normal(batch * cols, seed=341))
    dy = hip.DeviceBuffer(4 * batch * rows)
    s = hip.Stream()
    dt.matvec(dx.ptr, batch, dy.ptr, s.handle)
    s.synchronize()
    eager = dy.to_array(np.float32, (batch * rows,))
    g = hip.Graph(s)
    g.begin()
    dt.matvec(dx.ptr, batch, dy.ptr, s.handle)
    g.end()
    for i in range(3):
        dy.fill(0)
        g.replay()
        s.synchronize()
        assert np.array_equal(_bits(dy.to_array(np.float32, (batch * rows,))), _bits(eager)), i
        dt.matvec(dx.ptr, batch, dy.ptr, s.handle)
        s.synchronize()
    dt.close()


def test_device_batch_limit(qmv, gpu, hip):
    raw = qmv.synth_tensor(B.Q4_K, 64, 256, seed=350)
    dt = qmv.DeviceTensor(qmv.make_view(raw, B.Q4_K, 64, 256))
    dx = hip.DeviceBuffer(4 * 33 * 256)
    dy = hip.DeviceBuffer(4 * 33 * 64)
    with pytest.raises(qmv.QmvError):
        dt.matvec(dx.ptr, 33, dy.ptr, 0)
    dt.close()


@pytest.mark.parametrize("t", [B.Q4_K, B.Q6_K, B.Q5_0, B.Q8_0])
@pytest.mark.parametrize("rows,cols,batch", [(1, 256, 9), (63, 512, 32), (130, 256, 17), (65, 2304, 12),
                                             (257, 1024, 31)])
def test_prefill_edge_shapes(qmv, oracle, gpu, t, rows, cols, batch):
    """Tile groups with idle waves (1, 2 or 3 of 4 tiles real), partial last
    tiles, a single K-unit, and odd position counts."""
    raw = qmv.synth_tensor(t, rows, cols, seed=360 + rows)
    x = qmv.synth_normal(batch * cols, seed=361 + rows).reshape(batch, cols)
    v = qmv.make_view(raw, t, rows, cols)
    y = qmv.matvec(v, x)
    _check(oracle, raw, t, rows, cols, x, y, f"type {t} {rows}x{cols} B={batch}")
    qmv.release_tensor(v.data)


@pytest.mark.parametrize("t", [B.Q5_0, B.Q8_0])
@pytest.mark.parametrize("rows,cols,batch", [(130, 96, 17), (65, 7 * 32 + 512, 12), (200, 32, 32), (64, 1568, 25)])
def test_prefill_partial_units(qmv, oracle, gpu, t, rows, cols, batch):
    """Q5_0 / Q8_0 rows whose last 4-block unit is partial (K = 32 * odd):
    the blocks past K are skipped and no activation past K is read."""
    raw = qmv.synth_tensor(t, rows, cols, seed=370 + rows)
    x = qmv.synth_normal(batch * cols, seed=371 + rows).reshape(batch, cols)
    v = qmv.make_view(raw, t, rows, cols)
    y = qmv.matvec(v, x)
    _check(oracle, raw, t, rows, cols, x, y, f"type {t} {rows}x{cols} B={batch}")
    qmv.release_tensor(v.data)


def test_prefill_group_with_biases(qmv, oracle, gpu, hip):
    """q/k/v of different row counts in one prefill launch (jobs with 6, 1
    and 1 tile groups), each with its bias, at 24 positions."""
    t, cols, batch = B.Q4_K, 1536, 24
    shapes = [1536, 256, 256]
    raws = [qmv.synth_tensor(t, r, cols, seed=370 + i) for i, r in enumerate(shapes)]
    dts = [qmv.DeviceTensor(qmv.make_view(raw, t, r, cols)) for raw, r in zip(raws, shapes)]
    x = qmv.synth_normal(batch * cols, seed=373).reshape(batch, cols)
    dx = hip.DeviceBuffer.from_array(x)
    rng = np.random.default_rng(374)
    biases = [rng.standard_normal(r).astype(np.float32) for r in shapes]
    dbs = [hip.DeviceBuffer.from_array(b) for b in biases]
    plain = [hip.DeviceBuffer(4 * batch * r) for r in shapes]
    biased = [hip.DeviceBuffer(4 * batch * r) for r in shapes]
    s = hip.Stream()
    qmv.device_matvec_group(dts, dx.ptr, batch, [o.ptr for o in plain], s.handle)
    qmv.device_matvec_add_group(dts, dx.ptr, batch, [b.ptr for b in dbs], [0, 0, 0], [o.ptr for o in biased],
                                s.handle)
    s.synchronize()
    for raw, r, p_, b_, bias in zip(raws, shapes, plain, biased, biases):
        yp = p_.to_array(np.float32, (batch, r))
        _check(oracle, raw, t, r, cols, x, yp, f"group rows {r} B={batch}")
        assert np.array_equal(_bits(b_.to_array(np.float32, (batch, r))), _bits(yp + bias[None, :]))
    for d in dts:
        d.close()
