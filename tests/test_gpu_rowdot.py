"""GPU parity of the row-major single-position kernels (Q4_K, and Q6_K rows
of 17 to 128 super-blocks), through the C ABI.

Q4_K tensors whose tiled plan covers at most 2048 (64-row tile, 256-weight
unit) pairs keep their GGUF bytes on the device as well, and their
single-position launches run row-major (rowgroup_q4k_kernel): a lane takes
one 64-weight group of a super-block, a row's lanes form a segment of 16, 32
or 64 lanes (rows of up to 16 super-blocks; the workgroup's 4 waves share the
activations through LDS) or span several waves (longer rows), and a row's
sums are added inside the workgroup. Every case runs with 1, 2 and 4 rows per
row segment (qmv_set_rowmajor). The bars are those of the tiled path:
  * rows: |y - y_oracle| <= 1e-5 * sum_k |w_k x_k| (the reference's scalar
    row loop, src/quantized_matvec.cpp:152-158, restated by the oracle);
  * the addend: bit-identical to the plain launch's rows plus the addend;
  * SwiGLU: bit-identical to up * silu(gate) of the plain launch's rows
    computed by the same device expression, and within 4 ulp of the
    oracle's transformer_swiglu_f32;
  * fused argmax: logits bit-identical to the plain launch, index equal to
    the greedy argmax of those logits;
  * repeated launches are bit-identical;
  * ties and non-finite logits in the fused argmax follow the reference
    sampler (src/sampler.cpp:29-51);
  * with the row-major kernel switched off, new tensors keep no GGUF copy and
    run tiled, within the same bar.
Q6_K tensors whose rows hold 17 to 128 super-blocks keep a copy in a
chunked plane layout (210 bytes per super-block, rows padded to 16 bytes)
and run their single-position launches on rowloop_q6k_kernel (one row per
wave, taken in slices of 16 super-blocks, one 64-weight item per lane; a
launch's rows, over several tensors, fill workgroups of up to 16 waves); the
same row bar, addend and repeatability checks apply.
"""
import os

import numpy as np
import pytest

import _blocks as B

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(os.environ.get("QMV_ROWDOT", "1") == "0",
                                 reason="the row-major kernel is switched off (QMV_ROWDOT=0)")]

TOL = 1e-5
SWIGLU_ULPS = 4
SMALL_UNITS = 2048  # tiled (tile, unit) pairs up to which a launch runs row-major


def log(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def hip(qmv):
    import importlib
    return importlib.import_module("my-inference-engine_amd.hip_runtime")


ROWS_PER_SEGMENT = [1, 2, 4]


@pytest.fixture(params=ROWS_PER_SEGMENT)
def seg_rows(request, qmv):
    """Rows per row segment for the launches of one test; the default (2)
    is restored afterwards."""
    qmv.set_rowmajor(True, request.param)
    yield request.param
    qmv.set_rowmajor(True, 2)


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _tiled_units(rows, cols):
    return -(-rows // 64) * (cols // 256)


def _keeps_copy(rows, cols):
    """Launches of up to 2048 tiled pairs, rows of up to 128 super-blocks; any
    size with rows of up to 16 super-blocks."""
    sb = cols // 256
    return sb <= 128 and (_tiled_units(rows, cols) <= SMALL_UNITS or sb <= 16)


def _device(qmv, rows, cols, seed):
    raw = qmv.synth_tensor(B.Q4_K, rows, cols, seed=seed)
    dt = qmv.DeviceTensor(qmv.make_view(raw, B.Q4_K, rows, cols))
    tiled = -(-rows // 64) * (cols // 256) * 64 * 144
    packed = rows * (cols // 256) * 144
    # the extra GGUF copy is what routes the tensor's single-position launches
    assert dt.device_bytes == tiled + (packed if _keeps_copy(rows, cols) else 0), (rows, cols, dt.device_bytes)
    return raw, dt


def _check(oracle, raw, rows, cols, x, y, what, fmt=B.Q4_K):
    y_ref = oracle.matvec(raw, fmt, rows, cols, x)
    _, absdot = oracle.row_stats(raw, fmt, rows, cols, x)
    err = np.abs(y.astype(np.float64) - y_ref)
    bad = err > TOL * absdot
    assert not bad.any(), f"{what}: {int(bad.sum())} rows over tolerance"
    return float(np.max(err / np.maximum(absdot, 1e-300)))


# rows: odd counts (workgroups with missing rows), one row, tile edges;
# K in super-blocks: 16-lane segments (1, 2, 4), 32-lane segments (6, 8),
# 64-lane segments (14, 16), rows spanning 2 to 8 waves (17, 35, 64, 65,
# 100, 128).
SHAPES = [(1, 256), (2, 256), (3, 512), (5, 4 * 256), (63, 1536), (64, 1536), (9, 8 * 256), (65, 3584),
          (513, 3584), (3584, 3584), (70, 16 * 256), (33, 17 * 256), (257, 35 * 256), (130, 64 * 256),
          (64, 65 * 256), (131, 100 * 256), (1, 128 * 256), (128, 128 * 256)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_rowmajor_matches_oracle(qmv, oracle, gpu, hip, rows, cols, seg_rows):
    log(f"row-major Q4_K {rows}x{cols}, {seg_rows} rows per segment")
    raw, dt = _device(qmv, rows, cols, seed=700 + rows + cols // 256)
    assert _tiled_units(rows, cols) <= SMALL_UNITS
    x = qmv.synth_normal(cols, seed=701 + rows)
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(4 * rows)
    with hip.Stream() as s:
        dt.matvec(dx.ptr, 1, dy.ptr, s.handle)
        s.synchronize()
        y = dy.to_array(np.float32, (rows,))
        worst = _check(oracle, raw, rows, cols, x, y, f"{rows}x{cols}")
        for _ in range(2):
            dy.fill(0)
            dt.matvec(dx.ptr, 1, dy.ptr, s.handle)
            s.synchronize()
            assert np.array_equal(_bits(dy.to_array(np.float32, (rows,))), _bits(y))
    log(f"  worst err/sum|wx| = {worst:.2e}")
    dt.close()


def test_rowmajor_group_of_unequal_rows(qmv, oracle, gpu, hip, seg_rows):
    """q|k|v-shaped group (Qwen2.5-7B): three tensors of 3584, 512 and 512 rows
    over one input, one launch."""
    cols = 3584
    specs = [(3584, 710), (512, 711), (512, 712)]
    tensors = [_device(qmv, r, cols, seed) for r, seed in specs]
    x = qmv.synth_normal(cols, seed=713)
    dx = hip.DeviceBuffer.from_array(x)
    outs = [hip.DeviceBuffer(4 * r) for r, _ in specs]
    with hip.Stream() as s:
        qmv.device_matvec_group([dt for _, dt in tensors], dx.ptr, 1, [o.ptr for o in outs], s.handle)
        s.synchronize()
        for (raw, dt), (r, _), o in zip(tensors, specs, outs):
            _check(oracle, raw, r, cols, x, o.to_array(np.float32, (r,)), f"group {r}x{cols}")
            alone = hip.DeviceBuffer(4 * r)
            dt.matvec(dx.ptr, 1, alone.ptr, s.handle)
            s.synchronize()
            assert np.array_equal(_bits(alone.to_array(np.float32, (r,))), _bits(o.to_array(np.float32, (r,))))
    for _, dt in tensors:
        dt.close()


def test_rowmajor_addend_bit_exact(qmv, oracle, gpu, hip, seg_rows):
    cols = 1536
    specs = [(1536, 720), (256, 721), (255, 722)]
    tensors = [_device(qmv, r, cols, seed) for r, seed in specs]
    x = qmv.synth_normal(cols, seed=723)
    dx = hip.DeviceBuffer.from_array(x)
    with hip.Stream() as s:
        plain = [hip.DeviceBuffer(4 * r) for r, _ in specs]
        qmv.device_matvec_group([dt for _, dt in tensors], dx.ptr, 1, [p.ptr for p in plain], s.handle)
        adds = [qmv.synth_normal(r, seed=724 + i) for i, (r, _) in enumerate(specs)]
        dadds = [hip.DeviceBuffer.from_array(a) for a in adds]
        outs = [hip.DeviceBuffer(4 * r) for r, _ in specs]
        qmv.device_matvec_add_group([dt for _, dt in tensors], dx.ptr, 1, [d.ptr for d in dadds],
                                    [0] * len(specs), [o.ptr for o in outs], s.handle)
        s.synchronize()
        for (r, _), p, a, o in zip(specs, plain, adds, outs):
            want = p.to_array(np.float32, (r,)) + a
            assert np.array_equal(_bits(o.to_array(np.float32, (r,))), _bits(want))
    for _, dt in tensors:
        dt.close()


@pytest.mark.parametrize("rows,cols", [(1, 256), (65, 512), (896, 3584), (1000, 1536)])
def test_rowmajor_swiglu(qmv, oracle, gpu, hip, rows, cols, seg_rows):
    log(f"row-major SwiGLU {rows}x{cols}, {seg_rows} rows per segment")
    raw_g, dg = _device(qmv, rows, cols, 730)
    raw_u, du = _device(qmv, rows, cols, 731)
    x = qmv.synth_normal(cols, seed=732)
    dx = hip.DeviceBuffer.from_array(x)
    with hip.Stream() as s:
        g = hip.DeviceBuffer(4 * rows)
        u = hip.DeviceBuffer(4 * rows)
        qmv.device_matvec_group([dg, du], dx.ptr, 1, [g.ptr, u.ptr], s.handle)
        out = hip.DeviceBuffer(4 * rows)
        qmv.device_matvec_swiglu(dg, du, dx.ptr, 1, out.ptr, s.handle)
        s.synchronize()
        gate, up = g.to_array(np.float32, (rows,)), u.to_array(np.float32, (rows,))
        _check(oracle, raw_g, rows, cols, x, gate, "gate")
        _check(oracle, raw_u, rows, cols, x, up, "up")
        got = out.to_array(np.float32, (rows,)).astype(np.float64)
        ok, ref = oracle.swiglu(gate, up)
        assert ok == 1
        ref = np.asarray(ref, dtype=np.float64)
        assert (np.abs(got - ref) <= SWIGLU_ULPS * 2.0 ** -23 * np.abs(ref) + 1e-30).all()
    dg.close()
    du.close()


@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 512), (1000, 3584), (4099, 1536)])
def test_rowmajor_fused_argmax(qmv, oracle, gpu, hip, rows, cols, seg_rows):
    log(f"row-major fused argmax {rows}x{cols}, {seg_rows} rows per segment")
    raw, dt = _device(qmv, rows, cols, 740 + rows)
    x = qmv.synth_normal(cols, seed=741)
    dx = hip.DeviceBuffer.from_array(x)
    with hip.Stream() as s:
        plain = hip.DeviceBuffer(4 * rows)
        dt.matvec(dx.ptr, 1, plain.ptr, s.handle)
        logits = hip.DeviceBuffer(4 * rows)
        res = hip.DeviceBuffer(8)
        for _ in range(3):  # the candidate counters must be left at zero
            qmv.device_matvec_argmax(dt, dx.ptr, logits.ptr, res.ptr, s.handle)
            s.synchronize()
            y = logits.to_array(np.float32, (rows,))
            assert np.array_equal(_bits(y), _bits(plain.to_array(np.float32, (rows,))))
            token, finite = res.to_array(np.int32, (2,))
            assert finite == 1 and token == int(np.argmax(y)), (token, int(np.argmax(y)))
        _check(oracle, raw, rows, cols, x, y, "logits")
    dt.close()


@pytest.mark.parametrize("rows,cols", [(300, 3584), (1000, 1536), (70, 20 * 256)])
def test_rowmajor_argmax_ties_and_non_finite(qmv, gpu, hip, rows, cols, seg_rows):
    """All-zero input: every logit is 0, so the lowest id wins (token 0). A row
    whose first super-block has an infinite scale d gives a non-finite
    logit: token -1 and flag 0, the reference sampler's rejection."""
    log(f"row-major argmax ties / inf {rows}x{cols}, {seg_rows} rows per segment")
    raw = qmv.synth_tensor(B.Q4_K, rows, cols, seed=760)

    def fused(buf, x):
        dt = qmv.DeviceTensor(qmv.make_view(buf, B.Q4_K, rows, cols))
        assert dt.device_bytes > -(-rows // 64) * (cols // 256) * 64 * 144  # keeps the row-major copy
        dx = hip.DeviceBuffer.from_array(x)
        logits = hip.DeviceBuffer(4 * rows)
        res = hip.DeviceBuffer(8)
        with hip.Stream() as s:
            out = []
            for _ in range(2):
                qmv.device_matvec_argmax(dt, dx.ptr, logits.ptr, res.ptr, s.handle)
                s.synchronize()
                out.append(res.to_array(np.int32, (2,)).tolist())
        y = logits.to_array(np.float32, (rows,))
        dt.close()
        return out, y

    out, y = fused(raw, np.zeros(cols, dtype=np.float32))
    assert out == [[0, 1]] * 2 and not y.any()
    bad = raw.copy()
    row = rows - 3
    off = row * (cols // 256) * 144
    bad[off:off + 2] = np.frombuffer(np.uint16(0x7C00).tobytes(), dtype=np.uint8)
    out, y = fused(bad, qmv.synth_normal(cols, seed=761))
    assert not np.isfinite(y[row]) and np.isfinite(np.delete(y, row)).all()
    assert out == [[-1, 0]] * 2


def test_rowmajor_switched_off(qmv, oracle, gpu, hip):
    """qmv_set_rowmajor(0, .): a tensor uploaded afterwards keeps only the
    tiled layout, and its launches (tiled) stay within the row bar; switched
    back on, new tensors keep the copy again."""
    rows, cols = 3584, 3584
    raw = qmv.synth_tensor(B.Q4_K, rows, cols, seed=770)
    x = qmv.synth_normal(cols, seed=771)
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(4 * rows)
    tiled = 56 * 14 * 64 * 144
    qmv.set_rowmajor(False, 2)
    try:
        dt = qmv.DeviceTensor(qmv.make_view(raw, B.Q4_K, rows, cols))
        assert dt.device_bytes == tiled
        with hip.Stream() as s:
            dt.matvec(dx.ptr, 1, dy.ptr, s.handle)
            s.synchronize()
        _check(oracle, raw, rows, cols, x, dy.to_array(np.float32, (rows,)), "row-major off")
        dt.close()
    finally:
        qmv.set_rowmajor(True, 2)
    dt = qmv.DeviceTensor(qmv.make_view(raw, B.Q4_K, rows, cols))
    assert dt.device_bytes == tiled + rows * 14 * 144
    dt.close()


def test_large_launch_policy(qmv, gpu):
    """Large launches run row-major only over rows of at most 16 super-blocks:
    a gate-sized tensor (Qwen2.5-7B, 18944 x 3584, 4144 tiled pairs) keeps the
    GGUF copy, a long-row one (3584 x 18944, 74 super-blocks, 4144 pairs)
    stays tiled only."""
    raw = qmv.synth_tensor(B.Q4_K, 18944, 3584, seed=750)
    dt = qmv.DeviceTensor(qmv.make_view(raw, B.Q4_K, 18944, 3584))
    assert dt.device_bytes == 296 * 14 * 64 * 144 + 18944 * 14 * 144
    dt.close()
    raw = qmv.synth_tensor(B.Q4_K, 3584, 18944, seed=751)
    dt = qmv.DeviceTensor(qmv.make_view(raw, B.Q4_K, 3584, 18944))
    assert dt.device_bytes == 56 * 74 * 64 * 144
    dt.close()


@pytest.mark.parametrize("rows,cols", [(18944, 3584), (30000, 1536), (20000, 4096)])
def test_large_rowmajor_launches(qmv, oracle, gpu, hip, rows, cols):
    """Launches over more than 2048 tiled pairs (4 rows per segment): a
    gate|up-shaped group (Qwen2.5-7B 2 x 18944 x 3584), 32-lane segments
    (K = 1536, two groups of 30000 rows) and 16 super-blocks per row: each
    row within the oracle's bar, the group's rows equal to each tensor's own
    launch bit for bit, the fused SwiGLU equal to up * silu(gate) of those
    rows, and the fused argmax (which runs tiled at these sizes) equal to the
    argmax of its own logits, which are within the oracle's bar."""
    log(f"large row-major launch 2 x {rows}x{cols}")
    (raw_g, dg), (raw_u, du) = _device(qmv, rows, cols, 780), _device(qmv, rows, cols, 781)
    x = qmv.synth_normal(cols, seed=782)
    dx = hip.DeviceBuffer.from_array(x)
    with hip.Stream() as s:
        g, u, out, lg = (hip.DeviceBuffer(4 * rows) for _ in range(4))
        res = hip.DeviceBuffer(8)
        qmv.device_matvec_group([dg, du], dx.ptr, 1, [g.ptr, u.ptr], s.handle)
        qmv.device_matvec_swiglu(dg, du, dx.ptr, 1, out.ptr, s.handle)
        qmv.device_matvec_argmax(dg, dx.ptr, lg.ptr, res.ptr, s.handle)
        s.synchronize()
        gate, up = g.to_array(np.float32, (rows,)), u.to_array(np.float32, (rows,))
        _check(oracle, raw_g, rows, cols, x, gate, "gate")
        _check(oracle, raw_u, rows, cols, x, up, "up")
        alone = hip.DeviceBuffer(4 * rows)
        dg.matvec(dx.ptr, 1, alone.ptr, s.handle)
        s.synchronize()
        assert np.array_equal(_bits(alone.to_array(np.float32, (rows,))), _bits(gate))
        logits = lg.to_array(np.float32, (rows,))
        _check(oracle, raw_g, rows, cols, x, logits, "fused argmax logits")
        token, finite = res.to_array(np.int32, (2,))
        assert finite == 1 and token == int(np.argmax(logits))
        got = out.to_array(np.float32, (rows,)).astype(np.float64)
        ok, ref = oracle.swiglu(gate, up)
        assert ok == 1
        ref = np.asarray(ref, dtype=np.float64)
        assert (np.abs(got - ref) <= SWIGLU_ULPS * 2.0 ** -23 * np.abs(ref) + 1e-30).all()
    dg.close()
    du.close()


# ---- Q6_K ------------------------------------------------------------------

def _q6_stride(sb):
    return (210 * sb + 15) // 16 * 16


def _device_q6(qmv, rows, cols, seed):
    raw = qmv.synth_tensor(B.Q6_K, rows, cols, seed=seed)
    dt = qmv.DeviceTensor(qmv.make_view(raw, B.Q6_K, rows, cols))
    sb = cols // 256
    tiled = -(-rows // 64) * sb * 64 * 210
    copy = rows * _q6_stride(sb) if 16 < sb <= 128 else 0
    assert dt.device_bytes == tiled + copy, (rows, cols, dt.device_bytes)
    return raw, dt


# rows: one row, odd counts (workgroups with missing rows), tile edges, the
# Qwen2.5-7B down projection (3584 x 18944), workgroups of 1..16 waves; K:
# 17 (two slices, the second of one super-block), 19, 32 and 64 (whole last
# slices), 33, 74, 100, 112 and 128 super-blocks (8 slices).
Q6_SHAPES = [(1, 17 * 256), (2, 17 * 256), (5, 19 * 256), (63, 19 * 256), (65, 33 * 256), (130, 74 * 256),
             (7, 100 * 256), (1, 128 * 256), (129, 128 * 256), (3584, 74 * 256), (225, 32 * 256),
             (3, 64 * 256), (449, 112 * 256)]


@pytest.mark.parametrize("rows,cols", Q6_SHAPES)
def test_rowmajor_q6k_matches_oracle(qmv, oracle, gpu, hip, rows, cols):
    log(f"row-major Q6_K {rows}x{cols}")
    raw, dt = _device_q6(qmv, rows, cols, seed=800 + rows + cols // 256)
    x = qmv.synth_normal(cols, seed=801 + rows)
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(4 * rows)
    with hip.Stream() as s:
        dt.matvec(dx.ptr, 1, dy.ptr, s.handle)
        s.synchronize()
        y = dy.to_array(np.float32, (rows,))
        worst = _check(oracle, raw, rows, cols, x, y, f"Q6_K {rows}x{cols}", fmt=B.Q6_K)
        for _ in range(2):
            dy.fill(0)
            dt.matvec(dx.ptr, 1, dy.ptr, s.handle)
            s.synchronize()
            assert np.array_equal(_bits(dy.to_array(np.float32, (rows,))), _bits(y))
    log(f"  worst err/sum|wx| = {worst:.2e}")
    dt.close()


def test_rowmajor_q6k_group_and_addend(qmv, oracle, gpu, hip):
    """Three Q6_K tensors over one input in one launch (3584, 100 and 1 rows
    of 74 super-blocks): each within the bar and equal to its own launch bit
    for bit; with addends, equal to those rows plus the addend."""
    cols = 74 * 256
    specs = [(3584, 810), (100, 811), (1, 812)]
    tensors = [_device_q6(qmv, r, cols, seed) for r, seed in specs]
    x = qmv.synth_normal(cols, seed=813)
    dx = hip.DeviceBuffer.from_array(x)
    outs = [hip.DeviceBuffer(4 * r) for r, _ in specs]
    adds = [qmv.synth_normal(r, seed=814 + i) for i, (r, _) in enumerate(specs)]
    dadds = [hip.DeviceBuffer.from_array(a) for a in adds]
    sums = [hip.DeviceBuffer(4 * r) for r, _ in specs]
    with hip.Stream() as s:
        qmv.device_matvec_group([dt for _, dt in tensors], dx.ptr, 1, [o.ptr for o in outs], s.handle)
        qmv.device_matvec_add_group([dt for _, dt in tensors], dx.ptr, 1, [d.ptr for d in dadds],
                                    [0] * len(specs), [o.ptr for o in sums], s.handle)
        s.synchronize()
        for (raw, dt), (r, _), o, a, sm in zip(tensors, specs, outs, adds, sums):
            y = o.to_array(np.float32, (r,))
            _check(oracle, raw, r, cols, x, y, f"Q6_K group {r}x{cols}", fmt=B.Q6_K)
            alone = hip.DeviceBuffer(4 * r)
            dt.matvec(dx.ptr, 1, alone.ptr, s.handle)
            s.synchronize()
            assert np.array_equal(_bits(alone.to_array(np.float32, (r,))), _bits(y))
            assert np.array_equal(_bits(sm.to_array(np.float32, (r,))), _bits(y + a))
    for _, dt in tensors:
        dt.close()


def test_rowmajor_q6k_copy_policy(qmv, oracle, gpu, hip):
    """Q6_K rows of at most 16 super-blocks (896 x 3584) keep no copy; with the
    row-major kernels switched off, long rows keep none either; both run
    tiled within the bar, and two positions of a tensor with a copy run
    tiled within it too."""
    raw, dt = _device_q6(qmv, 896, 3584, seed=820)
    assert dt.device_bytes == 14 * 14 * 64 * 210
    x = qmv.synth_normal(3584, seed=821)
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(4 * 896)
    with hip.Stream() as s:
        dt.matvec(dx.ptr, 1, dy.ptr, s.handle)
        s.synchronize()
    _check(oracle, raw, 896, 3584, x, dy.to_array(np.float32, (896,)), "Q6_K short rows", fmt=B.Q6_K)
    dt.close()
    rows, cols = 200, 40 * 256
    raw = qmv.synth_tensor(B.Q6_K, rows, cols, seed=822)
    x2 = np.concatenate([qmv.synth_normal(cols, seed=823), qmv.synth_normal(cols, seed=824)])
    dx = hip.DeviceBuffer.from_array(x2)
    dy = hip.DeviceBuffer(4 * 2 * rows)
    qmv.set_rowmajor(False, 2)
    try:
        dt = qmv.DeviceTensor(qmv.make_view(raw, B.Q6_K, rows, cols))
        assert dt.device_bytes == 4 * 40 * 64 * 210
        with hip.Stream() as s:
            dt.matvec(dx.ptr, 1, dy.ptr, s.handle)
            s.synchronize()
        _check(oracle, raw, rows, cols, x2[:cols], dy.to_array(np.float32, (rows,)), "Q6_K switched off", fmt=B.Q6_K)
        dt.close()
    finally:
        qmv.set_rowmajor(True, 2)
    raw, dt = _device_q6(qmv, rows, cols, seed=822)
    with hip.Stream() as s:
        dt.matvec(dx.ptr, 2, dy.ptr, s.handle)
        s.synchronize()
    y = dy.to_array(np.float32, (2, rows))
    for b in range(2):
        _check(oracle, raw, rows, cols, x2[b * cols:(b + 1) * cols], y[b], f"Q6_K two positions, {b}", fmt=B.Q6_K)
    dt.close()


@pytest.mark.parametrize("rows,cols", [(1, 17 * 256), (65, 74 * 256), (300, 33 * 256), (130, 128 * 256)])
def test_rowmajor_q6k_swiglu(qmv, oracle, gpu, hip, rows, cols):
    """Fused SwiGLU over a Q6_K gate/up pair with long rows: within 4 ulp of
    the oracle's transformer_swiglu_f32 of the plain launch's rows, which are
    within the row bar."""
    log(f"row-major Q6_K SwiGLU {rows}x{cols}")
    raw_g, dg = _device_q6(qmv, rows, cols, 830)
    raw_u, du = _device_q6(qmv, rows, cols, 831)
    x = qmv.synth_normal(cols, seed=832)
    dx = hip.DeviceBuffer.from_array(x)
    with hip.Stream() as s:
        g = hip.DeviceBuffer(4 * rows)
        u = hip.DeviceBuffer(4 * rows)
        qmv.device_matvec_group([dg, du], dx.ptr, 1, [g.ptr, u.ptr], s.handle)
        out = hip.DeviceBuffer(4 * rows)
        qmv.device_matvec_swiglu(dg, du, dx.ptr, 1, out.ptr, s.handle)
        s.synchronize()
        gate, up = g.to_array(np.float32, (rows,)), u.to_array(np.float32, (rows,))
        _check(oracle, raw_g, rows, cols, x, gate, "gate", fmt=B.Q6_K)
        _check(oracle, raw_u, rows, cols, x, up, "up", fmt=B.Q6_K)
        got = out.to_array(np.float32, (rows,)).astype(np.float64)
        ok, ref = oracle.swiglu(gate, up)
        assert ok == 1
        ref = np.asarray(ref, dtype=np.float64)
        assert (np.abs(got - ref) <= SWIGLU_ULPS * 2.0 ** -23 * np.abs(ref) + 1e-30).all()
    dg.close()
    du.close()


@pytest.mark.parametrize("rows,cols", [(1, 17 * 256), (7, 74 * 256), (1000, 19 * 256), (3585, 74 * 256)])
def test_rowmajor_q6k_fused_argmax(qmv, oracle, gpu, hip, rows, cols):
    """Fused argmax over a Q6_K tensor with long rows (one candidate per
    workgroup): logits bit-identical to the plain launch on every repeat, the
    token the argmax of those logits, the logits within the row bar."""
    log(f"row-major Q6_K fused argmax {rows}x{cols}")
    raw, dt = _device_q6(qmv, rows, cols, 840 + rows)
    x = qmv.synth_normal(cols, seed=841)
    dx = hip.DeviceBuffer.from_array(x)
    with hip.Stream() as s:
        plain = hip.DeviceBuffer(4 * rows)
        dt.matvec(dx.ptr, 1, plain.ptr, s.handle)
        logits = hip.DeviceBuffer(4 * rows)
        res = hip.DeviceBuffer(8)
        for _ in range(3):  # the candidate counters must be left at zero
            qmv.device_matvec_argmax(dt, dx.ptr, logits.ptr, res.ptr, s.handle)
            s.synchronize()
            y = logits.to_array(np.float32, (rows,))
            assert np.array_equal(_bits(y), _bits(plain.to_array(np.float32, (rows,))))
            token, finite = res.to_array(np.int32, (2,))
            assert finite == 1 and token == int(np.argmax(y)), (token, int(np.argmax(y)))
        _check(oracle, raw, rows, cols, x, y, "Q6_K logits", fmt=B.Q6_K)
    dt.close()


def test_rowmajor_q6k_argmax_ties_and_non_finite(qmv, gpu, hip):
    """All-zero input: every logit is 0 and the lowest id wins. A row whose
    first super-block has an infinite d gives a non-finite logit: token -1
    and flag 0."""
    rows, cols = 500, 40 * 256
    raw = qmv.synth_tensor(B.Q6_K, rows, cols, seed=850)

    def fused(buf, x):
        dt = qmv.DeviceTensor(qmv.make_view(buf, B.Q6_K, rows, cols))
        assert dt.device_bytes == 8 * 40 * 64 * 210 + rows * _q6_stride(40)
        dx = hip.DeviceBuffer.from_array(x)
        logits = hip.DeviceBuffer(4 * rows)
        res = hip.DeviceBuffer(8)
        with hip.Stream() as s:
            out = []
            for _ in range(2):
                qmv.device_matvec_argmax(dt, dx.ptr, logits.ptr, res.ptr, s.handle)
                s.synchronize()
                out.append(res.to_array(np.int32, (2,)).tolist())
        y = logits.to_array(np.float32, (rows,))
        dt.close()
        return out, y

    out, y = fused(raw, np.zeros(cols, dtype=np.float32))
    assert out == [[0, 1]] * 2 and not y.any()
    bad = raw.copy()
    row = rows - 3
    off = row * 40 * 210 + 208  # d of the row's first super-block
    bad[off:off + 2] = np.frombuffer(np.uint16(0x7C00).tobytes(), dtype=np.uint8)
    out, y = fused(bad, qmv.synth_normal(cols, seed=851))
    assert not np.isfinite(y[row]) and np.isfinite(np.delete(y, row)).all()
    assert out == [[-1, 0]] * 2
