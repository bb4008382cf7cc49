"""GPU parity of the decode-step operations around the projections, through
the C ABI: the fused addend (q/k/v biases, residuals), the fused SwiGLU of
the gate and up projections, and RMSNorm.

Bars:
  * addend: bit-identical to the plain launch's rows plus the addend in fp32
    (the reference adds with a separate tensor_add_f32, src/tensor.cpp:5-23,
    after the same product);
  * SwiGLU: within SWIGLU_ULPS units in the last place of the oracle's
    transformer_swiglu_f32 (src/transformer_ops.cpp:163-176) applied to the
    plain launch's gate and up rows; the exponential is the only operation
    that is not correctly rounded on both sides;
  * RMSNorm: within RMS_REL relative of the float64 closed form, the bound the
    oracle and the reference's own build meet (tests/test_oracle.py);
  * the projections themselves: the row bar of test_gpu_parity.py against
    the oracle.
"""
import numpy as np
import pytest

import _blocks as B

pytestmark = pytest.mark.gpu

TOL = 1e-5  # rows: relative to sum |w x|
SWIGLU_ULPS = 4
RMS_REL = 2e-5
EPS = 1e-6


def log(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def hip(qmv):
    import importlib
    return importlib.import_module("my-inference-engine_amd.hip_runtime")


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _tensor(qmv, t, rows, cols, seed):
    raw = qmv.synth_tensor(t, rows, cols, seed=seed)
    return raw, qmv.DeviceTensor(qmv.make_view(raw, t, rows, cols))


def _plain(qmv, hip, dts, dx, batch, stream):
    outs = [hip.DeviceBuffer(4 * batch * d.rows) for d in dts]
    qmv.device_matvec_group(dts, dx.ptr, batch, [o.ptr for o in outs], stream.handle)
    stream.synchronize()
    return [o.to_array(np.float32, (batch, d.rows)) for o, d in zip(outs, dts)]


def _check_rows(oracle, raw, t, rows, cols, x, y, what):
    for b in range(x.shape[0]):
        y_ref = oracle.matvec(raw, t, rows, cols, x[b])
        _, absdot = oracle.row_stats(raw, t, rows, cols, x[b])
        err = np.abs(y[b].astype(np.float64) - y_ref)
        assert (err <= TOL * absdot).all(), f"{what} pos {b}"


# ---- bias and residual fused into the store ---------------------------------------

@pytest.mark.parametrize("t,shapes,cols", [
    (B.Q4_K, [3584, 512, 512], 3584),       # Qwen2-7B q/k/v with biases
    (B.Q5_0, [1536, 256, 256], 1536),       # Qwen2-1.5B q/k/v
    (B.Q8_0, [896, 128, 128], 896),         # Qwen2-0.5B q/k/v
    (B.Q6_K, [3584], 18944),                # FFN down (split along K)
])
@pytest.mark.parametrize("batch", [1, 3, 8])
def test_bias_epilogue_bit_exact(qmv, oracle, gpu, hip, t, shapes, cols, batch):
    log(f"bias epilogue type {t} rows {shapes} K {cols} M={batch}")
    pairs = [_tensor(qmv, t, r, cols, 70 + i) for i, r in enumerate(shapes)]
    raws, dts = [p[0] for p in pairs], [p[1] for p in pairs]
    x = qmv.synth_normal(batch * cols, seed=71).reshape(batch, cols)
    dx = hip.DeviceBuffer.from_array(x)
    stream = hip.Stream()
    plain = _plain(qmv, hip, dts, dx, batch, stream)
    _check_rows(oracle, raws[0], t, shapes[0], cols, x, plain[0], "plain")
    rng = np.random.default_rng(72)
    biases = [(rng.standard_normal(r) * 0.5).astype(np.float32) for r in shapes]
    dbias = [hip.DeviceBuffer.from_array(b) for b in biases]
    outs = [hip.DeviceBuffer(4 * batch * r) for r in shapes]
    qmv.device_matvec_add_group(dts, dx.ptr, batch, [b.ptr for b in dbias], [0] * len(dts),
                                [o.ptr for o in outs], stream.handle)
    stream.synchronize()
    for i, (o, r) in enumerate(zip(outs, shapes)):
        got = o.to_array(np.float32, (batch, r))
        assert np.array_equal(_bits(got), _bits(plain[i] + biases[i][None, :])), f"tensor {i}"
    # A null addend stores the plain product.
    outs2 = [hip.DeviceBuffer(4 * batch * r) for r in shapes]
    qmv.device_matvec_add_group(dts, dx.ptr, batch, [0] * len(dts), [0] * len(dts), [o.ptr for o in outs2],
                                stream.handle)
    stream.synchronize()
    for i, (o, r) in enumerate(zip(outs2, shapes)):
        assert np.array_equal(_bits(o.to_array(np.float32, (batch, r))), _bits(plain[i]))
    for d in dts:
        d.close()


@pytest.mark.parametrize("t,rows,cols", [(B.Q4_K, 3584, 3584), (B.Q6_K, 3584, 18944), (B.Q8_0, 896, 896),
                                         (B.Q5_0, 1536, 8960 // 32 * 32)])
@pytest.mark.parametrize("batch", [1, 8])
def test_residual_in_place_bit_exact(qmv, gpu, hip, t, rows, cols, batch):
    """x += W h with the residual stream as addend and output (stride N)."""
    log(f"residual in place type {t} {rows}x{cols} M={batch}")
    _, dt = _tensor(qmv, t, rows, cols, 80)
    h = qmv.synth_normal(batch * cols, seed=81).reshape(batch, cols)
    dh = hip.DeviceBuffer.from_array(h)
    stream = hip.Stream()
    plain = _plain(qmv, hip, [dt], dh, batch, stream)[0]
    resid = (np.random.default_rng(82).standard_normal((batch, rows)) * 3).astype(np.float32)
    dr = hip.DeviceBuffer.from_array(resid)
    qmv.device_matvec_add_group([dt], dh.ptr, batch, [dr.ptr], [rows], [dr.ptr], stream.handle)
    stream.synchronize()
    assert np.array_equal(_bits(dr.to_array(np.float32, (batch, rows))), _bits(plain + resid))
    dt.close()


def test_addend_overlap_rules(qmv, gpu, hip):
    cols = 1536
    _, dq = _tensor(qmv, B.Q4_K, 256, cols, 90)
    _, dk = _tensor(qmv, B.Q4_K, 256, cols, 91)
    dx = hip.DeviceBuffer.from_array(qmv.synth_normal(2 * cols, seed=92))
    y = hip.DeviceBuffer(4 * 2 * 256 * 2)
    a = hip.DeviceBuffer(4 * 2 * 256)
    s = hip.Stream()
    lib = qmv.hip_lib()
    # Output overlapping the input.
    with pytest.raises(qmv.QmvError, match="overlaps the input"):
        qmv.device_matvec_add_group([dq], dx.ptr, 1, [0], [0], [dx.ptr], s.handle)
    # Two outputs overlapping.
    with pytest.raises(qmv.QmvError, match="overlap each other"):
        qmv.device_matvec_add_group([dq, dk], dx.ptr, 1, [0, 0], [0, 0], [y.ptr, y.ptr + 4 * 100], s.handle)
    # Addend of one tensor is another tensor's output.
    with pytest.raises(qmv.QmvError, match="addend overlaps"):
        qmv.device_matvec_add_group([dq, dk], dx.ptr, 1, [y.ptr + 4 * 256, 0], [0, 0], [y.ptr, y.ptr + 4 * 256],
                                    s.handle)
    # In place with a broadcast stride would read overwritten values for M > 1.
    with pytest.raises(qmv.QmvError, match="addend overlaps"):
        qmv.device_matvec_add_group([dq], dx.ptr, 2, [a.ptr], [0], [a.ptr], s.handle)
    # Stride below the row count.
    with pytest.raises(qmv.QmvError, match="stride"):
        qmv.device_matvec_add_group([dq], dx.ptr, 2, [a.ptr], [100], [y.ptr], s.handle)
    assert lib.qmv_device_matvec_add_group_f32(None, 1, dx.ptr, 1, None, None, None, None) == 0
    dq.close()
    dk.close()


# ---- FFN gate and up fused with SwiGLU ---------------------------------------------

def _ulp_close(got, ref):
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    return np.abs(got - ref) <= SWIGLU_ULPS * 2.0 ** -23 * np.abs(ref) + 1e-30


@pytest.mark.parametrize("t,rows,cols,batch", [
    (B.Q4_K, 18944, 3584, 1), (B.Q4_K, 18944, 3584, 8), (B.Q4_K, 8960, 1536, 3),
    (B.Q6_K, 1000, 896 * 4, 2), (B.Q8_0, 4864, 896, 1), (B.Q5_0, 130, 1536, 5), (B.Q4_K, 65, 256, 7),
    (B.Q6_K, 1000, 896 * 4, 1), (B.Q5_0, 130, 1536, 1), (B.Q4_K, 65, 256, 1), (B.Q4_K, 4864, 18944, 1)])
def test_swiglu_fused_matches_oracle(qmv, oracle, gpu, hip, t, rows, cols, batch):
    log(f"fused SwiGLU type {t} {rows}x{cols} M={batch}")
    raw_g, dg = _tensor(qmv, t, rows, cols, 100)
    raw_u, du = _tensor(qmv, t, rows, cols, 101)
    x = qmv.synth_normal(batch * cols, seed=102).reshape(batch, cols)
    dx = hip.DeviceBuffer.from_array(x)
    stream = hip.Stream()
    gate, up = _plain(qmv, hip, [dg, du], dx, batch, stream)
    _check_rows(oracle, raw_g, t, rows, cols, x, gate, "gate")
    _check_rows(oracle, raw_u, t, rows, cols, x, up, "up")
    dout = hip.DeviceBuffer(4 * batch * rows)
    qmv.device_matvec_swiglu(dg, du, dx.ptr, batch, dout.ptr, stream.handle)
    stream.synchronize()
    got = dout.to_array(np.float32, (batch, rows))
    for b in range(batch):
        ok, ref = oracle.swiglu(gate[b], up[b])
        assert ok == 1
        close = _ulp_close(got[b], ref)
        assert close.all(), f"pos {b}: {int((~close).sum())} elements beyond {SWIGLU_ULPS} ulp"
    same = float(np.mean(_bits(got) == _bits(np.stack([oracle.swiglu(gate[b], up[b])[1] for b in range(batch)]))))
    log(f"  bit-identical to the oracle on {same:.4f} of elements")
    dg.close()
    du.close()


def test_swiglu_rejects_mismatched_pair(qmv, gpu, hip):
    _, dg = _tensor(qmv, B.Q4_K, 512, 1536, 110)
    _, du = _tensor(qmv, B.Q4_K, 256, 1536, 111)
    dx = hip.DeviceBuffer.from_array(qmv.synth_normal(1536, seed=112))
    dout = hip.DeviceBuffer(4 * 512)
    with pytest.raises(qmv.QmvError, match="share type, shape"):
        qmv.device_matvec_swiglu(dg, du, dx.ptr, 1, dout.ptr, 0)
    with pytest.raises(qmv.QmvError, match="overlaps the input"):
        qmv.device_matvec_swiglu(dg, dg, dx.ptr, 1, dx.ptr, 0)
    dg.close()
    du.close()


# ---- RMSNorm ------------------------------------------------------------------------

def _rms_f64(x, w):
    x64 = x.astype(np.float64)
    return x64 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + float(np.float32(EPS))) * w


@pytest.mark.parametrize("n,batch,scale", [(3584, 1, 1.0), (3584, 8, 1.0), (3584, 2, 1e-3), (896, 3, 30.0),
                                           (1536, 1, 1e-4), (7, 2, 1.0), (18944, 1, 0.05), (256, 1, 1.0)])
def test_rms_norm_matches_float64_and_oracle(qmv, oracle, gpu, hip, n, batch, scale):
    log(f"RMSNorm n={n} M={batch} scale={scale}")
    rng = np.random.default_rng(n + batch)
    x = (rng.standard_normal((batch, n)) * scale).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    dx, dw = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(w)
    dy = hip.DeviceBuffer(4 * batch * n)
    stream = hip.Stream()
    qmv.device_rms_norm(dx.ptr, dw.ptr, n, batch, EPS, dy.ptr, stream.handle)
    stream.synchronize()
    y = dy.to_array(np.float32, (batch, n))
    ref = _rms_f64(x, w)
    assert (np.abs(y - ref) <= RMS_REL * np.abs(ref) + 1e-30).all()
    for b in range(batch):
        ok, yo = oracle.rms_norm(x[b], w, EPS)
        assert ok == 1 and (np.abs(y[b].astype(np.float64) - yo) <= 2 * RMS_REL * np.abs(yo) + 1e-30).all()
    # In place gives the same bits.
    qmv.device_rms_norm(dx.ptr, dw.ptr, n, batch, EPS, dx.ptr, stream.handle)
    stream.synchronize()
    assert np.array_equal(_bits(dx.to_array(np.float32, (batch, n))), _bits(y))


def test_rms_norm_kat(qmv, gpu, hip):
    """tests/tensor_reference_test.cpp:84-93: {1, 1}, weight {2, 3}, eps 3 -> {1, 1.5}."""
    dx = hip.DeviceBuffer.from_array(np.array([1.0, 1.0], np.float32))
    dw = hip.DeviceBuffer.from_array(np.array([2.0, 3.0], np.float32))
    dy = hip.DeviceBuffer(8)
    qmv.device_rms_norm(dx.ptr, dw.ptr, 2, 1, 3.0, dy.ptr, 0)
    hip.synchronize()
    assert dy.to_array(np.float32, (2,)).tolist() == [1.0, 1.5]


# ---- RMSNorm fused into the projection that consumes it ------------------------------

NORM_SLACK = 1e-6  # rows: the norm's own rounding (h = x * w then / denom, vs (x / denom) * w)


def _norm_inputs(rng, batch, cols, scale):
    x = (rng.standard_normal((batch, cols)) * scale).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    return x, w


def _normed_rows(oracle, raw, t, rows, cols, x, w):
    """The reference's norm then matvec per position: rows and their bars."""
    ys, bars = [], []
    for b in range(x.shape[0]):
        ok, h = oracle.rms_norm(x[b], w, EPS)
        assert ok == 1
        h = np.asarray(h, np.float32)
        ys.append(np.asarray(oracle.matvec(raw, t, rows, cols, h), np.float64))
        bars.append((TOL + NORM_SLACK) * oracle.row_stats(raw, t, rows, cols, h)[1])
    return np.stack(ys), np.stack(bars)


@pytest.mark.parametrize("t,shapes,cols,batch,scale", [
    (B.Q4_K, [3584, 512, 512], 3584, 1, 1.0),    # Qwen2.5-7B attention norm + q/k/v: fused
    (B.Q4_K, [3584, 512, 512], 3584, 1, 1e-3),   # epsilon comparable to mean(x^2)
    (B.Q4_K, [1536, 256, 256], 1536, 1, 3.0),    # 6 super-blocks per row: 32-lane segments
    (B.Q4_K, [1000, 77], 1024, 1, 1.0),          # 4 super-blocks: 16-lane segments, ragged rows
    (B.Q4_K, [3584, 512, 512], 3584, 3, 1.0),    # three positions: norm launch, then the group
    (B.Q4_K, [300], 18 * 256, 1, 1.0),           # rows past 16 super-blocks: norm launch
    (B.Q6_K, [1000], 3584, 1, 1.0),              # not Q4_K: norm launch
    (B.Q8_0, [896, 128], 896, 2, 1.0),
])
def test_rms_norm_fused_matvec_matches_oracle(qmv, oracle, gpu, hip, t, shapes, cols, batch, scale):
    """qmv_device_rms_norm_matvec_add_group_f32 against the oracle's RMSNorm
    followed by its matvec and the bias: within the row bar on the normalised
    input, plus NORM_SLACK for the norm's own rounding (the fused launch
    scales x by the norm weights and divides each row by the denominator)."""
    log(f"fused norm + matvec type {t} rows {shapes} K {cols} M={batch} scale {scale}")
    rng = np.random.default_rng(cols + batch)
    pairs = [_tensor(qmv, t, r, cols, 150 + i) for i, r in enumerate(shapes)]
    x, w = _norm_inputs(rng, batch, cols, scale)
    biases = [(rng.standard_normal(r) * 0.5).astype(np.float32) for r in shapes]
    dx, dw = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(w)
    dbias = [hip.DeviceBuffer.from_array(b) for b in biases]
    dnormed = hip.DeviceBuffer(4 * batch * cols)
    outs = [hip.DeviceBuffer(4 * batch * r) for r in shapes]
    stream = hip.Stream()
    dts = [p[1] for p in pairs]
    qmv.device_rms_norm_matvec_add_group(dts, dx.ptr, dw.ptr, EPS, batch, [b.ptr for b in dbias], [0] * len(dts),
                                         [o.ptr for o in outs], dnormed.ptr, stream.handle)
    stream.synchronize()
    for i, ((raw, d), r) in enumerate(zip(pairs, shapes)):
        got = outs[i].to_array(np.float32, (batch, r)).astype(np.float64)
        ref, bar = _normed_rows(oracle, raw, t, r, cols, x, w)
        err = np.abs(got - (ref + biases[i][None, :]))
        assert (err <= bar).all(), f"tensor {i}: {int((err > bar).sum())} rows over the bar"
    # Plain stores (no addends): the same rows without the bias, to the bar.
    qmv.device_rms_norm_matvec_add_group(dts, dx.ptr, dw.ptr, EPS, batch, None, None, [o.ptr for o in outs],
                                         dnormed.ptr, stream.handle)
    stream.synchronize()
    raw0 = pairs[0][0]
    ref, bar = _normed_rows(oracle, raw0, t, shapes[0], cols, x, w)
    err = np.abs(outs[0].to_array(np.float32, (batch, shapes[0])).astype(np.float64) - ref)
    assert (err <= bar).all()
    for d in dts:
        d.close()


@pytest.mark.parametrize("t,rows,cols,batch", [(B.Q4_K, 18944, 3584, 1), (B.Q4_K, 8960, 1536, 1),
                                               (B.Q4_K, 18944, 3584, 2), (B.Q6_K, 1000, 3584, 1)])
def test_rms_norm_fused_swiglu_matches_oracle(qmv, oracle, gpu, hip, t, rows, cols, batch):
    """qmv_device_rms_norm_matvec_swiglu_f32 against the oracle's RMSNorm,
    gate and up matvecs and SwiGLU: each projection within its bar (as above),
    carried through silu(g) * u (|d silu / dg| <= 1.1), plus SWIGLU_ULPS."""
    log(f"fused norm + SwiGLU type {t} {rows}x{cols} M={batch}")
    rng = np.random.default_rng(rows + batch)
    raw_g, dg = _tensor(qmv, t, rows, cols, 160)
    raw_u, du = _tensor(qmv, t, rows, cols, 161)
    x, w = _norm_inputs(rng, batch, cols, 1.0)
    dx, dw = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(w)
    dnormed = hip.DeviceBuffer(4 * batch * cols)
    dout = hip.DeviceBuffer(4 * batch * rows)
    stream = hip.Stream()
    qmv.device_rms_norm_matvec_swiglu(dg, du, dx.ptr, dw.ptr, EPS, batch, dout.ptr, dnormed.ptr, stream.handle)
    stream.synchronize()
    got = dout.to_array(np.float32, (batch, rows)).astype(np.float64)
    g_ref, g_bar = _normed_rows(oracle, raw_g, t, rows, cols, x, w)
    u_ref, u_bar = _normed_rows(oracle, raw_u, t, rows, cols, x, w)
    with np.errstate(over="ignore"):  # exp(-g) overflows to inf for g < -88 in float32 terms; silu -> -0
        silu = g_ref / (1.0 + np.exp(-g_ref))
    ref = u_ref * silu
    bar = 1.1 * np.abs(u_ref) * g_bar + np.abs(silu) * u_bar + g_bar * u_bar + SWIGLU_ULPS * 2.0 ** -23 * np.abs(ref)
    err = np.abs(got - ref)
    assert (err <= bar + 1e-30).all(), f"{int((err > bar).sum())} elements over the bar"
    dg.close()
    du.close()


def test_rms_norm_fused_graph_replays(qmv, gpu, hip):
    """The fused launch captured in a graph replays to the eager bits, with
    eager launches of other work between the replays."""
    cols = 3584
    _, dq = _tensor(qmv, B.Q4_K, 3584, cols, 170)
    _, dk = _tensor(qmv, B.Q4_K, 512, cols, 171)
    rng = np.random.default_rng(172)
    x, w = _norm_inputs(rng, 1, cols, 1.0)
    dx, dw = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(w)
    dnormed = hip.DeviceBuffer(4 * cols)
    yq, yk, other = hip.DeviceBuffer(4 * 3584), hip.DeviceBuffer(4 * 512), hip.DeviceBuffer(4 * 3584)
    with hip.Stream() as stream:
        call = lambda: qmv.device_rms_norm_matvec_add_group([dq, dk], dx.ptr, dw.ptr, EPS, 1, None, None,
                                                            [yq.ptr, yk.ptr], dnormed.ptr, stream.handle)
        call()
        stream.synchronize()
        eager = (yq.to_array(np.float32, (3584,)).copy(), yk.to_array(np.float32, (512,)).copy())
        with hip.Graph(stream) as g:
            g.begin()
            call()
            g.end()
            for i in range(3):
                yq.fill(0)
                yk.fill(0)
                g.replay()
                stream.synchronize()
                assert np.array_equal(_bits(yq.to_array(np.float32, (3584,))), _bits(eager[0])), i
                assert np.array_equal(_bits(yk.to_array(np.float32, (512,))), _bits(eager[1])), i
                qmv.device_matvec_group([dq], dx.ptr, 1, [other.ptr], stream.handle)
                stream.synchronize()
    dq.close()
    dk.close()


def test_rms_norm_fused_argument_rules(qmv, gpu, hip):
    cols = 1536
    _, dq = _tensor(qmv, B.Q4_K, 256, cols, 180)
    dx = hip.DeviceBuffer.from_array(qmv.synth_normal(cols, seed=181))
    dw = hip.DeviceBuffer.from_array(np.ones(cols, np.float32))
    y, dn = hip.DeviceBuffer(4 * 256), hip.DeviceBuffer(4 * cols)
    with pytest.raises(qmv.QmvError, match="RMSNorm arguments"):
        qmv.device_rms_norm_matvec_add_group([dq], dx.ptr, dw.ptr, 0.0, 1, None, None, [y.ptr], dn.ptr, 0)
    with pytest.raises(qmv.QmvError, match="RMSNorm arguments"):
        qmv.device_rms_norm_matvec_add_group([dq], dx.ptr, 0, EPS, 1, None, None, [y.ptr], dn.ptr, 0)
    with pytest.raises(qmv.QmvError, match="d_normed overlaps"):
        qmv.device_rms_norm_matvec_add_group([dq], dx.ptr, dw.ptr, EPS, 1, None, None, [y.ptr], dx.ptr, 0)
    with pytest.raises(qmv.QmvError, match="d_normed overlaps an output"):
        qmv.device_rms_norm_matvec_add_group([dq], dx.ptr, dw.ptr, EPS, 1, None, None, [y.ptr], y.ptr, 0)
    with pytest.raises(qmv.QmvError, match="share type, shape"):
        _, du = _tensor(qmv, B.Q4_K, 128, cols, 182)
        qmv.device_rms_norm_matvec_swiglu(dq, du, dx.ptr, dw.ptr, EPS, 1, y.ptr, dn.ptr, 0)
    dq.close()


# ---- the decode step's projections chained on device, replayed as a graph ----------

def test_decode_layer_chain_graph(qmv, oracle, gpu, hip):
    """One Qwen2 layer's projections and their element operations on device
    buffers (src/qwen2_architecture.cpp:1241-1463 without RoPE and attention,
    whose output is stood in for by the query rows): RMSNorm -> q/k/v + bias
    -> o + residual -> RMSNorm -> gate/up SwiGLU -> down + residual. Every
    stage is checked against the oracle on the GPU's own stage inputs, and a
    captured graph of the chain replays to the eager bits."""
    dim, kv, hidden = 3584, 512, 18944
    t4, t6 = B.Q4_K, B.Q6_K
    raw = {}
    dts = {}
    for name, t, r, c, seed in [("q", t4, dim, dim, 1), ("k", t4, kv, dim, 2), ("v", t4, kv, dim, 3),
                                ("o", t4, dim, dim, 4), ("gate", t4, hidden, dim, 5), ("up", t4, hidden, dim, 6),
                                ("down", t6, dim, hidden, 7)]:
        raw[name], dts[name] = _tensor(qmv, t, r, c, 120 + seed)
    rng = np.random.default_rng(130)
    x0 = qmv.synth_normal(dim, seed=131)
    w_attn = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    w_ffn = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    bq, bk, bv = [(rng.standard_normal(r) * 0.1).astype(np.float32) for r in (dim, kv, kv)]
    B_ = hip.DeviceBuffer
    d = {"x0": B_.from_array(x0), "w_attn": B_.from_array(w_attn), "w_ffn": B_.from_array(w_ffn),
         "bq": B_.from_array(bq), "bk": B_.from_array(bk), "bv": B_.from_array(bv)}
    for name, n in [("h", dim), ("q", dim), ("k", kv), ("v", kv), ("x1", dim), ("h2", dim), ("act", hidden),
                    ("x2", dim)]:
        d[name] = B_(4 * n)
    stream = hip.Stream()

    def chain():
        s = stream.handle
        qmv.device_rms_norm(d["x0"].ptr, d["w_attn"].ptr, dim, 1, EPS, d["h"].ptr, s)
        qmv.device_matvec_add_group([dts["q"], dts["k"], dts["v"]], d["h"].ptr, 1,
                                    [d["bq"].ptr, d["bk"].ptr, d["bv"].ptr], [0, 0, 0],
                                    [d["q"].ptr, d["k"].ptr, d["v"].ptr], s)
        qmv.device_matvec_add_group([dts["o"]], d["q"].ptr, 1, [d["x0"].ptr], [dim], [d["x1"].ptr], s)
        qmv.device_rms_norm(d["x1"].ptr, d["w_ffn"].ptr, dim, 1, EPS, d["h2"].ptr, s)
        qmv.device_matvec_swiglu(dts["gate"], dts["up"], d["h2"].ptr, 1, d["act"].ptr, s)
        qmv.device_matvec_add_group([dts["down"]], d["act"].ptr, 1, [d["x1"].ptr], [dim], [d["x2"].ptr], s)

    chain()
    stream.synchronize()
    got = {k: d[k].to_array(np.float32, (d[k].nbytes // 4,)) for k in ("h", "q", "k", "v", "x1", "h2", "act", "x2")}

    def rows_ok(name, t, r, c, xin, y, addend=None):
        y_ref = oracle.matvec(raw[name], t, r, c, xin).astype(np.float64)
        _, absdot = oracle.row_stats(raw[name], t, r, c, xin)
        base = y.astype(np.float64) - (addend if addend is not None else 0)
        # y = fl(row + addend): allow the row bar plus the rounding of the add.
        slack = 2.0 ** -24 * np.abs(y.astype(np.float64))
        assert (np.abs(base - y_ref) <= TOL * absdot + slack).all(), name

    assert (np.abs(got["h"] - _rms_f64(x0, w_attn)) <= RMS_REL * np.abs(_rms_f64(x0, w_attn)) + 1e-30).all()
    rows_ok("q", t4, dim, dim, got["h"], got["q"], bq)
    rows_ok("k", t4, kv, dim, got["h"], got["k"], bk)
    rows_ok("v", t4, kv, dim, got["h"], got["v"], bv)
    rows_ok("o", t4, dim, dim, got["q"], got["x1"], x0)
    ref_h2 = _rms_f64(got["x1"], w_ffn)
    assert (np.abs(got["h2"] - ref_h2) <= RMS_REL * np.abs(ref_h2) + 1e-30).all()
    g_ref = oracle.matvec(raw["gate"], t4, hidden, dim, got["h2"])
    u_ref = oracle.matvec(raw["up"], t4, hidden, dim, got["h2"])
    _, act_ref = oracle.swiglu(g_ref, u_ref)
    # The activation's inputs differ from the oracle's by the row bar, so the
    # chain compares it loosely; test_swiglu_fused_matches_oracle holds the
    # element rule to a few ulp on identical inputs.
    _, g_abs = oracle.row_stats(raw["gate"], t4, hidden, dim, got["h2"])
    _, u_abs = oracle.row_stats(raw["up"], t4, hidden, dim, got["h2"])
    bound = 1.2 * (np.abs(u_ref) * TOL * g_abs + np.abs(g_ref) * TOL * u_abs) + 1e-6 * np.abs(act_ref) + 1e-12
    assert (np.abs(got["act"].astype(np.float64) - act_ref) <= bound).all()
    rows_ok("down", t6, dim, hidden, got["act"], got["x2"], got["x1"])

    g = hip.Graph(stream)
    g.begin()
    chain()
    g.end()
    for i in range(3):
        for k in ("h", "q", "k", "v", "x1", "h2", "act", "x2"):
            d[k].fill(0)
        g.replay()
        stream.synchronize()
        for k in ("h", "q", "k", "v", "x1", "h2", "act", "x2"):
            assert np.array_equal(_bits(d[k].to_array(np.float32, (d[k].nbytes // 4,))), _bits(got[k])), (i, k)
        chain()  # eager work between replays
        stream.synchronize()
    for dt in dts.values():
        dt.close()


def test_concurrent_streams_share_weights(qmv, gpu, hip):
    """Four host threads, each with its own stream and buffers, drive the
    fused SwiGLU, the in-place residual and a 20-position prefill launch on
    shared device tensors at once; every thread gets the single-threaded
    bits (each stream has its own workspace: partials, counters, pair
    counts)."""
    import threading
    t4, t6 = B.Q4_K, B.Q6_K
    dim, hidden = 1536, 4864
    _, dg = _tensor(qmv, t4, hidden, dim, 140)
    _, du = _tensor(qmv, t4, hidden, dim, 141)
    _, dd = _tensor(qmv, t6, dim, hidden, 142)
    n_threads, positions = 4, 20

    def run(i, stream):
        x = qmv.synth_normal(dim, seed=150 + i)
        xp = qmv.synth_normal(positions * dim, seed=160 + i)
        dx, dxp = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(xp)
        act = hip.DeviceBuffer(4 * hidden)
        resid = hip.DeviceBuffer.from_array(qmv.synth_normal(dim, seed=170 + i))
        pre = hip.DeviceBuffer(4 * positions * hidden)
        qmv.device_matvec_swiglu(dg, du, dx.ptr, 1, act.ptr, stream.handle)
        qmv.device_matvec_add_group([dd], act.ptr, 1, [resid.ptr], [dim], [resid.ptr], stream.handle)
        dg.matvec(dxp.ptr, positions, pre.ptr, stream.handle)
        stream.synchronize()
        return (act.to_array(np.float32, (hidden,)), resid.to_array(np.float32, (dim,)),
                pre.to_array(np.float32, (positions * hidden,)))

    ref = [run(i, hip.Stream()) for i in range(n_threads)]
    errors = []

    def worker(i):
        try:
            s = hip.Stream()
            for _ in range(8):
                got = run(i, s)
                for a, b in zip(got, ref[i]):
                    if not np.array_equal(_bits(a), _bits(b)):
                        errors.append(i)
        except Exception as e:  # pragma: no cover
            errors.append(repr(e))

    th = [threading.Thread(target=worker, args=(i,)) for i in range(n_threads)]
    for h in th:
        h.start()
    for h in th:
        h.join()
    assert not errors, errors
    for d in (dg, du, dd):
        d.close()
