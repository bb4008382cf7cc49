"""GPU parity: the HIP path against the CPU oracle, through the C ABI.

Bars (from the path's contract):
  * dequantisation: bit-identical to the reference decoders (all bits,
    including the sign of zero; NaN compared by class);
  * matvec / matmul rows: |y - y_oracle| <= 1e-5 * sum_k |w_k x_k| per row,
    y_oracle the scalar fp32 oracle, the sum in float64 (TOL below);
  * greedy argmax: the same index as the CPU argmax (lowest id on ties).
"""
import ctypes
import os
import sys
import threading

import numpy as np
import pytest

import _blocks as B

pytestmark = pytest.mark.gpu

TOL = 1e-5  # relative to sum |w x| per row


def log(msg):
    print(msg, flush=True)


def check_rows(y, y_ref, absdot, what=""):
    y = np.asarray(y, dtype=np.float64).ravel()
    y_ref = np.asarray(y_ref, dtype=np.float64).ravel()
    absdot = np.asarray(absdot, dtype=np.float64).ravel()
    err = np.abs(y - y_ref)
    bad = err > TOL * absdot
    assert not bad.any(), (f"{what}: {bad.sum()} rows over tolerance; worst err/absdot "
                           f"{np.max(err / np.maximum(absdot, 1e-300)):.3e} at row {int(np.argmax(err - TOL * absdot))}")
    return float(np.max(err / np.maximum(absdot, 1e-300)))


def matvec_parity(qmv, oracle, t, rows, cols, batch=1, seed=1, x=None, offset=0, what=""):
    raw = qmv.synth_tensor(t, rows, cols, seed=seed)
    if offset:
        buf = np.zeros(raw.size + offset, dtype=np.uint8)
        buf[offset:] = raw
    else:
        buf = raw
    if x is None:
        x = qmv.synth_normal(batch * cols, seed=seed + 1000).reshape(batch, cols)
    v = qmv.make_view(buf, t, rows, cols, offset)
    y = qmv.matvec(v, x if batch > 1 else x[0])
    y = y.reshape(batch, rows)
    y_ref = oracle.matvec(raw, t, rows, cols, x if batch > 1 else x[0]).reshape(batch, rows)
    worst = 0.0
    for b in range(batch):
        _, absdot = oracle.row_stats(raw, t, rows, cols, x[b])
        worst = max(worst, check_rows(y[b], y_ref[b], absdot, f"{what} pos {b}"))
    log(f"{what} {B.BLOCK_BYTES and t} {rows}x{cols} M={batch}: worst err/sum|wx| = {worst:.2e}")
    qmv.release_tensor(v.data)
    return y


# ---- dequantisation, bit for bit ----------------------------------------------------

def _dequant_compare(qmv, oracle, raw, t, rows, cols, first=0, count=None, offset=0):
    count = rows - first if count is None else count
    buf = raw
    if offset:
        buf = np.zeros(raw.size + offset, dtype=np.uint8)
        buf[offset:] = raw
    v = qmv.make_view(buf, t, rows, cols, offset)
    got = qmv.dequantize_rows(v, first, count)
    exp = oracle.dequantize_rows(raw, t, rows, cols, first, count)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))
    qmv.release_tensor(v.data)


@pytest.mark.parametrize("t", B.ALL_TYPES)
@pytest.mark.parametrize("rows,nblk", [(1, 1), (17, 3), (64, 4), (65, 5), (130, 9), (200, 16)])
def test_dequant_bit_exact_random_blocks(qmv, oracle, gpu, t, rows, nblk):
    """Random bytes with normal, subnormal, negative and zero fp16 scales;
    row counts off the 64-row tile and (Q8_0/Q5_0) partial 4-block units."""
    raw = B.raw_blocks(t, rows * nblk, seed=rows * 31 + nblk + t)
    _dequant_compare(qmv, oracle, raw, t, rows, nblk * B.BLOCK_ELEMENTS[t], offset=1)


def test_dequant_all_f16_scales(qmv, oracle, gpu):
    """Every fp16 scale code through the device decoder (Q8_0 rows with
    code r as scale and codes 1, 0, -1 in the first three weights)."""
    rows = 65536
    raw = np.zeros((rows, 34), dtype=np.uint8)
    codes = np.arange(rows, dtype=np.uint16)
    raw[:, 0] = codes & 0xFF
    raw[:, 1] = codes >> 8
    raw[:, 2] = 1
    raw[:, 4] = 0xFF
    _dequant_compare(qmv, oracle, raw.ravel(), B.Q8_0, rows, 32)


@pytest.mark.parametrize("t,rows,cols", [
    (B.Q8_0, 896, 896), (B.Q6_K, 896, 4864), (B.Q5_0, 1536, 1536), (B.Q5_0, 256, 1536),
    (B.Q4_K, 8960, 1536), (B.Q4_K, 1536, 8960), (B.Q4_K, 3584, 3584), (B.Q4_K, 512, 3584),
    (B.Q4_K, 18944, 3584), (B.Q6_K, 3584, 18944)])
def test_dequant_bit_exact_config_shapes(qmv, oracle, gpu, t, rows, cols):
    raw = qmv.synth_tensor(t, rows, cols, seed=rows + cols)
    _dequant_compare(qmv, oracle, raw, t, rows, cols)


def test_dequant_bit_exact_vocab_rows(qmv, oracle, gpu):
    rows, cols = 151936, 3584
    raw = qmv.synth_tensor(B.Q6_K, rows, cols, seed=4)
    for first, count in ((0, 300), (75000, 129), (rows - 70, 70)):
        _dequant_compare(qmv, oracle, raw, B.Q6_K, rows, cols, first, count)


# ---- known answers through the drop-in ----------------------------------------------------

def test_matvec_kats(qmv, gpu):
    k = B.KATS["matvec_q8_0_two_rows"]
    raw = np.frombuffer(b"".join(B.q8_0_block(bk["d"], bk["qs"]) for bk in k["blocks"]), dtype=np.uint8).copy()
    v = qmv.make_view(raw, B.Q8_0, 2, 32)
    assert list(qmv.matvec(v, B.sparse_vector(32, k["x"]))) == k["expected"]
    one = B.sparse_vector(256, {"0": 1.0})
    for t, blk, cols, key in (
            (B.Q5_0, B.q5_0_block(0x3800, {}, {}), 32, "matvec_q5_0_single"),
            (B.Q4_K, B.q4_k_block(0x3800, 0x3400, [1, 0, 0, 0, 1] + [0] * 7, {}), 256, "matvec_q4_k_single"),
            (B.Q6_K, B.q6_k_block(0x3800, [1] + [0] * 15, 0, {}), 256, "matvec_q6_k_single")):
        raw = np.frombuffer(blk, dtype=np.uint8).copy()
        v = qmv.make_view(raw, t, 1, cols)
        assert qmv.matvec(v, one[:cols])[0] == B.KATS[key]["expected"]
    # single-block dot KATs as 1-row matrices
    for t, blk, xs, key in ((B.Q8_0, B.kat_block("q8_0_dot"), B.KATS["q8_0_dot"]["x"], "q8_0_dot"),
                            (B.Q5_0, B.kat_block("q5_0"), B.KATS["q5_0_dot"]["x"], "q5_0_dot"),
                            (B.Q4_K, B.kat_block("q4_k"), B.KATS["q4_k_dot"]["x"], "q4_k_dot")):
        raw = np.frombuffer(blk, dtype=np.uint8).copy()
        n = B.BLOCK_ELEMENTS[t]
        v = qmv.make_view(raw, t, 1, n)
        assert abs(qmv.matvec(v, B.sparse_vector(n, xs))[0] - B.KATS[key]["expected"]) <= 1e-5
    raw = np.frombuffer(B.kat_block("q6_k"), dtype=np.uint8).copy()
    x = np.zeros(256, dtype=np.float32)
    x[B.KATS["q6_k_dot"]["x_ones_at"]] = 1.0
    assert abs(qmv.matvec(qmv.make_view(raw, B.Q6_K, 1, 256), x)[0] - B.KATS["q6_k_dot"]["expected"]) <= 1e-5


@pytest.mark.parametrize("t", B.ALL_TYPES)
def test_multirow_unaligned_with_sentinels(qmv, gpu, t):
    """tests/quantized_matvec_reference_test.cpp:156-202: 17 rows x 3 blocks at
    data+1, outputs written between two sentinels, results deterministic."""
    rows, bpr, be, bb = 17, 3, B.BLOCK_ELEMENTS[t], B.BLOCK_BYTES[t]
    cols = bpr * be
    storage = np.zeros(1 + rows * bpr * bb, dtype=np.uint8)
    vals = np.zeros((rows, bpr), dtype=np.float32)
    for r in range(rows):
        for b in range(bpr):
            idx = r * bpr + b
            blk, val = B.fixture_block(t, idx)
            storage[1 + idx * bb:1 + (idx + 1) * bb] = np.frombuffer(blk, dtype=np.uint8)
            vals[r, b] = val
    x = ((np.arange(cols) % 13 - 6) / 8.0).astype(np.float32)
    expected = np.array([sum(float(vals[r, b]) * float(x[b * be + c]) for b in range(bpr) for c in range(be))
                         for r in range(rows)])
    v = qmv.make_view(storage, t, rows, cols, offset=1)
    out = np.full(rows + 2, -999.0, dtype=np.float32)
    outv = out[1:-1]
    assert qmv.quantized_tensor_matvec_f32(v, x, cols, outv, rows) == 1
    assert out[0] == -999.0 and out[-1] == -999.0
    assert np.all(np.abs(outv - expected) <= 1e-5)
    again = np.empty(rows, dtype=np.float32)
    assert qmv.quantized_tensor_matvec_f32(v, x, cols, again, rows) == 1
    assert np.array_equal(again.view(np.uint32), outv.view(np.uint32))
    qmv.release_tensor(v.data)


def test_fixture_matvec_exact(qmv, gpu):
    """tests/qwen2_weight_reference_test.cpp:152-181: 3 rows x 2 constant
    blocks, input 1 then 2: every output exactly block_elements*(v0 + 2 v1)."""
    for t in B.ALL_TYPES:
        be, bb = B.BLOCK_ELEMENTS[t], B.BLOCK_BYTES[t]
        storage = np.zeros(1 + 6 * bb, dtype=np.uint8)
        vals = []
        for b in range(6):
            blk, val = B.fixture_block(t, b)
            storage[1 + b * bb:1 + (b + 1) * bb] = np.frombuffer(blk, dtype=np.uint8)
            vals.append(val)
        x = np.where(np.arange(2 * be) < be, 1.0, 2.0).astype(np.float32)
        y = qmv.matvec(qmv.make_view(storage, t, 3, 2 * be, offset=1), x)
        for r in range(3):
            assert y[r] == np.float32(be * (vals[2 * r] + 2 * vals[2 * r + 1])), (t, r)


def test_invalid_arguments_leave_output(qmv, gpu):
    raw = np.zeros(34, dtype=np.uint8)
    v = qmv.make_view(raw, B.Q8_0, 1, 32)
    x = np.zeros(32, dtype=np.float32)
    y = np.full(2, -7.0, dtype=np.float32)
    assert qmv.quantized_tensor_matvec_f32(v, x, 31, y, 1) == 0
    assert qmv.quantized_tensor_matvec_f32(v, x, 32, y, 2) == 0
    assert qmv.quantized_tensor_matmul_f32(v, x, 32, 0, y, 1) == 0
    assert (y == -7.0).all()
    raw = np.zeros(16, dtype=np.uint8)
    v = qmv.make_view(raw, B.Q4_K, 4864, 896)  # Q4_K 4864x896: K % 256 != 0
    assert qmv.quantized_tensor_matvec_f32(v, np.zeros(896, np.float32), 896, np.zeros(4864, np.float32), 4864) == 0


def test_failure_injection_publishes_nothing(qmv, gpu):
    """Forced failure after the kernel: the call returns 0 and the caller's
    output is untouched; the next call succeeds (the role of
    tests/quantized_matvec_failure_test.cpp)."""
    raw = qmv.synth_tensor(B.Q4_K, 64, 512, seed=3)
    v = qmv.make_view(raw, B.Q4_K, 64, 512)
    x = qmv.synth_normal(512, seed=4)
    y = np.full(64, -99.0, dtype=np.float32)
    qmv.hip_lib().qmv_debug_fail_next_calls(1)
    assert qmv.quantized_tensor_matvec_f32(v, x, 512, y, 64) == 0
    assert (y == -99.0).all()
    assert "inject" in qmv.last_error()
    assert qmv.quantized_tensor_matvec_f32(v, x, 512, y, 64) == 1
    assert np.isfinite(y).all()
    qmv.hip_lib().qmv_debug_fail_next_calls(0)


# ---- parity at the workload shapes ----------------------------------------------------------

def test_q8_0_896x896_q_proj(qmv, oracle, gpu):
    x = qmv.synth_normal(896, seed=0).reshape(1, 896)
    matvec_parity(qmv, oracle, B.Q8_0, 896, 896, seed=0, x=x, what="Q8_0 896x896")


def test_q6_k_896x4864_down(qmv, oracle, gpu):
    matvec_parity(qmv, oracle, B.Q6_K, 896, 4864, seed=2, what="Q6_K 896x4864")


@pytest.mark.parametrize("t,rows,cols", [(B.Q5_0, 1536, 1536), (B.Q5_0, 256, 1536), (B.Q4_K, 8960, 1536),
                                         (B.Q4_K, 1536, 8960)])
def test_qwen2_1_5b_prefill_m8(qmv, oracle, gpu, t, rows, cols):
    matvec_parity(qmv, oracle, t, rows, cols, batch=8, seed=3, what="1.5B prefill M=8")


@pytest.mark.parametrize("t,rows,cols", [(B.Q4_K, 3584, 3584), (B.Q4_K, 512, 3584), (B.Q4_K, 18944, 3584),
                                         (B.Q6_K, 3584, 18944)])
@pytest.mark.parametrize("batch", [1, 8])
def test_qwen2_7b_layer_shapes(qmv, oracle, gpu, t, rows, cols, batch):
    matvec_parity(qmv, oracle, t, rows, cols, batch=batch, seed=5, what="7B layer")


@pytest.mark.parametrize("t", B.ALL_TYPES)
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 6, 7, 8, 11])
def test_every_batch_size(qmv, oracle, gpu, t, batch):
    cols = 3 * B.BLOCK_ELEMENTS[t] if t in (B.Q4_K, B.Q6_K) else 7 * 32
    matvec_parity(qmv, oracle, t, 200, cols, batch=batch, seed=batch, offset=1, what=f"batch {batch}")


@pytest.mark.parametrize("t", B.ALL_TYPES)
@pytest.mark.parametrize("rows,cols", [(1, 256), (63, 512), (64, 1024), (65, 2304), (1000, 256 * 37)])
def test_odd_shapes(qmv, oracle, gpu, t, rows, cols):
    matvec_parity(qmv, oracle, t, rows, cols, seed=rows + cols, what="odd shape")


def _random_cases(n, seed):
    """Seeded shapes across every launch-plan branch: rows off the 64-row tile,
    short and long rows (one to 40 super-blocks, or 1 to 80 blocks of 32 with
    partial 4-block units), and batches of 1 to 40 (VALU half units, matrix
    cores, prefill launches, chunks past 32)."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        t = B.ALL_TYPES[i % len(B.ALL_TYPES)]
        rows = int(rng.integers(1, 700))
        if t in (B.Q4_K, B.Q6_K):
            cols = 256 * int(rng.integers(1, 41))
        else:
            cols = 32 * int(rng.integers(1, 81))
        batch = int(rng.choice([1, 1, 2, 3, 4, 5, 6, 7, 8, 9, 16, 17, 31, 32, 33, 40]))
        cases.append((t, rows, cols, batch, 5000 + i))
    return cases


@pytest.mark.parametrize("t,rows,cols,batch,seed", _random_cases(48, 2026))
def test_random_shapes_match_oracle(qmv, oracle, gpu, t, rows, cols, batch, seed):
    matvec_parity(qmv, oracle, t, rows, cols, batch=batch, seed=seed, what=f"random {rows}x{cols} M={batch}")


SWEEP_PLANS = [(0, 0, 0, 0)] * 6 + [(0, 2, 0, 0), (0, 0, 8, 0), (0, 0, 2, 0), (4096, 0, 0, 0), (0, 0, 0, 2),
                                   (0, 1, 5, 0), (0, 0, 0, 20)]


def test_random_sweep_with_plans(qmv, oracle, gpu):
    """600 seeded cases in one test: any format, 1..3000 rows, K up to 29
    super-blocks or 159 blocks of 32 (rows of up to 40 four-block units, so
    the prefill plans for long rows run too), batches of 1..50, under the
    default plan (half the cases) or a forced one (units per wave, waves per
    group, target waves, matrix cores from two positions or only from 20, which
    leaves tails of 9..19 positions to launches of 8)."""
    rng = np.random.default_rng(77)
    worst = 0.0
    for i in range(600):
        t = B.ALL_TYPES[int(rng.integers(0, 4))]
        rows = int(rng.choice([int(rng.integers(1, 200)), int(rng.integers(200, 3000))]))
        cols = 256 * int(rng.integers(1, 30)) if t in (B.Q4_K, B.Q6_K) else 32 * int(rng.integers(1, 160))
        batch = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 17, 24, 31, 32, 33, 40, 50]))
        plan = SWEEP_PLANS[int(rng.integers(0, len(SWEEP_PLANS)))]
        raw = qmv.synth_tensor(t, rows, cols, seed=20000 + i)
        x = qmv.synth_normal(batch * cols, seed=30000 + i).reshape(batch, cols)
        v = qmv.make_view(raw, t, rows, cols)
        qmv.set_launch_tuning(*plan)
        try:
            y = qmv.matvec(v, x if batch > 1 else x[0]).reshape(batch, rows)
        finally:
            qmv.set_launch_tuning(0, 0, 0, 0)
        y_ref = oracle.matvec(raw, t, rows, cols, x if batch > 1 else x[0]).reshape(batch, rows)
        for b in range(batch):
            _, absdot = oracle.row_stats(raw, t, rows, cols, x[b])
            worst = max(worst, check_rows(y[b], y_ref[b], absdot,
                                          f"case {i}: type {t} {rows}x{cols} M={batch} plan {plan} pos {b}"))
        qmv.release_tensor(v.data)
        if i % 100 == 0:
            log(f"sweep case {i}: type {t} {rows}x{cols} M={batch} plan {plan}; worst so far {worst:.2e}")
    log(f"sweep: 600 cases, worst err/sum|wx| = {worst:.2e}")


@pytest.mark.parametrize("t", B.ALL_TYPES)
@pytest.mark.parametrize("batch", [1, 8, 20])
@pytest.mark.parametrize("scale", ["1e-28", "1e28", "mixed"])
def test_activation_dynamic_range(qmv, oracle, gpu, t, batch, scale):
    """Activations far from N(0,1) stay within the row bar on every kernel:
    M = 1 on the VALU (Q4_K/Q6_K codes on v_fma_mix_f32, whose sums run scaled
    by 2^-24), M = 8 on the matrix cores (exact bf16 limbs), 20 positions in
    the prefill kernel (Q8_0/Q5_0: passes of 8 on the VALU). The whole vector
    at 1e-28 or 1e28, or magnitudes from 1e-20 to 1e20 element by element."""
    cols = 4 * 256
    rng = np.random.default_rng(batch * 7 + len(scale))
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    if scale == "mixed":
        x *= (10.0 ** rng.integers(-20, 21, size=x.shape)).astype(np.float32)
    else:
        x *= np.float32(float(scale))
    assert np.isfinite(x).all()
    matvec_parity(qmv, oracle, t, 130, cols, batch=batch, seed=batch + 90, x=x, what=f"range {scale}")


# Launch plans: (target_waves, units_per_wave, waves_per_group,
# mfma_min_batch). The default gives every wave one unit (the single-unit
# kernel variant) and runs Q4_K batches of 7 or more and Q6_K batches of 8 on
# the matrix cores; the others run the two-unit pipelined variant, one wave per
# workgroup, whole-K workgroups (no split), target-sized units, the VALU path
# for every batch of up to 8 (mfma_min_batch 9) and the matrix cores from batch 2.
PLANS = [(0, 0, 0, 0), (0, 2, 0, 0), (0, 3, 7, 0), (0, 1, 1, 0), (0, 1, 8, 0), (2048, 0, 0, 0), (0, 2, 1, 0),
         (0, 8, 8, 0), (0, 5, 3, 0), (0, 0, 0, 9), (0, 2, 0, 9), (0, 3, 7, 9), (0, 0, 0, 2), (0, 2, 0, 2)]


@pytest.mark.parametrize("plan", PLANS)
@pytest.mark.parametrize("t", B.ALL_TYPES)
def test_launch_plans_match_oracle(qmv, oracle, gpu, plan, t):
    """Every plan stays within tolerance, including a partial last unit
    (Q8_0/Q5_0 with K = 7 blocks of 32) and batches of 3 and 8."""
    cols = 5 * B.BLOCK_ELEMENTS[t] if t in (B.Q4_K, B.Q6_K) else 7 * 32 + 512
    qmv.set_launch_tuning(*plan)
    try:
        for batch in (1, 3, 8):
            matvec_parity(qmv, oracle, t, 130, cols, batch=batch, seed=batch + 40, what=f"plan {plan}")
    finally:
        qmv.set_launch_tuning(0, 0, 0, 0)


def test_vocab_151936x3584_projection_and_argmax(qmv, oracle, gpu):
    """Q6_K 151936 x 3584 (446 MB) then greedy argmax: the index equals the
    CPU argmax of the oracle's logits."""
    rows, cols = 151936, 3584
    raw = qmv.synth_tensor(B.Q6_K, rows, cols, seed=4)
    x = qmv.synth_normal(cols, seed=44)
    v = qmv.make_view(raw, B.Q6_K, rows, cols)
    y = qmv.matvec(v, x)
    y_ref = oracle.matvec(raw, B.Q6_K, rows, cols, x)
    dot, absdot = oracle.row_stats(raw, B.Q6_K, rows, cols, x)
    check_rows(y, y_ref, absdot, "C4")
    ok_cpu, tok_cpu = oracle.greedy_argmax(y_ref)
    ok_gpu, tok_gpu = qmv.greedy_sample(y)
    assert ok_cpu == 1 and ok_gpu == 1
    srt = np.sort(y_ref)
    gap = float(srt[-1] - srt[-2])
    bound = 2 * TOL * float(absdot[tok_cpu])
    log(f"vocab argmax {tok_cpu}: top-2 gap {gap:.3e} vs row error bound {bound:.3e}")
    assert tok_gpu == tok_cpu
    assert qmv.greedy_sample(y_ref) == (1, tok_cpu)
    qmv.release_tensor(v.data)


def test_greedy_argmax_contract(qmv, gpu):
    rng = np.random.default_rng(11)
    for n in (1, 7, 4096, 4097, 151936, 1 << 21):
        x = rng.standard_normal(n).astype(np.float32)
        assert qmv.greedy_sample(x) == (1, int(np.argmax(x)))
    x = np.zeros(100000, dtype=np.float32)
    x[[777, 5000, 99999]] = 3.0
    assert qmv.greedy_sample(x) == (1, 777)  # lowest id on ties
    for bad in (np.nan, np.inf, -np.inf):
        y = rng.standard_normal(5000).astype(np.float32)
        y[4321] = bad
        assert qmv.greedy_sample(y) == (0, -1)


# ---- engine contracts ------------------------------------------------------------------------

def test_deterministic_and_thread_safe(qmv, gpu):
    """Bit-identical results run to run and from 4 concurrent host threads
    sharing the same weights (sessions of include/engine_api.h:10-17)."""
    t, rows, cols = B.Q4_K, 3584, 3584
    raw = qmv.synth_tensor(t, rows, cols, seed=9)
    v = qmv.make_view(raw, t, rows, cols)
    xs = [qmv.synth_normal(cols, seed=100 + i) for i in range(4)]
    ref = [qmv.matvec(v, x) for x in xs]
    for i in range(4):
        assert np.array_equal(qmv.matvec(v, xs[i]).view(np.uint32), ref[i].view(np.uint32))
    errors = []

    def worker(i):
        try:
            for _ in range(20):
                y = qmv.matvec(v, xs[i])
                if not np.array_equal(y.view(np.uint32), ref[i].view(np.uint32)):
                    errors.append(i)
        except Exception as e:  # pragma: no cover
            errors.append(repr(e))

    th = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for h in th:
        h.start()
    for h in th:
        h.join()
    assert not errors
    qmv.release_tensor(v.data)


def test_cache_follows_new_contents(qmv, gpu):
    """A host buffer reused for another tensor is re-uploaded: explicitly via
    qmv_release_tensor, and by the content fingerprint otherwise."""
    t, rows, cols = B.Q6_K, 256, 1024
    buf = qmv.synth_tensor(t, rows, cols, seed=1)
    v = qmv.make_view(buf, t, rows, cols)
    x = qmv.synth_normal(cols, seed=2)
    y1 = qmv.matvec(v, x)
    buf[:] = qmv.synth_tensor(t, rows, cols, seed=2)
    y2 = qmv.matvec(v, x)
    assert not np.array_equal(y1, y2)
    assert qmv.release_tensor(v.data) >= 1
    buf[:] = qmv.synth_tensor(t, rows, cols, seed=1)
    assert np.array_equal(qmv.matvec(v, x), y1)
    assert qmv.register_tensor(v) == 1
    qmv.release_all()


def test_cxx_dropin_program(qmv, gpu):
    """The drop-in from C++ (tests/cxx/dropin_test.cpp): quantized_tensor_
    matvec_f32 / _matmul_f32 with their original signatures on all four
    formats, M = 1 to 40, each row within tolerance of the oracle."""
    import subprocess
    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cxx", "dropin_test")
    assert os.path.exists(exe), "tests/cxx/dropin_test missing: run __graft_entry__.build()"
    log("running tests/cxx/dropin_test")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.fixture(scope="module")
def hip(qmv):
    import importlib
    return importlib.import_module("my-inference-engine_amd.hip_runtime")


@pytest.mark.parametrize("t,rows,cols", [(B.Q4_K, 18944, 3584), (B.Q6_K, 3584, 18944)])
def test_device_api_matches_host_api(qmv, gpu, hip, t, rows, cols):
    """The host-pointer drop-in (input copied in, or for 32 KB and more read
    by a copy kernel; output written by the kernels into pinned memory) gives
    the device API's bits, at M = 1, 8 and 32."""
    raw = qmv.synth_tensor(t, rows, cols, seed=21)
    v = qmv.make_view(raw, t, rows, cols)
    dt = qmv.DeviceTensor(v)
    assert (dt.rows, dt.cols, dt.packed_bytes) == (rows, cols, raw.size)
    x = qmv.synth_normal(32 * cols, seed=22).reshape(32, cols)
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(32 * rows * 4)
    stream = hip.Stream()
    for m in (1, 8, 32):
        dt.matvec(dx.ptr, m, dy.ptr, stream.handle)
        stream.synchronize()
        host = qmv.matvec(v, x[:m] if m > 1 else x[0]).reshape(m, rows)
        got = dy.to_array(np.float32, (32, rows))[:m]
        assert np.array_equal(got.view(np.uint32), host.view(np.uint32)), m
    out = hip.DeviceBuffer(5 * cols * 4)
    dt.dequantize(100, 5, out.ptr, stream.handle)
    stream.synchronize()
    assert np.array_equal(out.to_array(np.float32, (5, cols)).view(np.uint32),
                          qmv.dequantize_rows(v, 100, 5).view(np.uint32))
    dt.close()
    qmv.release_all()


@pytest.mark.parametrize("shapes", [[(3584, 31), (512, 32), (512, 33)], [(18944, 35), (18944, 36)]],
                         ids=["q|k|v", "gate|up"])
def test_group_launch_matches_oracle(qmv, oracle, gpu, hip, shapes):
    """q/k/v (row-major) and gate/up (tiled, 8288 (tile, unit) pairs in
    splits of 4, 4, 4 and 2 units) sharing one input in one launch: each
    within tolerance of the oracle."""
    cols = 3584
    raws = [qmv.synth_tensor(B.Q4_K, r, cols, seed=s) for r, s in shapes]
    dts = [qmv.DeviceTensor(qmv.make_view(raw, B.Q4_K, r, cols)) for raw, (r, _) in zip(raws, shapes)]
    x = qmv.synth_normal(cols, seed=34)
    dx = hip.DeviceBuffer.from_array(x)
    outs = [hip.DeviceBuffer(4 * r) for r, _ in shapes]
    stream = hip.Stream()
    qmv.device_matvec_group(dts, dx.ptr, 1, [o.ptr for o in outs], stream.handle)
    stream.synchronize()
    for raw, (r, _), o in zip(raws, shapes, outs):
        y_ref = oracle.matvec(raw, B.Q4_K, r, cols, x)
        _, absdot = oracle.row_stats(raw, B.Q4_K, r, cols, x)
        check_rows(o.to_array(np.float32, (r,)), y_ref, absdot, "group")
    for d in dts:
        d.close()


@pytest.mark.parametrize("t,rows,cols,batch", [(B.Q6_K, 3584, 18944, 1), (B.Q6_K, 1000, 3584, 1),
                                               (B.Q4_K, 3584, 3584, 8), (B.Q6_K, 896, 4864, 8),
                                               (B.Q4_K, 512, 3584, 3)])
def test_graph_replays_match_eager(qmv, gpu, hip, t, rows, cols, batch):
    """A captured launch (split-K counters reset by the kernel itself, no
    memset nodes) replays to the eager result, with host work in between; at
    M = 8 the launch runs on the matrix cores. Q6_K 3584 x 18944 at one
    position runs row-major (no split); Q6_K 1000 x 3584 (14 K-units, tiled)
    splits K at one position."""
    raw = qmv.synth_tensor(t, rows, cols, seed=61)
    dt = qmv.DeviceTensor(qmv.make_view(raw, t, rows, cols))
    x = qmv.synth_normal(batch * cols, seed=62)
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(4 * rows * batch)
    stream = hip.Stream()
    dt.matvec(dx.ptr, batch, dy.ptr, stream.handle)  # sizes the stream's workspace
    stream.synchronize()
    eager = dy.to_array(np.float32, (batch * rows,))
    g = hip.Graph(stream)
    g.begin()
    dt.matvec(dx.ptr, batch, dy.ptr, stream.handle)
    g.end()
    for i in range(5):
        dy.fill(0)
        g.replay()
        stream.synchronize()
        assert np.array_equal(dy.to_array(np.float32, (batch * rows,)).view(np.uint32), eager.view(np.uint32)), i
        dt.matvec(dx.ptr, batch, dy.ptr, stream.handle)  # eager work between replays
        stream.synchronize()
    dt.close()


def test_device_argmax(qmv, gpu, hip):
    x = np.random.default_rng(5).standard_normal(151936).astype(np.float32)
    x[[10, 150000]] = 9.0
    dx = hip.DeviceBuffer.from_array(x)
    res = hip.DeviceBuffer(8)
    stream = hip.Stream()
    qmv.device_greedy_argmax(dx.ptr, x.size, res.ptr, stream.handle)
    stream.synchronize()
    assert res.to_array(np.int32, (2,)).tolist() == [10, 1]


# ---- vocabulary projection fused with greedy sampling ----------------------------

def _fused(qmv, hip, raw, t, rows, cols, x, reps=1, graph=False):
    dt = qmv.DeviceTensor(qmv.make_view(raw, t, rows, cols))
    dx = hip.DeviceBuffer.from_array(x)
    dl = hip.DeviceBuffer(4 * rows)
    dref = hip.DeviceBuffer(4 * rows)
    res = hip.DeviceBuffer(8)
    stream = hip.Stream()
    dt.matvec(dx.ptr, 1, dref.ptr, stream.handle)
    outs = []
    g = None
    if graph:
        qmv.device_matvec_argmax(dt, dx.ptr, dl.ptr, res.ptr, stream.handle)  # sizes the workspace
        stream.synchronize()
        g = hip.Graph(stream)
        g.begin()
        qmv.device_matvec_argmax(dt, dx.ptr, dl.ptr, res.ptr, stream.handle)
        g.end()
    for _ in range(reps):
        res.fill(0x55)
        if g is not None:
            g.replay()
        else:
            qmv.device_matvec_argmax(dt, dx.ptr, dl.ptr, res.ptr, stream.handle)
        stream.synchronize()
        outs.append(res.to_array(np.int32, (2,)).tolist())
    logits = dl.to_array(np.float32, (rows,))
    ref = dref.to_array(np.float32, (rows,))
    dt.close()
    return outs, logits, ref


@pytest.mark.parametrize("t,rows,cols", [(B.Q4_K, 1000, 3584), (B.Q6_K, 4864, 896 * 4), (B.Q8_0, 130, 896),
                                         (B.Q5_0, 64, 1536), (B.Q6_K, 7, 18944)])
def test_fused_argmax_matches_its_logits(qmv, oracle, gpu, hip, t, rows, cols):
    """The fused launch writes the same logits as the plain matvec (bit for
    bit) and returns the lowest-index argmax of exactly those logits; the
    logits are within tolerance of the oracle."""
    raw = qmv.synth_tensor(t, rows, cols, seed=rows)
    x = qmv.synth_normal(cols, seed=cols)
    outs, logits, ref = _fused(qmv, hip, raw, t, rows, cols, x, reps=3)
    assert np.array_equal(logits.view(np.uint32), ref.view(np.uint32))
    expect = int(np.argmax(logits))
    assert all(o == [expect, 1] for o in outs), (outs, expect)
    y_ref = oracle.matvec(raw, t, rows, cols, x)
    _, absdot = oracle.row_stats(raw, t, rows, cols, x)
    check_rows(logits, y_ref, absdot, "fused argmax logits")


def test_fused_argmax_vocab_shape_and_graph(qmv, gpu, hip):
    """Vocabulary shape (151936 x 3584 Q6_K): eager and graph-replayed fused
    launches agree with the argmax of their logits on every replay."""
    t, rows, cols = B.Q6_K, 151936, 3584
    raw = qmv.synth_tensor(t, rows, cols, seed=44)
    x = qmv.synth_normal(cols, seed=45)
    outs, logits, ref = _fused(qmv, hip, raw, t, rows, cols, x, reps=4, graph=True)
    assert np.array_equal(logits.view(np.uint32), ref.view(np.uint32))
    expect = int(np.argmax(logits))
    assert all(o == [expect, 1] for o in outs), (outs, expect)


def test_fused_argmax_ties_and_non_finite(qmv, gpu, hip):
    """All-zero input: every logit ties at 0 and the lowest id wins. A row
    with an infinite scale makes its logit non-finite: token -1, flag 0, as
    the reference sampler rejects non-finite logits."""
    t, rows, cols = B.Q8_0, 300, 256
    raw = qmv.synth_tensor(t, rows, cols, seed=9)
    outs, logits, _ = _fused(qmv, hip, raw, t, rows, cols, np.zeros(cols, dtype=np.float32))
    assert outs == [[0, 1]] and not logits.any()
    bad = raw.copy()
    bpr = cols // 32
    bad[(200 * bpr) * 34:(200 * bpr) * 34 + 2] = np.frombuffer(np.uint16(0x7C00).tobytes(), dtype=np.uint8)
    x = qmv.synth_normal(cols, seed=10)
    outs, logits, _ = _fused(qmv, hip, bad, t, rows, cols, x)
    assert not np.isfinite(logits[200])
    assert outs == [[-1, 0]]


# ---- embedding rows gathered by device token ids ------------------------------------

@pytest.mark.parametrize("t,rows,cols", [(B.Q4_K, 1000, 1536), (B.Q6_K, 130, 896 * 4), (B.Q8_0, 151, 7 * 32 + 512),
                                         (B.Q5_0, 64, 1536)])
def test_embed_rows_bit_exact(qmv, oracle, gpu, hip, t, rows, cols):
    """Gathered rows (duplicates, first and last rows, rows of the partial last
    tile) equal the oracle's decode bit for bit; an out-of-range id gives a
    NaN row, leaves the others exact and clears the status word (which a call
    with every id in range sets to 1, src/qwen2_architecture.cpp:384-393)."""
    raw = qmv.synth_tensor(t, rows, cols, seed=rows + 3)
    dt = qmv.DeviceTensor(qmv.make_view(raw, t, rows, cols))
    ids = np.array([0, rows - 1, 5, 5, rows // 2, rows - 2, 63 % rows, rows, -1, 1], dtype=np.int32)
    d_ids = hip.DeviceBuffer.from_array(ids)
    out = hip.DeviceBuffer(4 * ids.size * cols)
    status = hip.DeviceBuffer(4)
    stream = hip.Stream()
    status.fill(0x55)
    qmv.device_embed_rows(dt, d_ids.ptr, 7, out.ptr, stream.handle, d_status=status.ptr)  # ids 0..6: in range
    stream.synchronize()
    assert status.to_array(np.int32, (1,))[0] == 1
    qmv.device_embed_rows(dt, d_ids.ptr, ids.size, out.ptr, stream.handle, d_status=status.ptr)
    stream.synchronize()
    assert status.to_array(np.int32, (1,))[0] == 0
    got = out.to_array(np.float32, (ids.size, cols))
    for i, r in enumerate(ids.tolist()):
        if 0 <= r < rows:
            exp = oracle.dequantize_rows(raw, t, rows, cols, r, 1)[0]
            nan = np.isnan(exp)
            assert np.array_equal(np.isnan(got[i]), nan)
            assert np.array_equal(got[i][~nan].view(np.uint32), exp[~nan].view(np.uint32)), (i, r)
        else:
            assert np.isnan(got[i]).all(), (i, r)
    dt.close()
