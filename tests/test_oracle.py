"""Pin the CPU oracle (oracle/qmv_oracle.c) before it is used to check the GPU.

Each check is independent of the oracle's own code: the ldexp closed form
and numpy's binary16 for f16, the reference tests' known-answer blocks,
exact-rational decoders of the documented equations, the reference's LCG
dot-vs-dequant trials, and bit-for-bit equality with the reference's own
sources compiled into oracle/_ref (when that build exists).
"""
import ctypes
import math

import numpy as np
import pytest

import _blocks as B

pytestmark = []


def _p(a):
    return a.ctypes.data


def _dq(oracle, t, blk):
    fn = {B.Q8_0: "oracle_q8_0_dequantize_block", B.Q5_0: "oracle_q5_0_dequantize_block",
          B.Q4_K: "oracle_q4_k_dequantize_block", B.Q6_K: "oracle_q6_k_dequantize_block"}[t]
    out = np.empty(B.BLOCK_ELEMENTS[t], dtype=np.float32)
    buf = np.frombuffer(bytes(blk), dtype=np.uint8).copy()
    assert getattr(oracle.lib(), fn)(_p(buf), _p(out)) == 1
    return out


def _dot(oracle, t, blk, x):
    fn = {B.Q8_0: "oracle_q8_0_dot_f32", B.Q5_0: "oracle_q5_0_dot_f32",
          B.Q4_K: "oracle_q4_k_dot_f32", B.Q6_K: "oracle_q6_k_dot_f32"}[t]
    buf = np.frombuffer(bytes(blk), dtype=np.uint8).copy()
    x = np.ascontiguousarray(x, dtype=np.float32)
    r = np.zeros(1, dtype=np.float32)
    assert getattr(oracle.lib(), fn)(_p(buf), _p(x), _p(r)) == 1
    return r[0]


# ---- f16 ----------------------------------------------------------------------

def test_f16_all_codes_closed_form(oracle):
    """tests/q8_0_reference_test.cpp:48-64: every code vs ldexp, bit for bit."""
    lib = oracle.lib()
    out = np.array([lib.oracle_f16_to_f32(c) for c in range(65536)], dtype=np.float32)
    codes = np.arange(65536)
    exp5, frac = (codes >> 10) & 31, codes & 1023
    finite = exp5 != 31
    expected = np.where(exp5 == 0, np.ldexp(frac.astype(np.float64), -24),
                        np.ldexp((1024 + frac).astype(np.float64), exp5.astype(np.int64) - 25))
    expected = np.where(codes & 0x8000, -expected, expected).astype(np.float32)
    assert np.array_equal(out[finite].view(np.uint32), expected[finite].view(np.uint32))
    nan = (~finite) & (frac != 0)
    inf = (~finite) & (frac == 0)
    assert np.isnan(out[nan]).all()
    assert np.isinf(out[inf]).all() and np.array_equal(np.signbit(out[inf]), (codes[inf] & 0x8000) != 0)
    # numpy's own binary16 agrees too (including -0 and subnormals)
    assert np.array_equal(out[finite].view(np.uint32),
                          B.f16_values(codes[finite]).astype(np.float32).view(np.uint32))


def test_f16_kats(oracle):
    for code, val in B.KATS["f16"]:
        assert oracle.lib().oracle_f16_to_f32(code) == np.float32(val)


# ---- known-answer blocks (reference tests) --------------------------------------

def test_q8_0_kats(oracle):
    k = B.KATS
    out = _dq(oracle, B.Q8_0, B.kat_block("q8_0_dequant"))
    exp = B.sparse_vector(32, k["q8_0_dequant"]["expected"])
    assert np.array_equal(out, exp)
    x = B.sparse_vector(32, k["q8_0_dot"]["x"])
    assert _dot(oracle, B.Q8_0, B.kat_block("q8_0_dot"), x) == k["q8_0_dot"]["expected"]


def test_q5_0_kats(oracle):
    k = B.KATS
    out = _dq(oracle, B.Q5_0, B.kat_block("q5_0"))
    exp = np.full(32, k["q5_0_dequant"]["default"], dtype=np.float32)
    for i, v in k["q5_0_dequant"]["expected"].items():
        exp[int(i)] = v
    assert np.array_equal(out, exp)
    x = B.sparse_vector(32, k["q5_0_dot"]["x"])
    assert _dot(oracle, B.Q5_0, B.kat_block("q5_0"), x) == k["q5_0_dot"]["expected"]


def test_q4_k_kats(oracle):
    k = B.KATS
    blk = np.frombuffer(B.kat_block("q4_k"), dtype=np.uint8).copy()
    sc, mn = ctypes.c_uint8(), ctypes.c_uint8()
    for s in range(8):
        assert oracle.lib().oracle_q4_k_unpack_scale_min(_p(blk) + 4, s, ctypes.byref(sc), ctypes.byref(mn)) == 1
        assert (sc.value, mn.value) == (k["q4_k_unpack"]["scales"][s], k["q4_k_unpack"]["mins"][s])
    assert oracle.lib().oracle_q4_k_unpack_scale_min(_p(blk) + 4, 8, ctypes.byref(sc), ctypes.byref(mn)) == 0
    assert oracle.lib().oracle_q4_k_unpack_scale_min(_p(blk) + 4, -1, ctypes.byref(sc), ctypes.byref(mn)) == 0
    out = _dq(oracle, B.Q4_K, blk)
    exp = np.repeat(np.array(k["q4_k_dequant"]["default_per_subblock"], dtype=np.float32), 32)
    for i, v in k["q4_k_dequant"]["expected"].items():
        exp[int(i)] = v
    assert np.array_equal(out, exp)
    x = B.sparse_vector(256, k["q4_k_dot"]["x"])
    assert _dot(oracle, B.Q4_K, blk, x) == k["q4_k_dot"]["expected"]


def test_q6_k_kats(oracle):
    k = B.KATS
    blk = np.frombuffer(B.kat_block("q6_k"), dtype=np.uint8).copy()
    q, sc = ctypes.c_int8(), ctypes.c_int8()
    for n, (idx, val) in enumerate(zip(k["q6_k_unpack"]["indices"], k["q6_k_unpack"]["values"])):
        assert oracle.lib().oracle_q6_k_unpack_value(_p(blk), idx, ctypes.byref(q), ctypes.byref(sc)) == 1
        assert (q.value, sc.value) == (val, n + 1)
    assert oracle.lib().oracle_q6_k_unpack_value(_p(blk), 256, ctypes.byref(q), ctypes.byref(sc)) == 0
    out = _dq(oracle, B.Q6_K, blk)
    exp = np.empty(256, dtype=np.float32)
    for n in range(256):
        g, l = divmod(n, 128)
        r, o = divmod(l, 32)
        exp[n] = 0.5 * (8 * g + 2 * r + o // 16 + 1) * k["q6_k_dequant"]["default_per_region"][r]
    for idx, val in zip(k["q6_k_dequant"]["selected"], k["q6_k_dequant"]["selected_values"]):
        g, l = divmod(idx, 128)
        r, o = divmod(l, 32)
        exp[idx] = 0.5 * (8 * g + 2 * r + o // 16 + 1) * val
    assert np.array_equal(out, exp)
    x = np.zeros(256, dtype=np.float32)
    x[k["q6_k_dot"]["x_ones_at"]] = 1.0
    assert _dot(oracle, B.Q6_K, blk, x) == k["q6_k_dot"]["expected"]


def test_block_null_arguments(oracle):
    lib = oracle.lib()
    buf = np.zeros(256, dtype=np.uint8)
    out = np.zeros(256, dtype=np.float32)
    for name in ("q8_0", "q5_0", "q4_k", "q6_k"):
        assert getattr(lib, f"oracle_{name}_dequantize_block")(None, _p(out)) == 0
        assert getattr(lib, f"oracle_{name}_dequantize_block")(_p(buf), None) == 0
        assert getattr(lib, f"oracle_{name}_dot_f32")(None, _p(out), _p(out)) == 0
        assert getattr(lib, f"oracle_{name}_dot_f32")(_p(buf), None, _p(out)) == 0
        assert getattr(lib, f"oracle_{name}_dot_f32")(_p(buf), _p(out), None) == 0


# ---- LCG dot-vs-dequant trials ------------------------------------------------------

@pytest.mark.parametrize("t", B.ALL_TYPES)
def test_lcg_dot_vs_dequant(oracle, t):
    """128-trial randomized blocks of the reference tests, same tolerances."""
    a, r = B.LCG_TOLERANCE[t]
    for blk, x in B.lcg_trials(t):
        w = _dq(oracle, t, blk)
        expected = np.float32(0.0)
        for i in range(len(x)):
            expected = np.float32(expected + np.float32(w[i] * x[i]))
        actual = _dot(oracle, t, blk, x)
        assert abs(actual - expected) <= a + r * abs(expected)


# ---- exact decoders of the documented equations --------------------------------------

@pytest.mark.parametrize("t", B.ALL_TYPES)
def test_dequant_matches_exact_decoder(oracle, t):
    n = 24 if t == B.Q4_K else 200
    raw = B.raw_blocks(t, n, seed=100 + t)
    lcg = np.concatenate([blk for blk, _ in B.lcg_trials(t, 16)])
    raw = np.concatenate([raw, lcg])
    nb = raw.size // B.BLOCK_BYTES[t]
    got = oracle.dequantize_rows(raw, t, nb, B.BLOCK_ELEMENTS[t], 0, nb)
    exp = B.decode_exact(raw, t)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def _mistaken_decoders():
    """Plausible slips in a decoder, planted in CPU-side copies of the oracle's
    equations; each must disagree with the exact decoder on random blocks,
    which shows that equality with it pins the oracle's index math."""
    def q4k(raw, swap_halves=False, shift_scale=False, plus_min=False):
        b = raw.reshape(-1, 144).astype(np.int64)
        d = B.f16_values(b[:, 0] | (b[:, 1] << 8))
        dm = B.f16_values(b[:, 2] | (b[:, 3] << 8))
        p = b[:, 4:16]
        out = np.empty((b.shape[0], 256))
        for s in range(8):
            ss = (s + 1) % 8 if shift_scale else s
            if ss < 4:
                sc, mn = p[:, ss] & 63, p[:, ss + 4] & 63
            else:
                sc = (p[:, ss + 4] & 15) | ((p[:, ss - 4] >> 6) << 4)
                mn = (p[:, ss + 4] >> 4) | ((p[:, ss] >> 6) << 4)
            half = (s % 2) ^ (1 if swap_halves else 0)
            q = (b[:, 16 + 32 * (s // 2): 48 + 32 * (s // 2)] >> (4 * half)) & 15
            out[:, 32 * s:32 * s + 32] = (d * sc)[:, None] * q + (1 if plus_min else -1) * (dm * mn)[:, None]
        return out.astype(np.float32)

    def q6k_no_half_offset(raw):
        b = raw.reshape(-1, 210).astype(np.int64)
        d = B.f16_values(b[:, 208] | (b[:, 209] << 8))
        sc = b[:, 192:208].astype(np.uint8).view(np.int8).astype(np.float64)
        idx = np.arange(256)
        g, l = idx // 128, idx % 128
        r, o = l // 32, l % 32
        low = (b[:, 64 * g + 32 * (r % 2) + o] >> (4 * (r // 2))) & 15
        high = (b[:, 128 + 32 * g + o] >> (2 * r)) & 3
        return (d[:, None] * sc[:, 8 * g + 2 * r] * ((low | (high << 4)) - 32)).astype(np.float32)

    def q50_bit_from_wrong_word(raw):
        b = raw.reshape(-1, 22).astype(np.int64)
        d = B.f16_values(b[:, 0] | (b[:, 1] << 8))
        qh = b[:, 2] | (b[:, 3] << 8) | (b[:, 4] << 16) | (b[:, 5] << 24)
        nib = np.concatenate([b[:, 6:22] & 15, b[:, 6:22] >> 4], axis=1)
        bits = (qh[:, None] >> (np.arange(32) % 16)[None, :]) & 1
        return (d[:, None] * (nib + 16 * bits - 16)).astype(np.float32)

    return [
        (B.Q4_K, lambda r: q4k(r, swap_halves=True)),
        (B.Q4_K, lambda r: q4k(r, shift_scale=True)),
        (B.Q4_K, lambda r: q4k(r, plus_min=True)),
        (B.Q6_K, q6k_no_half_offset),
        (B.Q5_0, q50_bit_from_wrong_word),
    ]


@pytest.mark.parametrize("case", range(5))
def test_exact_decoder_rejects_planted_mistakes(case):
    t, wrong = _mistaken_decoders()[case]
    raw = B.raw_blocks(t, 8, seed=900 + case)
    exact = B.decode_exact(raw, t)
    assert not np.array_equal(exact.view(np.uint32), wrong(raw).view(np.uint32))


# ---- matvec contract ------------------------------------------------------------------

def _fixture_matrix(t, rows, blocks_per_row, offset=1):
    """Multi-row matrix of constant blocks at an unaligned address
    (tests/quantized_matvec_reference_test.cpp:156-202)."""
    bb, be = B.BLOCK_BYTES[t], B.BLOCK_ELEMENTS[t]
    storage = np.zeros(offset + rows * blocks_per_row * bb, dtype=np.uint8)
    vals = np.zeros((rows, blocks_per_row), dtype=np.float32)
    for r in range(rows):
        for b in range(blocks_per_row):
            idx = r * blocks_per_row + b
            blk, v = B.fixture_block(t, idx)
            storage[offset + idx * bb: offset + (idx + 1) * bb] = np.frombuffer(blk, dtype=np.uint8)
            vals[r, b] = v
    return storage, vals


@pytest.mark.parametrize("t", B.ALL_TYPES)
def test_multirow_unaligned_matvec(oracle, t):
    rows, bpr = 17, 3
    be = B.BLOCK_ELEMENTS[t]
    cols = bpr * be
    storage, vals = _fixture_matrix(t, rows, bpr)
    x = ((np.arange(cols) % 13 - 6) / 8.0).astype(np.float32)
    expected = np.zeros(rows, dtype=np.float32)
    for r in range(rows):
        for b in range(bpr):
            for c in range(be):
                expected[r] = np.float32(expected[r] + np.float32(vals[r, b] * x[b * be + c]))
    y = oracle.matvec(storage, t, rows, cols, x, offset=1)
    assert np.all(np.abs(y - expected) <= 1e-5)


def test_matvec_kats(oracle):
    k = B.KATS["matvec_q8_0_two_rows"]
    raw = np.frombuffer(b"".join(B.q8_0_block(bk["d"], bk["qs"]) for bk in k["blocks"]), dtype=np.uint8).copy()
    x = B.sparse_vector(32, k["x"])
    assert list(oracle.matvec(raw, B.Q8_0, 2, 32, x)) == k["expected"]
    one = B.sparse_vector(256, {"0": 1.0})
    raw = np.frombuffer(B.q5_0_block(0x3800, {}, {}), dtype=np.uint8).copy()
    assert oracle.matvec(raw, B.Q5_0, 1, 32, one[:32])[0] == B.KATS["matvec_q5_0_single"]["expected"]
    raw = np.frombuffer(B.q4_k_block(0x3800, 0x3400, [1, 0, 0, 0, 1] + [0] * 7, {}), dtype=np.uint8).copy()
    assert oracle.matvec(raw, B.Q4_K, 1, 256, one)[0] == B.KATS["matvec_q4_k_single"]["expected"]
    raw = np.frombuffer(B.q6_k_block(0x3800, [1] + [0] * 15, 0, {}), dtype=np.uint8).copy()
    assert oracle.matvec(raw, B.Q6_K, 1, 256, one)[0] == B.KATS["matvec_q6_k_single"]["expected"]


def test_matmul_equals_repeated_matvec(oracle):
    rng = np.random.default_rng(7)
    for t in B.ALL_TYPES:
        rows, cols = 9, 2 * B.BLOCK_ELEMENTS[t]
        raw = B.raw_blocks(t, rows * 2, seed=t)
        x = rng.standard_normal((5, cols)).astype(np.float32)
        ym = oracle.matvec(raw, t, rows, cols, x)
        for b in range(5):
            assert np.array_equal(ym[b], oracle.matvec(raw, t, rows, cols, x[b]))


def test_invalid_arguments(oracle):
    """tests/quantized_matvec_reference_test.cpp:223-259 plus the layout rules."""
    lib = oracle.lib()
    raw = np.zeros(34, dtype=np.uint8)
    x = np.zeros(32, dtype=np.float32)
    y = np.zeros(2, dtype=np.float32)
    v = oracle.view(raw, B.Q8_0, 1, 32)
    vp = ctypes.byref(v)
    assert lib.oracle_matvec_f32(None, _p(x), 32, _p(y), 1) == 0
    assert lib.oracle_matvec_f32(vp, None, 32, _p(y), 1) == 0
    assert lib.oracle_matvec_f32(vp, _p(x), 32, None, 1) == 0
    assert lib.oracle_matvec_f32(vp, _p(x), 31, _p(y), 1) == 0
    assert lib.oracle_matvec_f32(vp, _p(x), 32, _p(y), 2) == 0
    assert lib.oracle_matmul_f32(vp, _p(x), 32, 0, _p(y), 1) == 0
    for field, value in (("dimension_count", 1), ("ggml_type", 99), ("block_count", 0),
                         ("block_elements", 33), ("block_bytes", 35), ("element_count", 31)):
        w = oracle.view(raw, B.Q8_0, 1, 32)
        setattr(w, field, value)
        assert lib.oracle_matvec_f32(ctypes.byref(w), _p(x), 32, _p(y), 1) == 0
    assert lib.oracle_matvec_f32(vp, _p(x), 32, _p(y), 1) == 1


def test_q4_k_4864x896_is_rejected(oracle):
    """Q4_K 4864 x 896: 896 is not a multiple of 256 (src/quantized_matvec.cpp:136-138)."""
    raw = np.zeros(1, dtype=np.uint8)
    v = oracle.view(raw, B.Q4_K, 4864, 896)
    v.block_count = 4864 * 896 // 256
    x = np.zeros(896, dtype=np.float32)
    y = np.zeros(4864, dtype=np.float32)
    assert oracle.lib().oracle_matvec_f32(ctypes.byref(v), _p(x), 896, _p(y), 4864) == 0


def test_greedy_argmax(oracle):
    assert oracle.greedy_argmax(np.array([1, 3, 3, 2], dtype=np.float32)) == (1, 1)
    assert oracle.greedy_argmax(np.array([-5], dtype=np.float32)) == (1, 0)
    assert oracle.greedy_argmax(np.array([1, np.nan, 3], dtype=np.float32)) == (0, -1)
    assert oracle.greedy_argmax(np.array([1, np.inf], dtype=np.float32)) == (0, -1)
    x = np.random.default_rng(3).standard_normal(100000).astype(np.float32)
    assert oracle.greedy_argmax(x) == (1, int(np.argmax(x)))


# ---- the reference itself, compiled from its sources ---------------------------------------

def _ref_or_skip(oracle, kind):
    lib = oracle.ref_lib(kind)
    if lib is None:
        pytest.skip("oracle/_ref not built (the reference checkout is absent on this host)")
    return lib


@pytest.mark.parametrize("t", B.ALL_TYPES)
def test_oracle_bit_identical_to_reference_scalar_build(oracle, t):
    """Dequant and block dots bit-for-bit equal to the reference's scalar
    branches; matvec/matmul bit-for-bit equal to its row loop."""
    ref = _ref_or_skip(oracle, "scalar")
    name = {B.Q8_0: "q8_0", B.Q5_0: "q5_0", B.Q4_K: "q4_k", B.Q6_K: "q6_k"}[t]
    be = B.BLOCK_ELEMENTS[t]
    raw = B.raw_blocks(t, 64, seed=200 + t)
    rng = np.random.default_rng(t)
    for i in range(64):
        blk = raw[i * B.BLOCK_BYTES[t]:(i + 1) * B.BLOCK_BYTES[t]].copy()
        ours = _dq(oracle, t, blk)
        theirs = np.empty(be, dtype=np.float32)
        assert getattr(ref, f"ref_{name}_dequantize_block")(_p(blk), _p(theirs)) == 1
        assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))
        x = rng.standard_normal(be).astype(np.float32)
        r = np.zeros(1, dtype=np.float32)
        assert getattr(ref, f"ref_{name}_dot_f32")(_p(blk), _p(x), _p(r)) == 1
        assert np.float32(_dot(oracle, t, blk, x)).view(np.uint32) == r.view(np.uint32)[0]
    rows, cols = 13, 4 * be
    raw = B.raw_blocks(t, rows * 4, seed=300 + t)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    v = oracle.view(raw, t, rows, cols)
    for m in (1, 3):
        theirs = np.empty((m, rows), dtype=np.float32)
        if m == 1:
            assert ref.ref_quantized_tensor_matvec_f32(ctypes.byref(v), _p(x), cols, _p(theirs), rows) == 1
        else:
            assert ref.ref_quantized_tensor_matmul_f32(ctypes.byref(v), _p(x), cols, m, _p(theirs), rows) == 1
        ours = oracle.matvec(raw, t, rows, cols, x[0] if m == 1 else x[:m])
        assert np.array_equal(ours.reshape(m, rows).view(np.uint32), theirs.view(np.uint32))


def test_f16_bit_identical_to_reference(oracle):
    ref = _ref_or_skip(oracle, "scalar")
    r = ctypes.c_float()
    for code in range(65536):
        assert ref.ref_f16_bits_to_f32(code, ctypes.byref(r)) == 1
        ours = np.float32(oracle.lib().oracle_f16_to_f32(code))
        theirs = np.float32(r.value)
        if math.isnan(theirs):
            assert math.isnan(ours)
        else:
            assert ours.view(np.uint32) == theirs.view(np.uint32)


@pytest.mark.parametrize("t", B.ALL_TYPES)
def test_reference_avx2_build_within_tolerance(oracle, t):
    """The reference's as-deployed x86 build (AVX2/FMA) reduces in another
    order; it agrees with the scalar oracle under the row rule."""
    ref = _ref_or_skip(oracle, "avx2")
    be = B.BLOCK_ELEMENTS[t]
    rows, cols = 31, 8 * be
    raw = B.raw_blocks(t, rows * 8, seed=400 + t)
    x = np.random.default_rng(t).standard_normal(cols).astype(np.float32)
    v = oracle.view(raw, t, rows, cols)
    theirs = np.empty(rows, dtype=np.float32)
    assert ref.ref_quantized_tensor_matvec_f32(ctypes.byref(v), _p(x), cols, _p(theirs), rows) == 1
    ours = oracle.matvec(raw, t, rows, cols, x)
    _, absdot = oracle.row_stats(raw, t, rows, cols, x)
    ok = np.isfinite(absdot)
    assert np.all(np.abs(ours[ok] - theirs[ok]) <= 1e-5 * absdot[ok])


# ---- row-range helpers used by the GPU parity tests -----------------------------

@pytest.mark.parametrize("t", B.ALL_TYPES)
def test_row_helpers_against_independent_forms(oracle, t):
    """oracle_dequantize_rows is the per-block decoder (pinned above) laid out
    row by row; oracle_matvec_rows_f32 is a slice of the full matvec bit for
    bit; oracle_row_stats_f64 equals a float64 numpy dot over the decoded rows
    (sum of w*x and of |w*x|), so the tolerance denominator is pinned too."""
    be, bpr, rows = B.BLOCK_ELEMENTS[t], 6, 23
    cols = bpr * be
    raw = B.raw_blocks(t, rows * bpr, seed=900 + t)
    bb = B.BLOCK_BYTES[t]
    blocks = [raw[i * bb:(i + 1) * bb] for i in range(rows * bpr)]
    w = np.stack([np.concatenate([_dq(oracle, t, blocks[r * bpr + b]) for b in range(bpr)]) for r in range(rows)])
    got = oracle.dequantize_rows(raw, t, rows, cols, 5, 11)
    nan = np.isnan(w[5:16])
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), w[5:16][~nan].view(np.uint32))

    x = np.random.default_rng(t).standard_normal(cols).astype(np.float32)
    full = oracle.matvec(raw, t, rows, cols, x)
    part = oracle.matvec_rows(raw, t, rows, cols, x, 7, 9)
    assert np.array_equal(part.view(np.uint32), full[7:16].view(np.uint32))

    dot, absdot = oracle.row_stats(raw, t, rows, cols, x, 3, 17)
    prod = w[3:20].astype(np.float64) * x.astype(np.float64)
    fin = np.isfinite(prod).all(axis=1)
    assert np.allclose(dot[fin], prod[fin].sum(axis=1), rtol=1e-12, atol=1e-300)
    assert np.allclose(absdot[fin], np.abs(prod[fin]).sum(axis=1), rtol=1e-12, atol=1e-300)


# ---- decode-step element operations ----------------------------------------------------

U32 = 2.0 ** -24  # unit roundoff of binary32


def _rms_norm_f64(x, w, eps):
    x64 = x.astype(np.float64)
    return x64 / np.sqrt(np.mean(x64 * x64) + float(np.float32(eps))) * w.astype(np.float64)


def _swiglu_f64(g, u):
    g64 = g.astype(np.float64)
    return u.astype(np.float64) * (g64 / (1.0 + np.exp(-g64)))


# Relative error allowed against the float64 closed form. RMSNorm: the fp32
# sum of squares in index order is off by about sqrt(n) * u relative
# (3.6e-6 at n = 3584; a worst case of n * u / 2 = 1.1e-4 needs adversarial
# data), halved by the square root, plus three roundings; 2e-5 leaves a 5x
# margin and still rejects the plausible mistakes below (a dropped epsilon,
# n - 1 for n, a missing square root, a shifted weight index).
RMS_REL = 2e-5
SWIGLU_ULPS = 4


def _rms_inputs(n, scale, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    return x, w


def _rms_close(y, x, w, eps):
    ref = _rms_norm_f64(x, w, eps)
    return bool(np.all(np.abs(y.astype(np.float64) - ref) <= RMS_REL * np.abs(ref) + 1e-30))


def test_element_op_kats(oracle):
    """tests/tensor_reference_test.cpp:50-58, 84-93 and
    tests/transformer_ops_reference_test.cpp:95-103, at the reference's 1e-5."""
    ok, y = oracle.add([0.75, 0.85, 1.0], [0.0, -3.5, 5.0])
    assert ok == 1 and np.all(np.abs(y - np.array([0.75, -2.65, 6.0], np.float32)) <= 1e-5)
    ok, y = oracle.rms_norm([1.0, 1.0], [2.0, 3.0], 3.0)
    assert ok == 1 and y.tolist() == [1.0, 1.5]  # exact: sqrt(1 + 3) = 2
    ok, y = oracle.swiglu([0.0, 1.0, -1.0], [4.0, 2.0, 5.0])
    assert ok == 1 and np.all(np.abs(y - np.array([0.0, 1.462117, -1.344707], np.float32)) <= 1e-5)


def test_element_op_invalid_arguments(oracle):
    """src/tensor.cpp:11-17, 116-122 and src/transformer_ops.cpp:169-172; the
    reference's own table is tests/tensor_reference_test.cpp:145-156."""
    lib = oracle.lib()
    v = np.ones(3, dtype=np.float32)
    o = np.zeros(3, dtype=np.float32)
    assert lib.oracle_add_f32(None, _p(v), 3, _p(o)) == 0
    assert lib.oracle_add_f32(_p(v), _p(v), 0, _p(o)) == 0
    assert lib.oracle_rms_norm_f32(None, _p(v), 3, 1e-5, _p(o)) == 0
    assert lib.oracle_rms_norm_f32(_p(v), None, 3, 1e-5, _p(o)) == 0
    assert lib.oracle_rms_norm_f32(_p(v), _p(v), 3, 0.0, _p(o)) == 0
    assert lib.oracle_rms_norm_f32(_p(v), _p(v), 3, -1.0, _p(o)) == 0
    assert lib.oracle_rms_norm_f32(_p(v), _p(v), -3, 1e-5, _p(o)) == 0
    assert lib.oracle_swiglu_f32(None, _p(v), 3, _p(o)) == 0
    assert lib.oracle_swiglu_f32(_p(v), _p(v), 0, _p(o)) == 0
    # epsilon <= 0 is the only epsilon check: NaN passes it, as in the reference.
    assert lib.oracle_rms_norm_f32(_p(v), _p(v), 3, float("nan"), _p(o)) == 1


def test_add_is_fp32_add(oracle):
    rng = np.random.default_rng(11)
    a = rng.standard_normal(5000).astype(np.float32)
    b = (rng.standard_normal(5000) * 1e3).astype(np.float32)
    ok, y = oracle.add(a, b)
    assert ok == 1 and np.array_equal(y.view(np.uint32), (a + b).view(np.uint32))


@pytest.mark.parametrize("n,scale", [(3584, 1.0), (3584, 1e-3), (896, 30.0), (1536, 1e-4), (7, 1.0)])
def test_rms_norm_against_float64(oracle, n, scale):
    """The 1e-3 and 1e-4 scales put the mean square at or below epsilon, so a
    dropped or misplaced epsilon fails."""
    x, w = _rms_inputs(n, scale, n)
    ok, y = oracle.rms_norm(x, w, 1e-6)
    assert ok == 1 and _rms_close(y, x, w, 1e-6)


def test_rms_norm_constant_input(oracle):
    """x = c everywhere: y = c / sqrt(c^2 + eps) * w exactly up to three roundings."""
    x = np.full(1000, 0.5, np.float32)
    w = np.full(1000, 3.0, np.float32)
    ok, y = oracle.rms_norm(x, w, 0.75)  # mean 0.25 + 0.75 = 1: y = 0.5 * 3 exactly
    assert ok == 1 and np.all(y == 1.5)


def _rms_mistakes():
    def no_eps(x, w, eps):
        x64 = x.astype(np.float64)
        return (x64 / np.sqrt(np.mean(x64 * x64)) * w).astype(np.float32)

    def n_minus_one(x, w, eps):
        x64 = x.astype(np.float64)
        return (x64 / np.sqrt(np.sum(x64 * x64) / (x.size - 1) + eps) * w).astype(np.float32)

    def no_sqrt(x, w, eps):
        x64 = x.astype(np.float64)
        return (x64 / (np.mean(x64 * x64) + eps) * w).astype(np.float32)

    def shifted_weight(x, w, eps):
        return _rms_norm_f64(x, np.roll(w, 1), eps).astype(np.float32)

    return [no_eps, n_minus_one, no_sqrt, shifted_weight]


@pytest.mark.parametrize("case", range(4))
def test_rms_norm_check_rejects_planted_mistakes(case):
    """Each plausible RMSNorm mistake fails the float64 check on at least one
    of the inputs test_rms_norm_against_float64 uses."""
    wrong = _rms_mistakes()[case]
    caught = False
    for n, scale in [(3584, 1.0), (3584, 1e-3), (896, 30.0), (1536, 1e-4)]:
        x, w = _rms_inputs(n, scale, n)
        caught |= not _rms_close(wrong(x, w, 1e-6), x, w, 1e-6)
    assert caught


def test_swiglu_against_float64(oracle):
    rng = np.random.default_rng(5)
    g = np.concatenate([rng.standard_normal(20000) * 4, [0.0, -0.0, 90.0, -90.0, 1e-30, -1e-30]]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    ok, y = oracle.swiglu(g, u)
    ref = _swiglu_f64(g, u)
    assert ok == 1
    # The absolute floor covers gates near -90, where exp(-g) overflows fp32
    # and silu is -0 instead of about -1e-37.
    assert np.all(np.abs(y - ref) <= SWIGLU_ULPS * U32 * 2 * np.abs(ref) + 1e-30)
    # Large negative gates: exp overflows to inf and silu is -0 times up.
    ok, y = oracle.swiglu(np.array([-200.0], np.float32), np.array([2.0], np.float32))
    assert ok == 1 and y[0] == 0.0


def test_element_ops_bit_identical_to_reference_scalar_build(oracle):
    ref = _ref_or_skip(oracle, "scalar")
    rng = np.random.default_rng(21)
    for n, scale in [(3584, 1.0), (3584, 1e-3), (18944, 2.0), (5, 1.0)]:
        x, w = _rms_inputs(n, scale, n + 1)
        y_ref = np.empty_like(x)
        assert ref.ref_tensor_rms_norm_f32(_p(x), _p(w), n, 1e-6, _p(y_ref)) == 1
        ok, y = oracle.rms_norm(x, w, 1e-6)
        assert ok == 1 and np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
        g = (rng.standard_normal(n) * 3).astype(np.float32)
        u = rng.standard_normal(n).astype(np.float32)
        gate = g.copy()
        assert ref.ref_transformer_swiglu_f32(_p(gate), _p(u), n) == 1
        ok, y = oracle.swiglu(g, u)
        assert ok == 1 and np.array_equal(y.view(np.uint32), gate.view(np.uint32))
        s_ref = np.empty_like(x)
        assert ref.ref_tensor_add_f32(_p(x), _p(w), n, _p(s_ref)) == 1
        assert np.array_equal(oracle.add(x, w)[1].view(np.uint32), s_ref.view(np.uint32))


def test_reference_avx2_element_ops_within_tolerance(oracle):
    """The as-deployed build contracts the sum of squares into FMAs, so its
    RMSNorm differs in the last bits; it meets the same float64 bound."""
    ref = _ref_or_skip(oracle, "avx2")
    for n, scale in [(3584, 1.0), (3584, 1e-3), (896, 30.0)]:
        x, w = _rms_inputs(n, scale, n)
        y = np.empty_like(x)
        assert ref.ref_tensor_rms_norm_f32(_p(x), _p(w), n, 1e-6, _p(y)) == 1
        assert _rms_close(y, x, w, 1e-6)
