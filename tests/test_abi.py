"""CPU-only checks of the C-ABI library and the host-side logic: the library
loads, exports every entry point its headers declare (C ABI and the C++
drop-in symbols), and rejects invalid arguments before touching a GPU
(validation of src/quantized_matvec.cpp:93-149 and :168-191)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import _blocks as B

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_c_functions(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qmv_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_are_exported(qmv):
    lib = qmv.hip_lib()
    names = _declared_c_functions("qmv_hip.h")
    assert len(names) >= 18
    for name in names:
        assert hasattr(lib, name), name
        assert name in qmv.HIP_SIGNATURES, f"{name} missing from the Python mirror"


def test_cxx_drop_in_symbols_are_exported(qmv):
    """The reference's C++ entry points keep their mangled names
    (src/quantized_matvec.h:32-50 has no extern "C")."""
    out = subprocess.run(["nm", "-D", "--defined-only", qmv.HIP_LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    assert "_Z27quantized_tensor_matvec_f32PK23GgufQuantizedTensorViewPKfiPfi" in out
    assert "_Z27quantized_tensor_matmul_f32PK23GgufQuantizedTensorViewPKfiiPfi" in out
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    allowed = set(_declared_c_functions("qmv_hip.h")) | {
        "_Z27quantized_tensor_matvec_f32PK23GgufQuantizedTensorViewPKfiPfi",
        "_Z27quantized_tensor_matmul_f32PK23GgufQuantizedTensorViewPKfiiPfi"}
    assert exported <= allowed, sorted(exported - allowed)


def test_view_layout_matches_reference_struct(qmv):
    """QmvTensorView has GgufQuantizedTensorView's layout (src/gguf_reader.h:31-40)."""
    V = qmv.QmvTensorView
    assert ctypes.sizeof(V) == 8 + 4 + 4 + 32 + 8 * 4
    assert V.dimensions.offset == 16 and V.block_count.offset == 72


def _valid(qmv):
    raw = np.zeros(34, dtype=np.uint8)
    return raw, qmv.make_view(raw, B.Q8_0, 1, 32)


def test_invalid_arguments_fail_without_gpu(qmv):
    """Table of tests/quantized_matvec_reference_test.cpp:223-259 and the
    layout rules; all rejected in host code, so no device is needed."""
    lib = qmv.hip_lib()
    raw, v = _valid(qmv)
    x = np.zeros(64, dtype=np.float32)
    y = np.zeros(4, dtype=np.float32)
    vp = ctypes.byref(v)
    xp, yp = x.ctypes.data, y.ctypes.data
    assert lib.qmv_tensor_matvec_f32(None, xp, 32, yp, 1) == 0
    assert lib.qmv_tensor_matvec_f32(vp, None, 32, yp, 1) == 0
    assert lib.qmv_tensor_matvec_f32(vp, xp, 32, None, 1) == 0
    assert lib.qmv_tensor_matvec_f32(vp, xp, 31, yp, 1) == 0
    assert lib.qmv_tensor_matvec_f32(vp, xp, 32, yp, 2) == 0
    assert lib.qmv_tensor_matvec_f32(vp, xp, 0, yp, 1) == 0
    assert lib.qmv_tensor_matmul_f32(vp, xp, 32, 0, yp, 1) == 0
    assert lib.qmv_tensor_matmul_f32(vp, xp, 32, -3, yp, 1) == 0
    cases = [("dimension_count", 1), ("ggml_type", 99), ("ggml_type", 0), ("block_count", 0),
             ("block_elements", 33), ("block_bytes", 35), ("element_count", 31)]
    for field, value in cases:
        _, w = _valid(qmv)
        setattr(w, field, value)
        assert lib.qmv_tensor_matvec_f32(ctypes.byref(w), xp, 32, yp, 1) == 0, field
        assert qmv.last_error() != ""
    _, w = _valid(qmv)
    w.dimensions[1] = 2 ** 40
    assert lib.qmv_tensor_matvec_f32(ctypes.byref(w), xp, 32, yp, 1) == 0
    _, w = _valid(qmv)
    w.data = None
    assert lib.qmv_tensor_matvec_f32(ctypes.byref(w), xp, 32, yp, 1) == 0
    # the C++ drop-in rejects a null view too
    assert y[0] == 0.0


def test_q4_k_4864x896_rejected_without_gpu(qmv):
    """Q4_K 4864 x 896 (K not a multiple of 256) must return 0 like the reference."""
    raw = np.zeros(16, dtype=np.uint8)
    v = qmv.make_view(raw, B.Q4_K, 4864, 896)
    x = np.zeros(896, dtype=np.float32)
    y = np.full(4864, -99.0, dtype=np.float32)
    assert qmv.quantized_tensor_matvec_f32(v, x, 896, y, 4864) == 0
    assert (y == -99.0).all()


def test_invalid_sampler_and_device_args_fail_without_gpu(qmv):
    lib = qmv.hip_lib()
    tok = ctypes.c_int(5)
    assert lib.qmv_greedy_sample_f32(None, 10, ctypes.byref(tok)) == 0 and tok.value == -1
    x = np.zeros(3, dtype=np.float32)
    tok = ctypes.c_int(5)
    assert lib.qmv_greedy_sample_f32(x.ctypes.data, 0, ctypes.byref(tok)) == 0 and tok.value == -1
    assert lib.qmv_device_matvec_f32(None, None, 1, None, None) == 0
    assert lib.qmv_device_greedy_argmax_f32(None, 10, None, None) == 0
    assert lib.qmv_device_matvec_argmax_f32(None, None, None, None, None) == 0
    assert lib.qmv_device_embed_rows_f32(None, None, 1, None, None, None) == 0
    assert lib.qmv_device_matvec_add_group_f32(None, 1, None, 1, None, None, None, None) == 0
    assert lib.qmv_device_matvec_swiglu_f32(None, None, None, 1, None, None) == 0
    assert lib.qmv_device_tensor_create(None, None) == 0
    assert lib.qmv_dequantize_rows_f32(None, 0, 1, x.ctypes.data) == 0


def test_rms_norm_argument_table_without_gpu(qmv):
    """src/tensor.cpp:116-122 (null pointers, length <= 0, epsilon <= 0), plus
    batch_count <= 0 and the overlap rule; all rejected before any HIP call
    (the addresses are compared, never dereferenced)."""
    lib = qmv.hip_lib()
    buf = np.zeros(64, dtype=np.float32)
    a = buf.ctypes.data
    x, w, y = a, a + 4 * 16, a + 4 * 32
    assert lib.qmv_device_rms_norm_f32(None, w, 8, 1, 1e-6, y, None) == 0
    assert lib.qmv_device_rms_norm_f32(x, None, 8, 1, 1e-6, y, None) == 0
    assert lib.qmv_device_rms_norm_f32(x, w, 8, 1, 1e-6, None, None) == 0
    assert lib.qmv_device_rms_norm_f32(x, w, 0, 1, 1e-6, y, None) == 0
    assert lib.qmv_device_rms_norm_f32(x, w, 8, 0, 1e-6, y, None) == 0
    assert lib.qmv_device_rms_norm_f32(x, w, 8, 1, 0.0, y, None) == 0
    assert lib.qmv_device_rms_norm_f32(x, w, 8, 1, -1.0, y, None) == 0
    assert lib.qmv_device_rms_norm_f32(x, w, 8, 1, 1e-6, x + 4, None) == 0  # part of the input
    assert lib.qmv_device_rms_norm_f32(x, w, 8, 1, 1e-6, w + 4, None) == 0  # the weight
    assert "RMSNorm" in qmv.last_error()
    assert (buf == 0).all()


def test_cxx_dropin_argument_table_without_gpu(qmv):
    """The reference's C++ entry points, called from a C++ program built
    against include/quantized_matvec.h, reject the invalid-argument table
    before any device work (tests/cxx/dropin_test.cpp)."""
    exe = os.path.join(ROOT, "tests", "cxx", "dropin_test")
    assert os.path.exists(exe), "tests/cxx/dropin_test missing: run __graft_entry__.build()"
    r = subprocess.run([exe, "--args"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr


def test_synth_is_deterministic_and_distributed(qmv):
    a = qmv.synth_tensor(B.Q4_K, 64, 512, seed=5)
    b = qmv.synth_tensor(B.Q4_K, 64, 512, seed=5)
    c = qmv.synth_tensor(B.Q4_K, 64, 512, seed=6)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    blocks = a.reshape(-1, 144)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    assert (d >= 0).all() and 0.004 < d.mean() < 0.012  # |N(0, 0.01)| has mean 0.008
    q6 = qmv.synth_tensor(B.Q6_K, 32, 4864, seed=2).reshape(-1, 210)
    sc = q6[:, 192:208].view(np.int8)
    assert sc.min() >= -64 and sc.max() <= 63
    q8 = qmv.synth_tensor(B.Q8_0, 8, 896, seed=0).reshape(-1, 34)
    qs = q8[:, 2:].view(np.int8)
    assert qs.min() >= -127
    x = qmv.synth_normal(200000, seed=1)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01


def test_synth_f16_rounding_matches_numpy(qmv):
    rng = np.random.default_rng(0)
    vals = np.concatenate([np.abs(rng.standard_normal(20000)) * s for s in (1e-3, 1e-2, 1.0, 1e3)] +
                          [np.array([0.0, 5.96e-8, 2.98e-8, 6.1e-5, 65504.0, 65519.0, 65520.0])])
    ours = np.array([qmv.synth_lib().qmv_synth_f64_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(ours, vals.astype(np.float16).view(np.uint16))
