"""ORACLE — test infrastructure only.

ctypes access to the CPU oracle for the MI355X packed matvec path:
  * ``liboracle.so``: the plain-C restatement of the reference's scalar path
    (qmv_oracle.c; header qmv_oracle.h lists what pins each function);
  * ``_ref/libref_scalar.so`` / ``_ref/libref_avx2.so``: the reference's own
    src/quantization.cpp + src/quantized_matvec.cpp (and the decode-step
    element operations of src/tensor.cpp, src/transformer_ops.cpp) compiled
    from source by
    ``oracle/Makefile`` (present wherever they were built; they travel with the
    repository tree but are never committed).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this package, and only to check results or time the CPU baseline.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liboracle.so")
REF_SCALAR_LIB = os.path.join(HERE, "_ref", "libref_scalar.so")
REF_AVX2_LIB = os.path.join(HERE, "_ref", "libref_avx2.so")
REFERENCE_TREE = "/root/reference"

_vp = ctypes.c_void_p
_i = ctypes.c_int


class OracleView(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("ggml_type", ctypes.c_uint32),
        ("dimension_count", ctypes.c_uint32),
        ("dimensions", ctypes.c_uint64 * 4),
        ("element_count", ctypes.c_uint64),
        ("block_elements", ctypes.c_uint64),
        ("block_bytes", ctypes.c_uint64),
        ("block_count", ctypes.c_uint64),
    ]


_ORACLE_SIGS = {
    "oracle_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "oracle_q4_k_unpack_scale_min": (_i, [_vp, _i, _vp, _vp]),
    "oracle_q6_k_unpack_value": (_i, [_vp, _i, _vp, _vp]),
    "oracle_q8_0_dequantize_block": (_i, [_vp, _vp]),
    "oracle_q5_0_dequantize_block": (_i, [_vp, _vp]),
    "oracle_q4_k_dequantize_block": (_i, [_vp, _vp]),
    "oracle_q6_k_dequantize_block": (_i, [_vp, _vp]),
    "oracle_q8_0_dot_f32": (_i, [_vp, _vp, _vp]),
    "oracle_q5_0_dot_f32": (_i, [_vp, _vp, _vp]),
    "oracle_q4_k_dot_f32": (_i, [_vp, _vp, _vp]),
    "oracle_q6_k_dot_f32": (_i, [_vp, _vp, _vp]),
    "oracle_matvec_f32": (_i, [_vp, _vp, _i, _vp, _i]),
    "oracle_matmul_f32": (_i, [_vp, _vp, _i, _i, _vp, _i]),
    "oracle_matvec_rows_f32": (_i, [_vp, _vp, _i, _i, _vp]),
    "oracle_dequantize_rows": (_i, [_vp, _i, _i, _vp]),
    "oracle_row_stats_f64": (_i, [_vp, _vp, _i, _i, _vp, _vp]),
    "oracle_greedy_argmax": (_i, [_vp, _i, _vp]),
    "oracle_add_f32": (_i, [_vp, _vp, _i, _vp]),
    "oracle_rms_norm_f32": (_i, [_vp, _vp, _i, ctypes.c_float, _vp]),
    "oracle_swiglu_f32": (_i, [_vp, _vp, _i, _vp]),
}

_REF_SIGS = {
    "ref_f16_bits_to_f32": (_i, [ctypes.c_uint16, _vp]),
    "ref_q8_0_dequantize_block": (_i, [_vp, _vp]),
    "ref_q5_0_dequantize_block": (_i, [_vp, _vp]),
    "ref_q4_k_dequantize_block": (_i, [_vp, _vp]),
    "ref_q6_k_dequantize_block": (_i, [_vp, _vp]),
    "ref_q8_0_dot_f32": (_i, [_vp, _vp, _vp]),
    "ref_q5_0_dot_f32": (_i, [_vp, _vp, _vp]),
    "ref_q4_k_dot_f32": (_i, [_vp, _vp, _vp]),
    "ref_q6_k_dot_f32": (_i, [_vp, _vp, _vp]),
    "ref_q4_k_unpack_scale_min": (_i, [_vp, _i, _vp, _vp]),
    "ref_q6_k_unpack_value": (_i, [_vp, _i, _vp, _vp]),
    "ref_quantized_tensor_matvec_f32": (_i, [_vp, _vp, _i, _vp, _i]),
    "ref_quantized_tensor_matmul_f32": (_i, [_vp, _vp, _i, _i, _vp, _i]),
    "ref_tensor_add_f32": (_i, [_vp, _vp, _i, _vp]),
    "ref_tensor_rms_norm_f32": (_i, [_vp, _vp, _i, ctypes.c_float, _vp]),
    "ref_transformer_swiglu_f32": (_i, [_vp, _vp, _i]),
}

_cache = {}


def _load(path, sigs):
    if path not in _cache:
        lib = ctypes.CDLL(path)
        for name, (res, args) in sigs.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _cache[path] = lib
    return _cache[path]


def build_oracle() -> None:
    subprocess.run(["make", "-B", "-C", HERE, "liboracle.so"], check=True)


def build_reference() -> bool:
    """Compile the reference's path from its checkout into _ref/ (only where the
    checkout exists, i.e. not on the GPU host). Returns True if built."""
    if not os.path.isdir(os.path.join(REFERENCE_TREE, "src")):
        return False
    subprocess.run(["make", "-B", "-C", HERE, "ref", f"REF={REFERENCE_TREE}"], check=True)
    return True


def lib():
    if not os.path.exists(ORACLE_LIB):
        raise RuntimeError("oracle/liboracle.so missing: run __graft_entry__.build()")
    return _load(ORACLE_LIB, _ORACLE_SIGS)


def ref_lib(kind: str = "scalar"):
    """The reference's own compiled path, or None where it was not built."""
    path = REF_SCALAR_LIB if kind == "scalar" else REF_AVX2_LIB
    if not os.path.exists(path):
        return None
    return _load(path, _REF_SIGS)


def view(buf: np.ndarray, ggml_type: int, rows: int, cols: int, offset: int = 0) -> OracleView:
    be = {6: 32, 8: 32, 12: 256, 14: 256}[ggml_type]
    bb = {6: 22, 8: 34, 12: 144, 14: 210}[ggml_type]
    v = OracleView()
    v.data = buf.ctypes.data + offset
    v.ggml_type = ggml_type
    v.dimension_count = 2
    v.dimensions[0] = cols
    v.dimensions[1] = rows
    v.element_count = rows * cols
    v.block_elements = be
    v.block_bytes = bb
    v.block_count = rows * cols // be
    return v


def _p(a):
    return a.ctypes.data


def matvec(buf, ggml_type, rows, cols, x, offset=0):
    v = view(buf, ggml_type, rows, cols, offset)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        y = np.empty(rows, dtype=np.float32)
        assert lib().oracle_matvec_f32(ctypes.byref(v), _p(x), cols, _p(y), rows) == 1
    else:
        y = np.empty((x.shape[0], rows), dtype=np.float32)
        assert lib().oracle_matmul_f32(ctypes.byref(v), _p(x), cols, x.shape[0], _p(y), rows) == 1
    return y


def matvec_rows(buf, ggml_type, rows, cols, x, first_row, row_count):
    v = view(buf, ggml_type, rows, cols)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(row_count, dtype=np.float32)
    assert lib().oracle_matvec_rows_f32(ctypes.byref(v), _p(x), first_row, row_count, _p(y)) == 1
    return y


def dequantize_rows(buf, ggml_type, rows, cols, first_row, row_count, offset=0):
    v = view(buf, ggml_type, rows, cols, offset)
    out = np.empty((row_count, cols), dtype=np.float32)
    assert lib().oracle_dequantize_rows(ctypes.byref(v), first_row, row_count, _p(out)) == 1
    return out


def row_stats(buf, ggml_type, rows, cols, x, first_row=0, row_count=None):
    """Float64 brute force: (sum w*x, sum |w*x|) per row."""
    row_count = rows - first_row if row_count is None else row_count
    v = view(buf, ggml_type, rows, cols)
    x = np.ascontiguousarray(x, dtype=np.float32)
    dot = np.empty(row_count, dtype=np.float64)
    absdot = np.empty(row_count, dtype=np.float64)
    assert lib().oracle_row_stats_f64(ctypes.byref(v), _p(x), first_row, row_count, _p(dot), _p(absdot)) == 1
    return dot, absdot


def greedy_argmax(logits):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    tok = ctypes.c_int(-7)
    ok = lib().oracle_greedy_argmax(_p(logits), logits.size, ctypes.byref(tok))
    return ok, tok.value


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def add(left, right):
    """tensor_add_f32 restated: (ok, left + right in fp32)."""
    left, right = _f32(left), _f32(right)
    out = np.empty_like(left)
    ok = lib().oracle_add_f32(_p(left), _p(right), left.size, _p(out))
    return ok, out


def rms_norm(x, weight, epsilon):
    """tensor_rms_norm_f32 restated on one vector: (ok, output)."""
    x, weight = _f32(x), _f32(weight)
    out = np.empty_like(x)
    ok = lib().oracle_rms_norm_f32(_p(x), _p(weight), x.size, float(epsilon), _p(out))
    return ok, out


def swiglu(gate, up):
    """transformer_swiglu_f32 restated, out of place: (ok, up * silu(gate))."""
    gate, up = _f32(gate), _f32(up)
    out = np.empty_like(gate)
    ok = lib().oracle_swiglu_f32(_p(gate), _p(up), gate.size, _p(out))
    return ok, out
