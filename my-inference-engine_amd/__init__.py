"""MI355X packed-weight matrix-vector path (Q8_0 / Q5_0 / Q4_K / Q6_K x fp32).

Python mirror of the reference engine's packed matvec interface
(src/quantized_matvec.h:32-50 of trungnguyen21/my-inference-engine) on top of
the C ABI of ``csrc/libqmv_hip.so`` (declared in ``include/qmv_hip.h``).
Every compute call runs on the GPU; if the HIP library is missing the
loader raises instead of falling back to anything else.

Import with ``importlib.import_module("my-inference-engine_amd")`` (the
directory name is not a Python identifier).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
# QMV_HIP_LIB may name another build of the same library (e.g. a tuning variant).
HIP_LIB_PATH = os.environ.get("QMV_HIP_LIB") or os.path.join(CSRC, "libqmv_hip.so")
SYNTH_LIB_PATH = os.path.join(CSRC, "libqmv_synth.so")

# GGML type codes (src/gguf_reader.h:7-11) and block geometry
# (include/quantization.h:6-23).
GGML_TYPE_Q5_0 = 6
GGML_TYPE_Q8_0 = 8
GGML_TYPE_Q4_K = 12
GGML_TYPE_Q6_K = 14
BLOCK_ELEMENTS = {GGML_TYPE_Q5_0: 32, GGML_TYPE_Q8_0: 32, GGML_TYPE_Q4_K: 256, GGML_TYPE_Q6_K: 256}
BLOCK_BYTES = {GGML_TYPE_Q5_0: 22, GGML_TYPE_Q8_0: 34, GGML_TYPE_Q4_K: 144, GGML_TYPE_Q6_K: 210}
TYPE_NAMES = {GGML_TYPE_Q5_0: "Q5_0", GGML_TYPE_Q8_0: "Q8_0", GGML_TYPE_Q4_K: "Q4_K", GGML_TYPE_Q6_K: "Q6_K"}
MAX_BATCH = 32  # QMV_MAX_BATCH: positions per device call (host calls take any batch)
MAX_GROUP = 8


class QmvTensorView(ctypes.Structure):
    """Same layout as GgufQuantizedTensorView (src/gguf_reader.h:31-40)."""

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


def make_view(buf: np.ndarray, ggml_type: int, rows: int, cols: int, offset: int = 0) -> QmvTensorView:
    """A consistent view of ``rows x cols`` packed weights at ``buf[offset:]``.

    The view borrows ``buf``'s bytes, as the reference's views borrow the GGUF
    mmap; it also holds a Python reference to ``buf`` so that a temporary array
    passed straight in outlives the view."""
    be, bb = BLOCK_ELEMENTS[ggml_type], BLOCK_BYTES[ggml_type]
    v = QmvTensorView()
    v._owner = buf
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


def packed_bytes(ggml_type: int, rows: int, cols: int) -> int:
    return rows * (cols // BLOCK_ELEMENTS[ggml_type]) * BLOCK_BYTES[ggml_type]


_fp = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_view_p = ctypes.POINTER(QmvTensorView)

# name -> (restype, argtypes); mirrors include/qmv_hip.h
HIP_SIGNATURES = {
    "qmv_tensor_matvec_f32": (ctypes.c_int, [_view_p, _vp, ctypes.c_int, _vp, ctypes.c_int]),
    "qmv_tensor_matmul_f32": (ctypes.c_int, [_view_p, _vp, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int]),
    "qmv_register_tensor": (ctypes.c_int, [_view_p]),
    "qmv_reserve_calls": (ctypes.c_int, [_view_p, ctypes.c_int]),
    "qmv_reserve_contexts": (ctypes.c_int, [ctypes.c_int]),
    "qmv_allocation_count": (ctypes.c_ulonglong, []),
    "qmv_release_tensor": (ctypes.c_int, [_vp]),
    "qmv_release_all": (None, []),
    "qmv_dequantize_rows_f32": (ctypes.c_int, [_view_p, ctypes.c_int, ctypes.c_int, _vp]),
    "qmv_greedy_sample_f32": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]),
    "qmv_device_tensor_create": (ctypes.c_int, [_view_p, ctypes.POINTER(_vp)]),
    "qmv_device_tensor_destroy": (None, [_vp]),
    "qmv_device_tensor_info": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                                              ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint64),
                                              ctypes.POINTER(ctypes.c_uint64)]),
    "qmv_device_matvec_f32": (ctypes.c_int, [_vp, _vp, ctypes.c_int, _vp, _vp]),
    "qmv_device_matvec_group_f32": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.c_int, _vp, ctypes.c_int,
                                                   ctypes.POINTER(_vp), _vp]),
    "qmv_device_matvec_group_noalloc_f32": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.c_int, _vp, ctypes.c_int,
                                                           ctypes.POINTER(_vp), _vp]),
    "qmv_device_dequantize_f32": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _vp, _vp]),
    "qmv_device_greedy_argmax_f32": (ctypes.c_int, [_vp, ctypes.c_int, _vp, _vp]),
    "qmv_last_error": (ctypes.c_char_p, []),
    "qmv_set_device": (ctypes.c_int, [ctypes.c_int]),
    "qmv_device_count": (ctypes.c_int, []),
    "qmv_debug_fail_next_calls": (None, [ctypes.c_int]),
    "qmv_device_matvec_argmax_f32": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "qmv_device_embed_rows_f32": (ctypes.c_int, [_vp, _vp, ctypes.c_int, _vp, _vp, _vp]),
    "qmv_set_launch_tuning": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qmv_set_rowmajor": (None, [ctypes.c_int, ctypes.c_int]),
    "qmv_device_matvec_add_group_f32": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.c_int, _vp, ctypes.c_int,
                                                       ctypes.POINTER(_vp), ctypes.POINTER(ctypes.c_int),
                                                       ctypes.POINTER(_vp), _vp]),
    "qmv_device_matvec_swiglu_f32": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int, _vp, _vp]),
    "qmv_device_rms_norm_f32": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_float, _vp, _vp]),
    "qmv_device_rms_norm_matvec_add_group_f32": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.c_int, _vp, _vp,
                                                                ctypes.c_float, ctypes.c_int, ctypes.POINTER(_vp),
                                                                ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_vp),
                                                                _vp, _vp]),
    "qmv_device_rms_norm_matvec_swiglu_f32": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_float, ctypes.c_int, _vp,
                                                             _vp, _vp]),
}

SYNTH_SIGNATURES = {
    "qmv_synth_tensor_bytes": (ctypes.c_uint64, [ctypes.c_uint32, ctypes.c_int, ctypes.c_int]),
    "qmv_synth_tensor": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_int, ctypes.c_int, ctypes.c_uint64, _vp,
                                        ctypes.c_uint64]),
    "qmv_synth_normal_f32": (ctypes.c_int, [_vp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double]),
    "qmv_synth_f64_to_f16": (ctypes.c_uint16, [ctypes.c_double]),
    "qmv_synth_hash": (ctypes.c_uint64, [_vp, ctypes.c_uint64]),
}

_hip = None
_synth = None


def _bind(lib, sigs):
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def hip_lib() -> ctypes.CDLL:
    """The product library. Raises if it has not been built."""
    global _hip
    if _hip is None:
        if not os.path.exists(HIP_LIB_PATH):
            raise RuntimeError(f"{HIP_LIB_PATH} is missing: run __graft_entry__.build() (make -C csrc)")
        _hip = _bind(ctypes.CDLL(HIP_LIB_PATH), HIP_SIGNATURES)
    return _hip


def synth_lib() -> ctypes.CDLL:
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_LIB_PATH):
            raise RuntimeError(f"{SYNTH_LIB_PATH} is missing: run __graft_entry__.build()")
        _synth = _bind(ctypes.CDLL(SYNTH_LIB_PATH), SYNTH_SIGNATURES)
    return _synth


def build(jobs: int = 8) -> None:
    """Compile csrc/ in place (always recompiles)."""
    subprocess.run(["make", "-B", f"-j{jobs}", "-C", CSRC], check=True)


def last_error() -> str:
    return hip_lib().qmv_last_error().decode()


class QmvError(RuntimeError):
    pass


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


# ---- drop-in host-pointer API ------------------------------------------------

def quantized_tensor_matvec_f32(view: QmvTensorView, inp: np.ndarray, input_count: int, out: np.ndarray,
                                output_count: int) -> int:
    """Same arguments and 1/0 result as the reference's function."""
    return hip_lib().qmv_tensor_matvec_f32(ctypes.byref(view), _ptr(inp), input_count, _ptr(out), output_count)


def quantized_tensor_matmul_f32(view: QmvTensorView, inp: np.ndarray, input_count: int, batch_count: int,
                                out: np.ndarray, output_count: int) -> int:
    return hip_lib().qmv_tensor_matmul_f32(ctypes.byref(view), _ptr(inp), input_count, batch_count, _ptr(out),
                                           output_count)


def matvec(view: QmvTensorView, x: np.ndarray) -> np.ndarray:
    """y = W x (x: [K] or [B, K] float32) on the GPU; raises on failure."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = int(view.dimensions[1]), int(view.dimensions[0])
    batch = 1 if x.ndim == 1 else x.shape[0]
    y = np.empty((batch, rows) if x.ndim == 2 else (rows,), dtype=np.float32)
    ok = quantized_tensor_matmul_f32(view, x, cols, batch, y, rows)
    if not ok:
        raise QmvError(last_error())
    return y


def dequantize_rows(view: QmvTensorView, first_row: int, row_count: int) -> np.ndarray:
    out = np.empty((row_count, int(view.dimensions[0])), dtype=np.float32)
    if not hip_lib().qmv_dequantize_rows_f32(ctypes.byref(view), first_row, row_count, _ptr(out)):
        raise QmvError(last_error())
    return out


def greedy_sample(logits: np.ndarray):
    """(ok, token_id) with the reference sampler's contract."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    tok = ctypes.c_int(-7)
    ok = hip_lib().qmv_greedy_sample_f32(_ptr(logits), logits.size, ctypes.byref(tok))
    return ok, tok.value


def set_launch_tuning(target_waves: int = 0, units_per_wave: int = 0, waves_per_group: int = 0,
                      mfma_min_batch: int = 0) -> None:
    """Process-wide launch-plan override (0 = automatic); see qmv_hip.h."""
    hip_lib().qmv_set_launch_tuning(target_waves, units_per_wave, waves_per_group, mfma_min_batch)


def set_rowmajor(enable: bool = True, rows: int = 2) -> None:
    """Row-major kernel for small single-position Q4_K launches on/off (and
    its GGUF copies for tensors uploaded afterwards); rows per row segment."""
    hip_lib().qmv_set_rowmajor(1 if enable else 0, rows)


def register_tensor(view: QmvTensorView) -> int:
    return hip_lib().qmv_register_tensor(ctypes.byref(view))


def reserve_calls(view: QmvTensorView, max_batch: int) -> None:
    """Register the tensor and pre-size every pooled host context's staging
    and workspace for host calls of up to ``max_batch`` positions on it, from
    any thread."""
    if not hip_lib().qmv_reserve_calls(ctypes.byref(view), max_batch):
        raise QmvError(last_error())


def reserve_contexts(count: int) -> None:
    """Declare ``count`` concurrent host-pointer callers: the device's context
    pool gets that many contexts, sized like the reservations, and is closed."""
    if not hip_lib().qmv_reserve_contexts(count):
        raise QmvError(last_error())


def allocation_count() -> int:
    """Device/pinned allocations and stream creations made by the library."""
    return hip_lib().qmv_allocation_count()


def release_tensor(data_ptr: int) -> int:
    return hip_lib().qmv_release_tensor(data_ptr)


def release_all() -> None:
    hip_lib().qmv_release_all()


# ---- device-resident API ---------------------------------------------------------

class DeviceTensor:
    """A packed tensor resident in HBM (tiled layout), owned by this object."""

    def __init__(self, view: QmvTensorView):
        h = ctypes.c_void_p()
        if not hip_lib().qmv_device_tensor_create(ctypes.byref(view), ctypes.byref(h)):
            raise QmvError(last_error())
        self.handle = h
        r, c, t = ctypes.c_int(), ctypes.c_int(), ctypes.c_uint32()
        pb, db = ctypes.c_uint64(), ctypes.c_uint64()
        hip_lib().qmv_device_tensor_info(h, ctypes.byref(r), ctypes.byref(c), ctypes.byref(t), ctypes.byref(pb),
                                         ctypes.byref(db))
        self.rows, self.cols, self.ggml_type = r.value, c.value, t.value
        self.packed_bytes, self.device_bytes = pb.value, db.value

    def matvec(self, d_x: int, batch: int, d_y: int, stream: int = 0) -> None:
        if not hip_lib().qmv_device_matvec_f32(self.handle, d_x, batch, d_y, stream):
            raise QmvError(last_error())

    def dequantize(self, first_row: int, row_count: int, d_out: int, stream: int = 0) -> None:
        if not hip_lib().qmv_device_dequantize_f32(self.handle, first_row, row_count, d_out, stream):
            raise QmvError(last_error())

    def close(self) -> None:
        if self.handle:
            hip_lib().qmv_device_tensor_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def device_matvec_group(tensors: Sequence[DeviceTensor], d_x: int, batch: int, d_outs: Sequence[int],
                        stream: int = 0) -> None:
    n = len(tensors)
    hs = (ctypes.c_void_p * n)(*[t.handle for t in tensors])
    outs = (ctypes.c_void_p * n)(*d_outs)
    if not hip_lib().qmv_device_matvec_group_f32(hs, n, d_x, batch, outs, stream):
        raise QmvError(last_error())


def device_matvec_group_noalloc(tensors: Sequence[DeviceTensor], d_x: int, batch: int, d_outs: Sequence[int],
                                stream: int = 0) -> None:
    """device_matvec_group with its split-K workspace in the library's fixed
    device scratch array: allocates nothing; overlapping calls on one GPU race."""
    n = len(tensors)
    hs = (ctypes.c_void_p * n)(*[t.handle for t in tensors])
    outs = (ctypes.c_void_p * n)(*d_outs)
    if not hip_lib().qmv_device_matvec_group_noalloc_f32(hs, n, d_x, batch, outs, stream):
        raise QmvError(last_error())


def device_matvec_add_group(tensors: Sequence[DeviceTensor], d_x: int, batch: int, d_adds: Sequence[int],
                            add_strides: Sequence[int], d_outs: Sequence[int], stream: int = 0) -> None:
    """Grouped matvec with y_i += add_i fused (stride 0: a bias for every
    position; stride N_i with add_i == y_i: a residual added in place; a 0
    address: no addend)."""
    n = len(tensors)
    hs = (ctypes.c_void_p * n)(*[t.handle for t in tensors])
    adds = (ctypes.c_void_p * n)(*[a or None for a in d_adds])
    lds = (ctypes.c_int * n)(*add_strides)
    outs = (ctypes.c_void_p * n)(*d_outs)
    if not hip_lib().qmv_device_matvec_add_group_f32(hs, n, d_x, batch, adds, lds, outs, stream):
        raise QmvError(last_error())


def device_matvec_swiglu(gate: DeviceTensor, up: DeviceTensor, d_x: int, batch: int, d_out: int,
                         stream: int = 0) -> None:
    """d_out[b, r] = up(x_b)[r] * silu(gate(x_b)[r]) in one launch."""
    if not hip_lib().qmv_device_matvec_swiglu_f32(gate.handle, up.handle, d_x, batch, d_out, stream):
        raise QmvError(last_error())


def device_rms_norm(d_x: int, d_weight: int, length: int, batch: int, epsilon: float, d_out: int,
                    stream: int = 0) -> None:
    if not hip_lib().qmv_device_rms_norm_f32(d_x, d_weight, length, batch, epsilon, d_out, stream):
        raise QmvError(last_error())


def device_rms_norm_matvec_add_group(tensors: Sequence[DeviceTensor], d_x: int, d_norm_w: int, epsilon: float,
                                     batch: int, d_adds: Optional[Sequence[int]], add_strides: Optional[Sequence[int]],
                                     d_outs: Sequence[int], d_normed: int, stream: int = 0) -> None:
    """RMSNorm of x (norm weights d_norm_w) fused with the grouped matvec (and
    its addends, as device_matvec_add_group; None for plain stores). d_normed:
    batch x K floats the library may use for the normalised input."""
    n = len(tensors)
    hs = (ctypes.c_void_p * n)(*[t.handle for t in tensors])
    adds = (ctypes.c_void_p * n)(*[a or None for a in d_adds]) if d_adds is not None else None
    lds = (ctypes.c_int * n)(*add_strides) if add_strides is not None else None
    outs = (ctypes.c_void_p * n)(*d_outs)
    if not hip_lib().qmv_device_rms_norm_matvec_add_group_f32(hs, n, d_x, d_norm_w, epsilon, batch, adds, lds, outs,
                                                              d_normed, stream):
        raise QmvError(last_error())


def device_rms_norm_matvec_swiglu(gate: DeviceTensor, up: DeviceTensor, d_x: int, d_norm_w: int, epsilon: float,
                                  batch: int, d_out: int, d_normed: int, stream: int = 0) -> None:
    """RMSNorm of x fused with the gate/up projections and SwiGLU."""
    if not hip_lib().qmv_device_rms_norm_matvec_swiglu_f32(gate.handle, up.handle, d_x, d_norm_w, epsilon, batch,
                                                           d_out, d_normed, stream):
        raise QmvError(last_error())


def device_matvec_argmax(tensor: "DeviceTensor", d_x: int, d_logits: int, d_result: int, stream: int = 0) -> None:
    """Fused vocab projection + greedy argmax (M = 1) on device buffers."""
    if hip_lib().qmv_device_matvec_argmax_f32(tensor.handle, d_x, d_logits, d_result, stream) != 1:
        raise QmvError(last_error())


def device_embed_rows(tensor: "DeviceTensor", d_ids: int, count: int, d_out: int, stream: int = 0,
                      d_status: int = 0) -> None:
    """Decode rows d_ids[0..count) of a device tensor into d_out[count, K];
    with d_status, d_status[0] = 1 if every id was in range, else 0."""
    if hip_lib().qmv_device_embed_rows_f32(tensor.handle, d_ids, count, d_out, d_status or None, stream) != 1:
        raise QmvError(last_error())


def device_greedy_argmax(d_logits: int, vocab: int, d_result: int, stream: int = 0) -> None:
    if not hip_lib().qmv_device_greedy_argmax_f32(d_logits, vocab, d_result, stream):
        raise QmvError(last_error())


# ---- synthetic inputs ------------------------------------------------------------------

def synth_tensor(ggml_type: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Seeded packed tensor (row-major GGUF bytes) with the benchmark distributions."""
    lib = synth_lib()
    n = lib.qmv_synth_tensor_bytes(ggml_type, rows, cols)
    if n == 0:
        raise ValueError("invalid shape for type")
    buf = np.empty(n, dtype=np.uint8)
    if not lib.qmv_synth_tensor(ggml_type, rows, cols, seed, _ptr(buf), n):
        raise RuntimeError("synth failed")
    return buf


def synth_normal(n: int, seed: int, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    synth_lib().qmv_synth_normal_f32(_ptr(out), n, seed, sigma)
    return out


def content_hash(a: np.ndarray) -> int:
    return synth_lib().qmv_synth_hash(_ptr(a), a.nbytes)
