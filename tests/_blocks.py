"""Test-side block builders and independent decoders.

* Block assembly from the field-by-field known-answer fixtures
  (tests/golden/reference_kats.json).
* The reference's LCG (rng = rng * 1664525 + 1013904223, seed 0x12345678) and
  its 128-trial random blocks (tests/q*_reference_test.cpp).
* The constant-valued blocks of tests/qwen2_quantized_test_utils.h:29-71.
* Float64 / exact-rational decoders written straight from the documented
  equations (include/quantization.h), vectorised with numpy and structured
  differently from the oracle, so a mistake in the oracle's index math
  or rounding shows up as a mismatch.
"""
from __future__ import annotations

import json
import os
from fractions import Fraction

import numpy as np

Q5_0, Q8_0, Q4_K, Q6_K = 6, 8, 12, 14
BLOCK_ELEMENTS = {Q5_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q5_0: 22, Q8_0: 34, Q4_K: 144, Q6_K: 210}
ALL_TYPES = (Q5_0, Q8_0, Q4_K, Q6_K)
NAMES = {Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def _u16(v):
    return [v & 0xFF, (v >> 8) & 0xFF]


def _fill(arr, mapping):
    for k, v in mapping.items():
        arr[int(k)] = v & 0xFF if isinstance(v, int) else v
    return arr


def q8_0_block(d, qs_map):
    qs = [0] * 32
    _fill(qs, qs_map)
    return bytes(_u16(d) + [q & 0xFF for q in qs])


def q5_0_block(d, qs_map, qh_map):
    qh = _fill([0] * 4, qh_map)
    qs = _fill([0] * 16, qs_map)
    return bytes(_u16(d) + qh + qs)


def q4_k_block(d, dmin, scales, qs_map):
    qs = _fill([0] * 128, qs_map)
    return bytes(_u16(d) + _u16(dmin) + list(scales) + qs)


def q6_k_block(d, scales, qh_fill, ql_map):
    ql = _fill([0] * 128, ql_map)
    qh = [qh_fill] * 64
    return bytes(ql + qh + [s & 0xFF for s in scales] + _u16(d))


def kat_block(name):
    k = KATS
    if name == "q8_0_dequant":
        return q8_0_block(k[name]["d"], k[name]["qs"])
    if name == "q8_0_dot":
        return q8_0_block(k[name]["d"], k[name]["qs"])
    if name == "q5_0":
        b = k["q5_0_block"]
        return q5_0_block(b["d"], b["qs"], b["qh"])
    if name == "q4_k":
        b = k["q4_k_block"]
        return q4_k_block(b["d"], b["dmin"], b["scales"], b["qs"])
    if name == "q6_k":
        b = k["q6_k_block"]
        return q6_k_block(b["d"], b["scales"], b["qh_fill"], b["ql"])
    raise KeyError(name)


def sparse_vector(n, mapping):
    x = np.zeros(n, dtype=np.float32)
    for kk, v in mapping.items():
        x[int(kk)] = v
    return x


class Lcg:
    """rng = rng * 1664525 + 1013904223 (mod 2^32), seed 0x12345678."""

    def __init__(self, seed=0x12345678):
        self.s = seed

    def next_byte(self):
        self.s = (self.s * 1664525 + 1013904223) & 0xFFFFFFFF
        return self.s >> 24

    def next_input(self):
        return np.float32((self.next_byte() - 128) / 32.0)


def lcg_trials(ggml_type, trials=128):
    """The reference's randomized blocks and inputs, trial by trial, in the
    same draw order as its tests."""
    rng = Lcg()
    out = []
    for t in range(trials):
        if ggml_type == Q8_0:
            d = 0xB800 if t & 1 else 0x3800
            qs, x = [], []
            for _ in range(32):
                qs.append(rng.next_byte())
                x.append(rng.next_input())
            blk = bytes(_u16(d) + qs)
        elif ggml_type == Q5_0:
            d = 0xB800 if t & 1 else 0x3800
            qh = [rng.next_byte() for _ in range(4)]
            qs = [rng.next_byte() for _ in range(16)]
            x = [rng.next_input() for _ in range(32)]
            blk = bytes(_u16(d) + qh + qs)
        elif ggml_type == Q4_K:
            d = 0xB800 if t & 1 else 0x3800
            dm = 0xB400 if t & 2 else 0x3400
            sc = [rng.next_byte() for _ in range(12)]
            qs = [rng.next_byte() for _ in range(128)]
            x = [rng.next_input() for _ in range(256)]
            blk = bytes(_u16(d) + _u16(dm) + sc + qs)
        else:
            d = 0xB800 if t & 1 else 0x3800
            ql = [rng.next_byte() for _ in range(128)]
            qh = [rng.next_byte() for _ in range(64)]
            sc = [rng.next_byte() for _ in range(16)]
            x = [rng.next_input() for _ in range(256)]
            blk = bytes(ql + qh + sc + _u16(d))
        out.append((np.frombuffer(blk, dtype=np.uint8).copy(), np.array(x, dtype=np.float32)))
    return out


LCG_TOLERANCE = {Q8_0: (1e-4, 2e-5), Q5_0: (1e-4, 2e-5), Q4_K: (0.002, 5e-5), Q6_K: (0.01, 5e-5)}


def fixture_block(ggml_type, index, small_scale=False):
    """(bytes, value) of the reference's constant-valued fixture block."""
    scale = KATS["fixture_scales"][index % 6]
    factor = float(index % 6 + 1)
    if small_scale:
        scale -= 10 << 10
        factor /= 1024.0
    if ggml_type == Q5_0:
        blk = bytes(_u16(scale) + [0] * 20)
    elif ggml_type == Q8_0:
        blk = bytes(_u16(scale) + [2] * 32)
    elif ggml_type == Q4_K:
        blk = bytes(_u16(scale) + [0, 0] + [1] * 12 + [0x33] * 128)
    else:
        blk = bytes([0] * 192 + [1] * 16 + _u16(scale))
    return blk, KATS["fixture_values_per_factor"][str(ggml_type)] * factor


# ---- independent decoders ------------------------------------------------------

def f16_values(codes: np.ndarray) -> np.ndarray:
    """numpy's own binary16 conversion (an independent implementation)."""
    return np.asarray(codes, dtype=np.uint16).view(np.float16).astype(np.float64)


def _blocks(raw: np.ndarray, ggml_type) -> np.ndarray:
    bb = BLOCK_BYTES[ggml_type]
    return np.asarray(raw, dtype=np.uint8).reshape(-1, bb)


def decode_exact(raw: np.ndarray, ggml_type) -> np.ndarray:
    """Float32 weights [nblocks, block_elements], rounded exactly once (RNE)
    from the exact value of each documented equation."""
    b = _blocks(raw, ggml_type)
    n = b.shape[0]
    if ggml_type == Q8_0:
        d = f16_values(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
        q = b[:, 2:34].view(np.int8).astype(np.float64)
        return (d[:, None] * q).astype(np.float32)  # product exact in both
    if ggml_type == Q5_0:
        d = f16_values(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
        qh = (b[:, 2].astype(np.uint32) | (b[:, 3].astype(np.uint32) << 8) |
              (b[:, 4].astype(np.uint32) << 16) | (b[:, 5].astype(np.uint32) << 24))
        qs = b[:, 6:22].astype(np.int64)
        nib = np.concatenate([qs & 15, qs >> 4], axis=1)  # weights 0..15, 16..31
        bits = (qh[:, None] >> np.arange(32, dtype=np.uint32)[None, :]) & 1
        q = (nib + 16 * bits.astype(np.int64) - 16).astype(np.float64)
        return (d[:, None] * q).astype(np.float32)
    if ggml_type == Q6_K:
        ql = b[:, 0:128].astype(np.int64)
        qh = b[:, 128:192].astype(np.int64)
        sc = b[:, 192:208].view(np.int8).astype(np.float64)
        d = f16_values(b[:, 208].astype(np.uint16) | (b[:, 209].astype(np.uint16) << 8))
        idx = np.arange(256)
        g, l = idx // 128, idx % 128
        r, o = l // 32, l % 32
        low = (ql[:, 64 * g + 32 * (r % 2) + o] >> (4 * (r // 2))) & 15
        high = (qh[:, 32 * g + o] >> (2 * r)) & 3
        q = (low | (high << 4)) - 32
        s = sc[:, 8 * g + 2 * r + o // 16]
        return (d[:, None] * s * q).astype(np.float32)  # exact: <= 24 significant bits
    # Q4_K: the one decode with a rounding; compute exactly and round once.
    d = f16_values(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    dmin = f16_values(b[:, 2].astype(np.uint16) | (b[:, 3].astype(np.uint16) << 8))
    p = b[:, 4:16].astype(np.int64)
    sc = np.empty((n, 8), dtype=np.int64)
    mn = np.empty((n, 8), dtype=np.int64)
    for s in range(8):
        if s < 4:
            sc[:, s] = p[:, s] & 63
            mn[:, s] = p[:, s + 4] & 63
        else:
            sc[:, s] = (p[:, s + 4] & 15) | ((p[:, s - 4] >> 6) << 4)
            mn[:, s] = (p[:, s + 4] >> 4) | ((p[:, s] >> 6) << 4)
    qs = b[:, 16:144].astype(np.int64)
    out = np.empty((n, 256), dtype=np.float32)
    for blk in range(n):
        for s in range(8):
            a64 = d[blk] * float(sc[blk, s])       # exact in float64, keeps the sign of zero
            m64 = dmin[blk] * float(mn[blk, s])
            a, m = Fraction(a64), Fraction(m64)
            grp = qs[blk, 32 * (s // 2): 32 * (s // 2) + 32]
            vals = (grp >> (4 * (s % 2))) & 15
            for j in range(32):
                exact = a * int(vals[j]) - m
                if exact == 0:
                    # IEEE sum of zeros: -0 only when both terms are -0.
                    t1, t2 = a64 * float(vals[j]), -m64
                    neg = t1 == 0 and t2 == 0 and np.signbit(t1) and np.signbit(t2)
                    out[blk, 32 * s + j] = np.float32(-0.0 if neg else 0.0)
                else:
                    out[blk, 32 * s + j] = f32_round(exact)
    return out


def f32_round(f: Fraction) -> np.float32:
    """Round an exact rational to binary32, nearest-even."""
    if f == 0:
        return np.float32(0.0)
    c = np.float32(float(f))
    cands = {float(c), float(np.nextafter(c, np.float32(np.inf))), float(np.nextafter(c, np.float32(-np.inf)))}

    def key(v):
        bits = int(np.array(v, dtype=np.float32).view(np.uint32))
        return (abs(Fraction(v) - f), bits & 1)

    return np.float32(min(cands, key=key))


def raw_blocks(ggml_type, nblocks, seed):
    """Random bytes for nblocks blocks with finite, varied fp16 scales (normal,
    subnormal, negative, zero)."""
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(nblocks, BLOCK_BYTES[ggml_type]), dtype=np.uint8)
    specials = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0x1234, 0x8123],
                        dtype=np.uint16)

    def scale_code():
        if rng.random() < 0.3:
            return int(rng.choice(specials))
        code = int(rng.integers(0, 0x7C00))  # finite, any exponent
        return code | (0x8000 if rng.random() < 0.5 else 0)

    for i in range(nblocks):
        if ggml_type == Q6_K:
            raw[i, 208:210] = _u16(scale_code())
        else:
            raw[i, 0:2] = _u16(scale_code())
            if ggml_type == Q4_K:
                raw[i, 2:4] = _u16(scale_code())
    return raw.reshape(-1)
