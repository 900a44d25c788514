"""ctypes front end of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loads oracle/liboracle.so (the plain-C restatement, qc_oracle.c) and, when it
has been built, oracle/_ref/libqcref.so (the reference's own sources compiled
by oracle/Makefile `ref`).  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import this module, and only as the checker.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libqcref.so")

Q8_0, Q4_0 = 0, 1
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}

_P = ctypes.c_void_p
_LL = ctypes.c_longlong


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def build():
    subprocess.check_call(["make", "-s", "-C", HERE, "all"])


_ROPE_ARGS = [ctypes.c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P, _LL, _LL, _LL, _LL, _LL, _LL,
              ctypes.c_int, ctypes.c_int]


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    lib.qco_fp16_to_fp32.restype = ctypes.c_float
    lib.qco_fp16_to_fp32.argtypes = [ctypes.c_uint16]
    lib.qco_fp32_to_fp16.restype = ctypes.c_uint16
    lib.qco_fp32_to_fp16.argtypes = [ctypes.c_float]
    lib.qco_packed_size.argtypes = [ctypes.c_int, _LL, _LL, ctypes.POINTER(ctypes.c_size_t)]
    lib.qco_pack.argtypes = [ctypes.c_int, _P, _LL, _LL, _P]
    lib.qco_unpack.argtypes = [ctypes.c_int, _P, _LL, _LL, _P]
    for name in ("qco_q8_0_gemv", "qco_q4_0_gemv_ref"):
        getattr(lib, name).argtypes = [_P, _P, _P, _LL, _LL]
        getattr(lib, name).restype = None
    lib.qco_q4_0_gemv_avx2order.argtypes = [_P, _P, _P, _LL, _LL, ctypes.c_int]
    lib.qco_q4_0_gemv_avx2order.restype = None
    lib.qco_qgemv_f64.argtypes = [ctypes.c_int, _P, _P, _P, _P, _LL, _LL]
    lib.qco_quantize_int8.argtypes = [_P, _P, _P, _LL, _LL, _LL]
    lib.qco_qgemv_w8a8.argtypes = [ctypes.c_int, _P, _P, _P, _LL, _LL]
    lib.qco_int8_gemm.argtypes = [_P, _P, _P, _P, _P, _P, _P, _LL, _LL, _LL, ctypes.c_int]
    lib.qco_int8_gemm_entries.argtypes = [_P, _P, _P, _P, _P, _P, _LL, _LL, _P, _P]
    lib.qco_rms_norm_add_quant_int8.argtypes = [_P, _P, _P, _P, _P, _P, _LL, _LL,
                                                ctypes.c_float, _LL]
    lib.qco_quantize_int8_asymmetric.argtypes = [_P, _P, _P, _P, _LL, _LL]
    lib.qco_dequantize_int8_asymmetric.argtypes = [_P, _P, _P, _P, _LL, _LL]
    lib.qco_int8_gemm_entries.restype = None
    lib.qco_qgemv_qkv_rope_kv.argtypes = _ROPE_ARGS
    return lib


lib = _load()


def fp16_to_fp32(h: int) -> float:
    return lib.qco_fp16_to_fp32(h)


def fp32_to_fp16(f: float) -> int:
    return lib.qco_fp32_to_fp16(f)


def packed_size(fmt, n, k):
    size = ctypes.c_size_t(0)
    st = lib.qco_packed_size(fmt, n, k, ctypes.byref(size))
    return st, size.value


def pack(fmt, w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    st, size = packed_size(fmt, n, k)
    if st:
        return st, None
    out = np.zeros(size, dtype=np.uint8)
    st = lib.qco_pack(fmt, _ptr(w), n, k, _ptr(out))
    return st, out


def unpack(fmt, packed: np.ndarray, n, k):
    out = np.empty((n, k), dtype=np.float32)
    st = lib.qco_unpack(fmt, _ptr(packed), n, k, _ptr(out))
    assert st == 0, st
    return out


def gemv(fmt, packed, x, n, k, order="reference"):
    """f32 GEMV in the summation order of the reference's x86 route.

    q8_0: the sequential ref kernel; q4_0: the AVX2 q4_rows order
    (order="portable" selects q4_0_gemv_ref instead)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n, dtype=np.float32)
    if fmt == Q8_0:
        lib.qco_q8_0_gemv(_ptr(packed), _ptr(x), _ptr(y), n, k)
    elif order == "portable":
        lib.qco_q4_0_gemv_ref(_ptr(packed), _ptr(x), _ptr(y), n, k)
    else:
        lib.qco_q4_0_gemv_avx2order(_ptr(packed), _ptr(x), _ptr(y), n, k, AVX2_FLAGS)
    return y


# Contraction pattern of the reference's AVX2 q4_0 build, pinned against
# oracle/_ref in tests/test_oracle.py (bit 0: fused scale-add, bit 1: fused
# lane-pair sum).
AVX2_FLAGS = 3


def gemv_f64(fmt, packed, x, n, k):
    """f64 contract oracle over exactly dequantized weights, plus row norms."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n, dtype=np.float64)
    wn = np.empty(n, dtype=np.float64)
    st = lib.qco_qgemv_f64(fmt, _ptr(packed), _ptr(x), _ptr(y), _ptr(wn), n, k)
    assert st == 0, st
    return y, wn


def qgemm_f64(fmt, packed, x, n, k):
    """Per-row contract oracle of qgemm (kernels/quantization/qgemm_ref.cpp:156-162)."""
    m = x.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    wn = None
    for r in range(m):
        y[r], wn = gemv_f64(fmt, packed, x[r], n, k)
    return y, wn


def quantize_int8(x: np.ndarray, group_size=0):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, dim = x.shape
    g = dim if group_size == 0 else group_size
    codes = np.zeros((rows, dim), dtype=np.int8)
    scales = np.zeros((rows, dim // g if g and dim % g == 0 else 1), dtype=np.float32)
    st = lib.qco_quantize_int8(_ptr(x), _ptr(codes), _ptr(scales), rows, dim, group_size)
    return st, codes, scales


# Sentinels for outputs a call may leave unwritten (invalid groups).
CODE_SENTINEL = 0x5A
SCALE_SENTINEL = -7.0


def _norm_outputs(rows, hidden, group_size):
    g = hidden if group_size == 0 else group_size
    groups = hidden // g if g > 0 and hidden % g == 0 else 1
    codes = np.full((rows, hidden), CODE_SENTINEL, dtype=np.int8)
    resid = np.zeros((rows, hidden), dtype=np.float32)
    scales = np.full((rows, groups), SCALE_SENTINEL, dtype=np.float32)
    return codes, resid, scales


def rms_norm_add_quant_int8(x, residual, weight, eps=1e-5, group_size=0):
    """Residual add + RMSNorm + dynamic int8 quantization.  Returns (status,
    codes, residual_out, scales); unwritten outputs keep the sentinels."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    residual = np.ascontiguousarray(residual, dtype=np.float32)
    weight = np.ascontiguousarray(weight, dtype=np.float32)
    rows, hidden = x.shape
    codes, resid, scales = _norm_outputs(rows, hidden, group_size)
    st = lib.qco_rms_norm_add_quant_int8(_ptr(x), _ptr(residual), _ptr(weight), _ptr(codes),
                                         _ptr(resid), _ptr(scales), rows, hidden, eps,
                                         group_size)
    return st, codes, resid, scales


def quantize_int8_asymmetric(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, dim = x.shape
    codes = np.zeros((rows, dim), dtype=np.int8)
    scales = np.zeros(rows, dtype=np.float32)
    zps = np.zeros(rows, dtype=np.int32)
    st = lib.qco_quantize_int8_asymmetric(_ptr(x), _ptr(codes), _ptr(scales), _ptr(zps), rows,
                                          dim)
    return st, codes, scales, zps


def dequantize_int8_asymmetric(codes, scales, zps):
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    rows, dim = codes.shape
    out = np.zeros((rows, dim), dtype=np.float32)
    st = lib.qco_dequantize_int8_asymmetric(_ptr(codes), _ptr(np.ascontiguousarray(scales, np.float32)),
                                            _ptr(np.ascontiguousarray(zps, np.int32)), _ptr(out),
                                            rows, dim)
    return st, out


def _rope_kv_call(fn, fmt, pq, pk, pv, x, cosine, sine, query_heads, kv_heads, head_dim,
                  input_dim, slots, max_position, position, slot, key_cache=None,
                  value_cache=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    cosine = np.ascontiguousarray(cosine, dtype=np.float32)
    sine = np.ascontiguousarray(sine, dtype=np.float32)
    q = np.zeros(max(query_heads * head_dim, 1), dtype=np.float32)
    kv = max(slots * kv_heads * head_dim, 1)
    kc = np.zeros(kv, np.float32) if key_cache is None else np.array(key_cache, np.float32)
    vc = np.zeros(kv, np.float32) if value_cache is None else np.array(value_cache, np.float32)
    st = fn(fmt, _ptr(pq), _ptr(pk), _ptr(pv), _ptr(x), _ptr(cosine), _ptr(sine), _ptr(q),
            _ptr(kc), _ptr(vc), query_heads, kv_heads, head_dim, input_dim, slots, max_position,
            position, slot)
    return st, q, kc, vc


def qkv_rope_kv(fmt, pq, pk, pv, x, cosine, sine, query_heads, kv_heads, head_dim, input_dim,
                slots, max_position, position, slot, key_cache=None, value_cache=None):
    """qgemv_qkv_rope_kv in the reference's x86 row orders.  Returns
    (status, q, key_cache, value_cache); the caches start as given (zeros)."""
    return _rope_kv_call(lib.qco_qgemv_qkv_rope_kv, fmt, pq, pk, pv, x, cosine, sine,
                         query_heads, kv_heads, head_dim, input_dim, slots, max_position,
                         position, slot, key_cache, value_cache)


# ------------------------------------------------------------ canonical int8 ---

def cint8_dequant(codes, scales, zeros, rows, cols, groups):
    """The reference's f32 decode of a kInt8Symmetric / kInt8Affine tensor
    (kernels/quantization/qgemm_canonical.cpp:168-174): value = scale * (code -
    zero), each step rounded in f32; scale / zero of group col // (cols /
    groups) of the row."""
    q = np.asarray(codes, dtype=np.int8).reshape(rows, cols).astype(np.float32)
    g = cols // groups
    s = np.repeat(np.asarray(scales, np.float32).reshape(rows, groups), g, axis=1)
    if zeros is None:
        return (s * q).astype(np.float32)
    z = np.repeat(np.asarray(zeros, np.float32).reshape(rows, groups), g, axis=1)
    return (s * (q - z).astype(np.float32)).astype(np.float32)


def cint8_project_f64(x, what):
    """f64 projection x [m][cols] . what^T over the decoded weights, and each
    output row's ||w_hat_row||_2 (for the normalised contract)."""
    w = what.astype(np.float64)
    return np.asarray(x, np.float64) @ w.T, np.linalg.norm(w, axis=1)


def linear_activation_f64(v, act):
    """projection_activation (qgemm_canonical.cpp:361-379) in f64."""
    import math
    v = np.asarray(v, np.float64)
    if act == 1:
        return 0.5 * v * (1.0 + np.vectorize(math.erf)(v / math.sqrt(2.0)))
    if act == 2:
        return 0.5 * v * (1.0 + np.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))
    if act == 3:
        return v / (1.0 + np.exp(-v))
    if act == 4:
        return np.where(v > 0, v * v, 0.0)
    return v


def gemv_w8a8(fmt, packed, x, n, k):
    """qgemv_w8a8: per-32-block int8 activations, integer block dots,
    y = sum_b (float(dot) * d_w) * d_x in block order.  Returns (status, y)."""
    x = None if x is None else np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(max(n, 0), dtype=np.float32)
    st = lib.qco_qgemv_w8a8(fmt, _ptr(packed), _ptr(x), _ptr(y), n, k)
    return st, y


def gemv_w8a8_f64(fmt, packed, x, n, k):
    """The reference test's tight oracle (tests/correctness/test_qgemv_w8a8.cpp:
    65-98): dequantized weights times dequantized blockwise-int8 activations in
    f64."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    st, codes, scales = quantize_int8(x.reshape(1, k), 32)
    assert st == 0, st
    xq = codes.reshape(-1, 32).astype(np.float64) * scales.reshape(-1, 1).astype(np.float64)
    w = unpack(fmt, packed, n, k).astype(np.float64)
    return w @ xq.reshape(k)


def int8_gemm(w, x, ws, as_, row_sum=None, zp=None, asymmetric=False):
    m, k = x.shape
    n = w.shape[0]
    y = np.zeros((m, n), dtype=np.float32)
    st = lib.qco_int8_gemm(_ptr(w), _ptr(x), _ptr(ws), _ptr(as_), _ptr(row_sum), _ptr(zp),
                           _ptr(y), m, n, k, int(asymmetric))
    return st, y


def int8_gemm_entries(w, x, ws, as_, rows, cols):
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    cols = np.ascontiguousarray(cols, dtype=np.int64)
    acc = np.empty(len(rows), dtype=np.int64)
    y = np.empty(len(rows), dtype=np.float32)
    lib.qco_int8_gemm_entries(_ptr(w), _ptr(x), _ptr(ws), _ptr(as_), _ptr(rows), _ptr(cols),
                              len(rows), x.shape[1], _ptr(acc), _ptr(y))
    return acc, y


def within_contract(y, y64, wnorm, x, tol=1e-4):
    """BASELINE gate: |y - y64| <= tol * ||x||_2 * ||w_hat_row||_2, per output."""
    xn = float(np.linalg.norm(np.asarray(x, dtype=np.float64)))
    err = np.abs(np.asarray(y, dtype=np.float64) - y64)
    bound = tol * xn * wnorm
    worst = float(np.max(err / np.maximum(bound, 1e-300) * tol)) if err.size else 0.0
    return bool(np.all(err <= bound)), worst


# ------------------------------------------------------------ reference ---

class Reference:
    """The reference's own compiled hot-path functions (oracle/_ref)."""

    def __init__(self, path=REF_PATH):
        self.lib = ctypes.CDLL(path)
        L = self.lib
        L.qcref_q8_0_pack.argtypes = [_P, _LL, _LL, _P]
        L.qcref_q4_0_pack.argtypes = [_P, _LL, _LL, _P]
        for name in ("qcref_q8_0_gemv", "qcref_q4_0_gemv_avx2", "qcref_q4_0_gemv_portable"):
            getattr(L, name).argtypes = [_P, _P, _P, _LL, _LL]
            getattr(L, name).restype = None
        L.qcref_qgemm.argtypes = [ctypes.c_int, _P, _P, _P, _LL, _LL, _LL]
        L.qcref_qgemm.restype = None
        L.qcref_quantize_int8.argtypes = [_P, _P, _P, _LL, _LL, _LL]
        L.qcref_int8_gemm.argtypes = [_P, _P, _P, _P, _P, _P, _P, _LL, _LL, _LL, ctypes.c_int]
        L.qcref_int8_gemm_variant.restype = ctypes.c_char_p
        for name in ("qcref_q4_0_gemv_w8a8", "qcref_q8_0_gemv_w8a8"):
            getattr(L, name).argtypes = [_P, _P, _P, _LL, _LL]
            getattr(L, name).restype = None
        L.qcref_set_num_threads.argtypes = [ctypes.c_int]
        L.qcref_rms_norm_add_quant_int8.argtypes = [_P, _P, _P, _P, _P, _P, _LL, _LL,
                                                    ctypes.c_float, _LL]
        L.qcref_quantize_int8_asymmetric.argtypes = [_P, _P, _P, _P, _LL, _LL]
        L.qcref_dequantize_int8_asymmetric.argtypes = [_P, _P, _P, _P, _LL, _LL]
        L.qcref_set_num_threads.restype = None
        L.qcref_prepare_gguf.argtypes = [ctypes.c_int, _P, _LL, _LL, ctypes.c_int, _P, _LL, _P]
        L.qcref_prepare_smoothquant.argtypes = [_P, _P, _LL, _LL, _P, _LL, _P, ctypes.c_int, _P,
                                                _LL, _P]
        L.qcref_qgemv_qkv_rope_kv.argtypes = _ROPE_ARGS
        L.qcref_prepare_canonical_int8.argtypes = [
            ctypes.c_int, _LL, _LL, _LL, ctypes.c_int, _P, _P, _LL, _P, _P, _LL, _P, _P,
            ctypes.c_int, _P, _LL, _P]

    @staticmethod
    def available(path=REF_PATH):
        return os.path.exists(path)

    def qkv_rope_kv(self, fmt, pq, pk, pv, x, cosine, sine, query_heads, kv_heads, head_dim,
                    input_dim, slots, max_position, position, slot, key_cache=None,
                    value_cache=None):
        return _rope_kv_call(self.lib.qcref_qgemv_qkv_rope_kv, fmt, pq, pk, pv, x, cosine, sine,
                             query_heads, kv_heads, head_dim, input_dim, slots, max_position,
                             position, slot, key_cache, value_cache)

    def storage_scenarios(self, directory):
        """Runs tests/cpp/storage_scenarios.h through the reference's own
        prepared storage projections, writing under `directory`."""
        self.lib.qcref_storage_scenarios.argtypes = [ctypes.c_char_p]
        return self.lib.qcref_storage_scenarios(str(directory).encode())

    def canonical_quant_scenarios(self, directory):
        """Runs tests/cpp/canonical_quant_scenarios.h through the reference's
        own quantize_canonical / dequantize_canonical, writing under
        `directory`."""
        self.lib.qcref_canonical_quant_scenarios.argtypes = [ctypes.c_char_p]
        return self.lib.qcref_canonical_quant_scenarios(str(directory).encode())

    def pack(self, fmt, w):
        w = np.ascontiguousarray(w, dtype=np.float32)
        n, k = w.shape
        out = np.zeros(n * (k // 32) * BLOCK_BYTES[fmt], dtype=np.uint8)
        fn = self.lib.qcref_q8_0_pack if fmt == Q8_0 else self.lib.qcref_q4_0_pack
        st = fn(_ptr(w), n, k, _ptr(out))
        return st, out

    def gemv(self, fmt, packed, x, n, k, portable=False):
        y = np.empty(n, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        if fmt == Q8_0:
            self.lib.qcref_q8_0_gemv(_ptr(packed), _ptr(x), _ptr(y), n, k)
        elif portable:
            self.lib.qcref_q4_0_gemv_portable(_ptr(packed), _ptr(x), _ptr(y), n, k)
        else:
            self.lib.qcref_q4_0_gemv_avx2(_ptr(packed), _ptr(x), _ptr(y), n, k)
        return y

    def qgemm(self, fmt, packed, x, n, k):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty((x.shape[0], n), dtype=np.float32)
        self.lib.qcref_qgemm(fmt, _ptr(packed), _ptr(x), _ptr(y), x.shape[0], n, k)
        return y

    def quantize_int8(self, x, group_size=0):
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, dim = x.shape
        g = dim if group_size == 0 else group_size
        codes = np.zeros((rows, dim), dtype=np.int8)
        scales = np.zeros((rows, max(dim // g, 1)), dtype=np.float32)
        st = self.lib.qcref_quantize_int8(_ptr(x), _ptr(codes), _ptr(scales), rows, dim,
                                          group_size)
        return st, codes, scales

    def int8_gemm(self, w, x, ws, as_, row_sum=None, zp=None, asymmetric=False):
        m, k = x.shape
        n = w.shape[0]
        y = np.zeros((m, n), dtype=np.float32)
        st = self.lib.qcref_int8_gemm(_ptr(w), _ptr(x), _ptr(ws), _ptr(as_), _ptr(row_sum),
                                      _ptr(zp), _ptr(y), m, n, k, int(asymmetric))
        return st, y

    def gemv_w8a8(self, fmt, packed, x, n, k):
        y = np.empty(n, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        fn = self.lib.qcref_q8_0_gemv_w8a8 if fmt == Q8_0 else self.lib.qcref_q4_0_gemv_w8a8
        fn(_ptr(packed), _ptr(x), _ptr(y), n, k)
        return y

    def rms_norm_add_quant_int8(self, x, residual, weight, eps=1e-5, group_size=0):
        x = np.ascontiguousarray(x, dtype=np.float32)
        residual = np.ascontiguousarray(residual, dtype=np.float32)
        weight = np.ascontiguousarray(weight, dtype=np.float32)
        rows, hidden = x.shape
        codes, resid, scales = _norm_outputs(rows, hidden, group_size)
        st = self.lib.qcref_rms_norm_add_quant_int8(_ptr(x), _ptr(residual), _ptr(weight),
                                                    _ptr(codes), _ptr(resid), _ptr(scales),
                                                    rows, hidden, eps, group_size)
        return st, codes, resid, scales

    def quantize_int8_asymmetric(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, dim = x.shape
        codes = np.zeros((rows, dim), dtype=np.int8)
        scales = np.zeros(rows, dtype=np.float32)
        zps = np.zeros(rows, dtype=np.int32)
        st = self.lib.qcref_quantize_int8_asymmetric(_ptr(x), _ptr(codes), _ptr(scales),
                                                     _ptr(zps), rows, dim)
        return st, codes, scales, zps

    def dequantize_int8_asymmetric(self, codes, scales, zps):
        codes = np.ascontiguousarray(codes, dtype=np.int8)
        rows, dim = codes.shape
        out = np.zeros((rows, dim), dtype=np.float32)
        st = self.lib.qcref_dequantize_int8_asymmetric(
            _ptr(codes), _ptr(np.ascontiguousarray(scales, np.float32)),
            _ptr(np.ascontiguousarray(zps, np.int32)), _ptr(out), rows, dim)
        return st, out

    def prepare_gguf(self, fmt, packed, rows, cols, layout):
        """The reference's CpuPackedWeights::prepare: (status, panel bytes, info[24])."""
        info = np.zeros(24, dtype=np.int64)
        cap = max(1, len(packed)) * 32 + (1 << 16)
        panel = np.zeros(cap, dtype=np.uint8)
        st = self.lib.qcref_prepare_gguf(fmt, _ptr(np.ascontiguousarray(packed)), rows, cols,
                                         layout, _ptr(panel), cap, _ptr(info))
        return st, panel[:int(info[13])] if st == 0 else None, info

    def prepare_canonical_int8(self, affine, data, rows, cols, group_size, scale_mode, scales,
                               zps=None, act_scales=None, act_zps=None, row_sums=None,
                               layout=0):
        info = np.zeros(24, dtype=np.int64)
        cap = rows * cols * 32 + (1 << 16)
        panel = np.zeros(cap, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, np.float32)
        a = np.ascontiguousarray(act_scales if act_scales is not None else [], np.float32)
        st = self.lib.qcref_prepare_canonical_int8(
            int(affine), rows, cols, group_size, scale_mode,
            _ptr(np.ascontiguousarray(data, np.int8)), _ptr(scales), len(scales),
            _ptr(None if zps is None else np.ascontiguousarray(zps, np.float32)),
            _ptr(a), len(a), _ptr(None if act_zps is None else np.ascontiguousarray(act_zps, np.int32)),
            _ptr(None if row_sums is None else np.ascontiguousarray(row_sums, np.int32)),
            layout, _ptr(panel), cap, _ptr(info))
        return st, panel[:int(info[13])] if st == 0 else None, info

    def prepare_smoothquant(self, w, ws, act_scales, act_zps, layout):
        rows, cols = w.shape
        info = np.zeros(24, dtype=np.int64)
        cap = rows * cols * 32 + (1 << 16)
        panel = np.zeros(cap, dtype=np.uint8)
        st = self.lib.qcref_prepare_smoothquant(
            _ptr(np.ascontiguousarray(w, np.int8)), _ptr(np.ascontiguousarray(ws, np.float32)),
            rows, cols, _ptr(np.ascontiguousarray(act_scales, np.float32)), len(act_scales),
            _ptr(None if act_zps is None else np.ascontiguousarray(act_zps, np.int32)), layout,
            _ptr(panel), cap, _ptr(info))
        return st, panel[:int(info[13])] if st == 0 else None, info

    def variant(self):
        return self.lib.qcref_int8_gemm_variant().decode()

    def set_threads(self, n):
        self.lib.qcref_set_num_threads(n)
