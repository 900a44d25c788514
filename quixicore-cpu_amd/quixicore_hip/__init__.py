"""Python binding of the gfx950 C ABI (include/quixicore_hip.h) over ctypes.

Tensors are torch tensors on the GPU; their data pointers and the current
torch stream are handed to the C ABI unchanged.  There is no CPU fallback:
importing this module without the built library raises, and every call runs
a HIP kernel.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.dirname(HERE)
LIB_PATH = os.path.join(PKG_DIR, "lib", "libquixicore_hip.so")
SYNTH_PATH = os.path.join(HERE, "libqcsynth.so")

Q8_0, Q4_0 = 0, 1
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}
STATUS = {0: "kOk", 1: "kInvalidShape", 2: "kUnsupportedFormat", 3: "kInvalidArgument",
          4: "kOutOfMemory", 5: "kDeviceError"}

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is not built; run `make -C quixicore-cpu_amd` (or __graft_entry__.build())")

_P = ctypes.c_void_p
_LL = ctypes.c_longlong
_I = ctypes.c_int

lib = ctypes.CDLL(LIB_PATH)

_SIGS = {
    "qc_hip_version": ([], ctypes.c_char_p),
    "qc_hip_last_error": ([], ctypes.c_char_p),
    "qc_hip_qgemv_packed_size": ([_I, _LL, _LL, ctypes.POINTER(ctypes.c_size_t)], _I),
    "qc_hip_qgemv_pack": ([_I, _P, _LL, _LL, _P, _P, _P], _I),
    "qc_hip_qgemv_unpack": ([_I, _P, _LL, _LL, _P, _P], _I),
    "qc_hip_qgemv": ([_I, _P, _P, _P, _LL, _LL, _P], _I),
    "qc_hip_qgemm": ([_I, _P, _P, _P, _LL, _LL, _LL, _P], _I),
    "qc_hip_qgemm_noalloc": ([_I, _P, _P, _P, _LL, _LL, _LL, _P], _I),
    "qc_hip_qgemv_w8a8": ([_I, _P, _P, _P, _LL, _LL, _P, _P], _I),
    "qc_hip_qgemv_up_gate": ([_I, _P, _P, _P, _P, _P, _LL, _LL, _P], _I),
    "qc_hip_qgemv_up_gate_activation": ([_I, _P, _P, _P, _P, _LL, _LL, _I, _P], _I),
    "qc_hip_qgemv_qkv": ([_I, _P, _P, _P, _P, _P, _P, _P, _LL, _LL, _LL, _P], _I),
    "qc_hip_cint8_project": ([_I, _P, _I, _P, _I, _LL, _P, _P, _P, _I, _P, _P, _LL, _P], _I),
    "qc_hip_qgemv_qkv_rope_kv": ([_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _LL, _LL, _LL, _LL,
                                  _LL, _LL, _I, _I, _P], _I),
    "qc_hip_qgemv_w8a8_packed_size": ([_I, _LL, _LL, _P], _I),
    "qc_hip_qgemv_w8a8_variant": ([_I], ctypes.c_char_p),
    "qc_hip_quantize_int8": ([_P, _P, _P, _LL, _LL, _LL, _P, _P], _I),
    "qc_hip_int8_gemm": ([_P, _P, _P, _P, _P, _P, _P, _LL, _LL, _LL, _I, _P, _P], _I),
    "qc_hip_qgemm_w8a8": ([_P, _P, _P, _P, _P, _LL, _LL, _LL, _P, _P], _I),
    "qc_hip_int8_gemm_i32": ([_P, _P, _P, _LL, _LL, _LL, _P], _I),
    "qc_hip_nonfinite_scan": ([_P, _LL, _P, _P], _I),
    "qc_hip_qgemv_variant": ([_I], ctypes.c_char_p),
    "qc_hip_int8_gemm_variant": ([], ctypes.c_char_p),
    "qc_hip_set_gemv_rows_per_wave": ([_I], _I),
    "qc_hip_set_int8_gemm_route": ([_I], _I),
    "qc_hip_set_qgemm_plan": ([_I, _I], _I),
    "qc_hip_rms_norm_add_quant_int8": ([_P, _P, _P, _P, _P, _P, _LL, _LL, ctypes.c_float, _LL,
                                        _P, _P], _I),
    "qc_hip_quantize_int8_asymmetric": ([_P, _P, _P, _P, _LL, _LL, _P, _P], _I),
    "qc_hip_dequantize_int8_asymmetric": ([_P, _P, _P, _P, _LL, _LL, _P], _I),
    "qc_hip_set_norm_sequential_sum": ([_I], _I),
    "qc_hip_set_qgemm_panel": ([_I], _I),
    "qc_hip_set_qgemm_rows": ([_I], _I),
    "qc_hip_set_qgemm_fold": ([_I], _I),
    "qc_hip_set_cint8_dot": ([_I], _I),
    "qc_hip_stream_read": ([_P, _LL, _P, _I, _P], _I),
    "qc_hip_cint8_dequantize": ([_P, _P, _P, _P], _I),
    "qc_hip_cint8_quantized_gemm": ([_P, _P, _P, _P, _P], _I),
    "qc_hip_storage_to_f32": ([_P, _I, _LL, _P, _P], _I),
}
for _name, (_args, _res) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.argtypes = _args
    _fn.restype = _res

EXPORTED = tuple(_SIGS)


class QcError(RuntimeError):
    def __init__(self, status, what):
        detail = lib.qc_hip_last_error().decode()
        super().__init__(f"{what}: {STATUS.get(status, status)}" + (f" ({detail})" if detail else ""))
        self.status = status


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is not None:
        return ctypes.c_void_p(stream)
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check(status, what):
    if status != 0:
        raise QcError(status, what)


def packed_size(fmt, n, k):
    size = ctypes.c_size_t(0)
    st = lib.qc_hip_qgemv_packed_size(fmt, n, k, ctypes.byref(size))
    return st, size.value


# Raw entry points: return the status integer (tests exercise error paths).
def qgemv_raw(fmt, packed, x, y, n, k, stream=None):
    return lib.qc_hip_qgemv(fmt, _ptr(packed), _ptr(x), _ptr(y), n, k, _stream(stream))


def qgemv_w8a8_raw(fmt, packed, x, y, n, k, dev_status=None, stream=None):
    return lib.qc_hip_qgemv_w8a8(fmt, _ptr(packed), _ptr(x), _ptr(y), n, k, _ptr(dev_status),
                                 _stream(stream))


def qgemv_up_gate_raw(fmt, p_up, p_gate, x, up, gate, n, k, stream=None):
    return lib.qc_hip_qgemv_up_gate(fmt, _ptr(p_up), _ptr(p_gate), _ptr(x), _ptr(up), _ptr(gate),
                                    n, k, _stream(stream))


def qgemv_up_gate_activation_raw(fmt, p_up, p_gate, x, out, n, k, gelu_tanh=True, stream=None):
    return lib.qc_hip_qgemv_up_gate_activation(fmt, _ptr(p_up), _ptr(p_gate), _ptr(x), _ptr(out),
                                               n, k, int(bool(gelu_tanh)), _stream(stream))


def qgemv_qkv_raw(fmt, pq, pk, pv, x, q, k_out, v_out, query_dim, kv_dim, input_dim, stream=None):
    return lib.qc_hip_qgemv_qkv(fmt, _ptr(pq), _ptr(pk), _ptr(pv), _ptr(x), _ptr(q), _ptr(k_out),
                                _ptr(v_out), query_dim, kv_dim, input_dim, _stream(stream))


def qgemv_qkv_rope_kv_raw(fmt, pq, pk, pv, x, cosine, sine, q, key_cache, value_cache,
                         query_heads, kv_heads, head_dim, input_dim, slots, max_position,
                         position, slot, stream=None):
    return lib.qc_hip_qgemv_qkv_rope_kv(fmt, _ptr(pq), _ptr(pk), _ptr(pv), _ptr(x), _ptr(cosine),
                                        _ptr(sine), _ptr(q), _ptr(key_cache), _ptr(value_cache),
                                        query_heads, kv_heads, head_dim, input_dim, slots,
                                        max_position, position, slot, _stream(stream))


class CInt8Weights(ctypes.Structure):
    """qc_cint8_weights (include/quixicore_hip.h)."""
    _fields_ = [("codes", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("zero_points", ctypes.c_void_p), ("rows", ctypes.c_longlong),
                ("cols", ctypes.c_longlong), ("groups", ctypes.c_longlong)]


STORAGE = {"f32": 0, "f16": 1, "bf16": 2}


def cint8_weights(codes, scales, zero_points, rows, cols, groups):
    """A qc_cint8_weights over device tensors; the caller keeps the tensors
    alive while the struct is in use (it holds raw pointers)."""
    return CInt8Weights(None if codes is None else codes.data_ptr(),
                        None if scales is None else scales.data_ptr(),
                        None if zero_points is None else zero_points.data_ptr(), rows, cols, groups)


def cint8_project_raw(mode, weights, x, x_type, m, ys, y_types, bias=None, activation=0,
                      rope_cos=None, rope_sin=None, head_dim=0, stream=None):
    """qc_hip_cint8_project: weights is a list of CInt8Weights, ys a list of
    output tensors (or None), types as STORAGE ids."""
    arr = (CInt8Weights * max(len(weights), 1))(*weights)
    yp = (ctypes.c_void_p * max(len(ys), 1))(*[None if y is None else y.data_ptr() for y in ys])
    yt = (ctypes.c_int * max(len(y_types), 1))(*y_types)
    return lib.qc_hip_cint8_project(mode, arr, len(weights), _ptr(x), x_type, m, yp, yt,
                                    _ptr(bias), activation, _ptr(rope_cos), _ptr(rope_sin),
                                    head_dim, _stream(stream))


def cint8_dequantize_raw(weights, out, group_index=None, stream=None):
    """qc_hip_cint8_dequantize: weights a CInt8Weights, out f32 [rows][cols]."""
    return lib.qc_hip_cint8_dequantize(ctypes.byref(weights), _ptr(group_index), _ptr(out),
                                       _stream(stream))


def cint8_quantized_gemm_raw(weights, activation, y, a_int_zero_points=None, stream=None):
    """qc_hip_cint8_quantized_gemm: weights / activation CInt8Weights, y f32 [m][n]."""
    return lib.qc_hip_cint8_quantized_gemm(ctypes.byref(weights), ctypes.byref(activation),
                                           _ptr(a_int_zero_points), _ptr(y), _stream(stream))


def storage_to_f32_raw(x, x_type, count, out, stream=None):
    """qc_hip_storage_to_f32: x of STORAGE type x_type, out f32 [count]."""
    return lib.qc_hip_storage_to_f32(_ptr(x), x_type, count, _ptr(out), _stream(stream))


def qgemm_raw(fmt, packed, x, y, m, n, k, stream=None):
    return lib.qc_hip_qgemm(fmt, _ptr(packed), _ptr(x), _ptr(y), m, n, k, _stream(stream))


def qgemm_noalloc_raw(fmt, packed, x, y, m, n, k, stream=None):
    return lib.qc_hip_qgemm_noalloc(fmt, _ptr(packed), _ptr(x), _ptr(y), m, n, k,
                                    _stream(stream))


def pack_raw(fmt, w, packed, n, k, dev_status=None, stream=None):
    return lib.qc_hip_qgemv_pack(fmt, _ptr(w), n, k, _ptr(packed), _ptr(dev_status),
                                 _stream(stream))


def unpack_raw(fmt, packed, w, n, k, stream=None):
    return lib.qc_hip_qgemv_unpack(fmt, _ptr(packed), n, k, _ptr(w), _stream(stream))


def quantize_int8_raw(x, codes, scales, rows, dim, group_size=0, dev_status=None, stream=None):
    return lib.qc_hip_quantize_int8(_ptr(x), _ptr(codes), _ptr(scales), rows, dim, group_size,
                                    _ptr(dev_status), _stream(stream))


def rms_norm_add_quant_int8_raw(x, residual, weight, codes, residual_out, scales, rows, hidden,
                                eps=1e-5, group_size=0, dev_status=None, stream=None):
    return lib.qc_hip_rms_norm_add_quant_int8(_ptr(x), _ptr(residual), _ptr(weight), _ptr(codes),
                                              _ptr(residual_out), _ptr(scales), rows, hidden, eps,
                                              group_size, _ptr(dev_status), _stream(stream))


def quantize_int8_asymmetric_raw(x, codes, scales, zero_points, rows, dim, dev_status=None,
                                 stream=None):
    return lib.qc_hip_quantize_int8_asymmetric(_ptr(x), _ptr(codes), _ptr(scales),
                                               _ptr(zero_points), rows, dim, _ptr(dev_status),
                                               _stream(stream))


def dequantize_int8_asymmetric_raw(codes, scales, zero_points, out, rows, dim, stream=None):
    return lib.qc_hip_dequantize_int8_asymmetric(_ptr(codes), _ptr(scales), _ptr(zero_points),
                                                 _ptr(out), rows, dim, _stream(stream))


def int8_gemm_raw(w, x, ws, as_, row_sum, zp, y, m, n, k, asymmetric=False, dev_status=None,
                  stream=None):
    return lib.qc_hip_int8_gemm(_ptr(w), _ptr(x), _ptr(ws), _ptr(as_), _ptr(row_sum), _ptr(zp),
                                _ptr(y), m, n, k, int(asymmetric), _ptr(dev_status),
                                _stream(stream))


def int8_gemm_i32_raw(w, x, acc, m, n, k, stream=None):
    return lib.qc_hip_int8_gemm_i32(_ptr(w), _ptr(x), _ptr(acc), m, n, k, _stream(stream))


# Tensor-level helpers (torch GPU tensors in, new tensors out).
def pack(fmt, w):
    import torch
    n, k = w.shape
    st, size = packed_size(fmt, n, k)
    _check(st, "qgemv_packed_size")
    out = torch.empty(size, dtype=torch.uint8, device=w.device)
    _check(pack_raw(fmt, w, out, n, k), "qgemv_pack")
    return out


def unpack(fmt, packed, n, k):
    import torch
    out = torch.empty((n, k), dtype=torch.float32, device=packed.device)
    _check(unpack_raw(fmt, packed, out, n, k), "qgemv_unpack")
    return out


def qgemv(fmt, packed, x, n, k, y=None):
    import torch
    if y is None:
        y = torch.empty(n, dtype=torch.float32, device=x.device)
    _check(qgemv_raw(fmt, packed, x, y, n, k), "qgemv")
    return y


def qgemv_w8a8(fmt, packed, x, n, k, y=None):
    import torch
    if y is None:
        y = torch.empty(n, dtype=torch.float32, device=x.device)
    _check(qgemv_w8a8_raw(fmt, packed, x, y, n, k), "qgemv_w8a8")
    return y


def qgemm(fmt, packed, x, n, k, y=None):
    import torch
    m = x.shape[0]
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    _check(qgemm_raw(fmt, packed, x, y, m, n, k), "qgemm")
    return y


def quantize_int8(x, group_size=0, dev_status=None):
    import torch
    rows, dim = x.shape
    g = dim if group_size == 0 else group_size
    codes = torch.empty((rows, dim), dtype=torch.int8, device=x.device)
    scales = torch.empty((rows, dim // g), dtype=torch.float32, device=x.device)
    _check(quantize_int8_raw(x, codes, scales, rows, dim, group_size, dev_status),
           "quantize_int8")
    return codes, scales


def int8_gemm(w, x, ws, as_, row_sum=None, zp=None, asymmetric=False, dev_status=None, y=None):
    import torch
    m, k = x.shape
    n = w.shape[0]
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    _check(int8_gemm_raw(w, x, ws, as_, row_sum, zp, y, m, n, k, asymmetric, dev_status),
           "int8_gemm")
    return y


def int8_gemm_i32(w, x):
    import torch
    m, k = x.shape
    n = w.shape[0]
    acc = torch.empty((m, n), dtype=torch.int32, device=x.device)
    _check(int8_gemm_i32_raw(w, x, acc, m, n, k), "int8_gemm_i32")
    return acc


def set_gemv_rows_per_wave(rows):
    _check(lib.qc_hip_set_gemv_rows_per_wave(rows), "set_gemv_rows_per_wave")


def set_qgemm_plan(waves=0, stages=0):
    """Small-batch GEMM work split: waves per workgroup (4/8) and K stages
    per workgroup (1/2/4/8/16); 0 = from the shape."""
    _check(lib.qc_hip_set_qgemm_plan(waves, stages), "set_qgemm_plan")


def set_qgemm_panel(mode=0):
    """qgemm route for M >= 2: 0 = 2-D GEMM for M >= 64, -1 = never,
    1 / 2 = always with one / two K ranges."""
    _check(lib.qc_hip_set_qgemm_panel(mode), "set_qgemm_panel")


def set_qgemm_rows(mode=0):
    """qgemm route for 2 <= M <= 8: 0 = by shape (exact-digit rows kernel for
    M = 2, and M <= 4 with N <= 8192, at K <= 4096), -1 = never (MFMA
    small-batch kernels), 1 = always."""
    _check(lib.qc_hip_set_qgemm_rows(mode), "set_qgemm_rows")


def set_cint8_dot(mode=0):
    """Canonical int8 projections: 0 = the row-plane route (int8 MFMA) for two
    or more activation rows (three, or five for groups of 32, with group
    scales), else the exact digit-dot kernels where they apply; 1 = never the
    row-plane route; -1 = always the f32 kernel."""
    _check(lib.qc_hip_set_cint8_dot(mode), "set_cint8_dot")


def set_qgemm_fold(mode=0):
    """Digit-layout small-batch GEMM: 0 = builds its own digits where it can
    (no prep launch), -1 = always runs the prep launch (same bits)."""
    _check(lib.qc_hip_set_qgemm_fold(mode), "set_qgemm_fold")


def set_norm_sequential_sum(on):
    """Replay the element-order sum of squares for every row of
    rms_norm_add_quant_int8 (results are identical either way)."""
    _check(lib.qc_hip_set_norm_sequential_sum(int(bool(on))), "set_norm_sequential_sum")


def rms_norm_add_quant_int8(x, residual, weight, eps=1e-5, group_size=0, dev_status=None):
    """Returns (codes, residual_out, scales)."""
    import torch
    rows, hidden = x.shape
    g = hidden if group_size == 0 else group_size
    codes = torch.empty((rows, hidden), dtype=torch.int8, device=x.device)
    resid = torch.empty((rows, hidden), dtype=torch.float32, device=x.device)
    scales = torch.empty((rows, hidden // g), dtype=torch.float32, device=x.device)
    _check(rms_norm_add_quant_int8_raw(x, residual, weight, codes, resid, scales, rows, hidden,
                                       eps, group_size, dev_status), "rms_norm_add_quant_int8")
    return codes, resid, scales


def quantize_int8_asymmetric(x, dev_status=None):
    """Returns (codes, scales, zero_points)."""
    import torch
    rows, dim = x.shape
    codes = torch.empty((rows, dim), dtype=torch.int8, device=x.device)
    scales = torch.empty(rows, dtype=torch.float32, device=x.device)
    zps = torch.empty(rows, dtype=torch.int32, device=x.device)
    _check(quantize_int8_asymmetric_raw(x, codes, scales, zps, rows, dim, dev_status),
           "quantize_int8_asymmetric")
    return codes, scales, zps


def set_int8_gemm_route(route):
    """0 = from the shape, 1 = full-line ring, 2 = 64-byte-step DMA,
    3 = register-staged, 4 = one thread per output."""
    _check(lib.qc_hip_set_int8_gemm_route(route), "set_int8_gemm_route")


def qgemv_variant(fmt):
    return lib.qc_hip_qgemv_variant(fmt).decode()


def qgemv_w8a8_variant(fmt):
    return lib.qc_hip_qgemv_w8a8_variant(fmt).decode()


def int8_gemm_variant():
    return lib.qc_hip_int8_gemm_variant().decode()


def version():
    return lib.qc_hip_version().decode()
