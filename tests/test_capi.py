"""CPU checks of the boundary: the library loads, exports every entry point
include/quixicore_hip.h declares, and rejects invalid calls in the
reference's validation order before touching the device (no GPU needed)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "quixicore_hip.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(qc_hip_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = declared()
    for required in ("qc_hip_qgemv", "qc_hip_qgemm", "qc_hip_quantize_int8", "qc_hip_int8_gemm",
                     "qc_hip_qgemm_w8a8", "qc_hip_qgemv_pack", "qc_hip_qgemv_packed_size"):
        assert required in names


def test_library_exports_every_declared_symbol():
    import quixicore_hip as q
    lib = ctypes.CDLL(q.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared()) == set(q.EXPORTED)


def test_cpp_dropin_symbols_exported():
    import subprocess
    import quixicore_hip as q
    out = subprocess.run(["nm", "-D", "-C", "--defined-only", q.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    for sym in ("quixicore_cpu::qgemv(", "quixicore_cpu::qgemm(", "quixicore_cpu::quantize_int8(",
                "quixicore_cpu::int8_gemm(", "quixicore_cpu::qgemm_w8a8(",
                "quixicore_cpu::qgemv_w8a8(", "quixicore_cpu::qgemv_w8a8_packed_size(",
                "quixicore_cpu::qgemm_prepacked(", "quixicore_cpu::CpuPackedWeights::prepare(",
                "quixicore_cpu::rms_norm_add_quant_int8(",
                "quixicore_cpu::quantize_int8_asymmetric(",
                "quixicore_cpu::dequantize_int8_asymmetric(",
                "quixicore_cpu::Workspace::allocate(", "quixicore_cpu::quantize_canonical(",
                "quixicore_cpu::dequantize_canonical("):
        assert sym in out, sym


def test_packed_size_and_validation_without_device():
    import quixicore_hip as q
    assert q.packed_size(0, 4, 64) == (0, 4 * 2 * 34)
    assert q.packed_size(1, 4, 64) == (0, 4 * 2 * 18)
    assert q.packed_size(0, 4, 4096) == (0, 4 * 128 * 34)
    assert q.packed_size(0, 4, 33)[0] == 1
    assert q.packed_size(0, 0, 32)[0] == 1
    assert q.packed_size(0, 1 << 62, 128)[0] == 1
    assert q.packed_size(3, 4, 64)[0] == 2
    assert q.lib.qc_hip_qgemv_packed_size(0, 1, 32, None) == 3
    # qgemv: format, shape, then nulls -- all before any launch
    assert q.lib.qc_hip_qgemv(7, None, None, None, 1, 32, None) == 2
    assert q.lib.qc_hip_qgemv(0, None, None, None, 4, 33, None) == 1
    assert q.lib.qc_hip_qgemv(0, None, None, None, 1, 32, None) == 3
    # qgemm: products, nulls, then format
    assert q.lib.qc_hip_qgemm(9, None, None, None, 0, 1, 32, None) == 1
    assert q.lib.qc_hip_qgemm(9, None, None, None, 1, 1, 32, None) == 3
    # quantize_int8: shape then nulls
    assert q.lib.qc_hip_quantize_int8(None, None, None, 2, 6, 4, None, None) == 1
    assert q.lib.qc_hip_quantize_int8(None, None, None, 2, 8, 4, None, None) == 3
    # int8_gemm: shape then nulls (asymmetric needs row sums and zero points)
    assert q.lib.qc_hip_int8_gemm(None, None, None, None, None, None, None, 0, 1, 1, 0, None,
                                  None) == 1
    assert q.lib.qc_hip_int8_gemm(None, None, None, None, None, None, None, 1, 1, 1, 0, None,
                                  None) == 3
    assert q.lib.qc_hip_int8_gemm_i32(None, None, None, 1, 1, 131072, None) == 1
    # fused projections (kernels/quantization/qgemv_fused_ref.cpp:194-327):
    # shape products, nulls, then the packed layout (format, K)
    L = q.lib
    assert L.qc_hip_qgemv_up_gate(1, None, None, None, None, None, 0, 64, None) == 1
    assert L.qc_hip_qgemv_up_gate(9, None, None, None, None, None, 4, 64, None) == 3
    assert L.qc_hip_qgemv_up_gate_activation(1, None, None, None, None, 4, -1, 1, None) == 1
    assert L.qc_hip_qgemv_qkv(1, None, None, None, None, None, None, None, 4, 0, 64, None) == 1
    assert L.qc_hip_qgemv_qkv(1, None, None, None, None, None, None, None,
                              2, (1 << 62), 1, None) == 1
    assert L.qc_hip_qgemv_qkv(1, None, None, None, None, None, None, None, 4, 4, 64, None) == 3
    # qgemv_w8a8 (src/dispatch/qgemv_w8a8.cpp:99-105,130-143): format, shape, nulls
    assert q.lib.qc_hip_qgemv_w8a8(7, None, None, None, 1, 32, None, None) == 2
    assert q.lib.qc_hip_qgemv_w8a8(7, None, None, None, 1, 33, None, None) == 2
    assert q.lib.qc_hip_qgemv_w8a8(1, None, None, None, 96, 257, None, None) == 1
    assert q.lib.qc_hip_qgemv_w8a8(1, None, None, None, 96, 256, None, None) == 3
    nbytes = ctypes.c_longlong(0)
    assert q.lib.qc_hip_qgemv_w8a8_packed_size(1, 96, 256, ctypes.byref(nbytes)) == 0
    assert nbytes.value == 96 * 8 * 18
    assert q.lib.qc_hip_qgemv_w8a8_packed_size(0, 96, 256, None) == 3
    assert q.lib.qc_hip_qgemv_w8a8_packed_size(2, 96, 256, ctypes.byref(nbytes)) == 2
    assert q.qgemv_w8a8_variant(1) == "hip_gfx950_w8a8_q4_0"
    assert q.qgemv_w8a8_variant(3) == "unsupported"
    assert q.qgemv_variant(0) == "hip_gfx950_q8_0" and q.qgemv_variant(5) == "unsupported"
    assert q.lib.qc_hip_set_gemv_rows_per_wave(3) == 3
    # rms_norm_add_quant_int8 (kernels/norms/norm_quant_ref.cpp:106-130): rows x
    # hidden, finite eps >= 0, group dividing hidden, then nulls
    for rows, hidden, eps, group in ((0, 8, 1e-5, 0), (2, 8, float("nan"), 0), (2, 8, -1.0, 0),
                                     (2, 8, float("inf"), 0), (2, 8, 1e-5, 3),
                                     (2, 8, 1e-5, -8)):
        assert L.qc_hip_rms_norm_add_quant_int8(None, None, None, None, None, None, rows, hidden,
                                                eps, group, None, None) == 1
    assert L.qc_hip_rms_norm_add_quant_int8(None, None, None, None, None, None, 2, 8, 0.0, 4,
                                            None, None) == 3
    # quantize / dequantize_int8_asymmetric (quantization_ref.cpp:190-197,228-235)
    assert L.qc_hip_quantize_int8_asymmetric(None, None, None, None, 0, 8, None, None) == 1
    assert L.qc_hip_quantize_int8_asymmetric(None, None, None, None, 2, 8, None, None) == 3
    assert L.qc_hip_dequantize_int8_asymmetric(None, None, None, None, 2, -1, None) == 1
    assert L.qc_hip_dequantize_int8_asymmetric(None, None, None, None, 2, 8, None) == 3


def test_product_does_not_reference_oracle():
    """The shipped library and binding never load or name the CPU oracle."""
    import quixicore_hip as q
    blob = open(q.LIB_PATH, "rb").read()
    assert b"liboracle" not in blob and b"qco_" not in blob and b"qcref_" not in blob
    pkg = os.path.join(ROOT, "quixicore-cpu_amd")
    needles = ("liboracle", "qco_", "qcref_", "import oracle", "oracle/", "oracle.py",
               "_ref/libqcref")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h", ".c", "Makefile")):
                text = open(os.path.join(dirpath, f)).read()
                for needle in needles:
                    assert needle not in text, (f, needle)


def test_integration_binding_is_the_compiled_one():
    """The reference-side binding printed in INTEGRATION.md is the text of
    tests/cpp/reference_binding.h, which reference_binding_check compiles
    and tests/test_gpu_reference_binding.py runs: the document cannot drift
    from the code that is tested."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    header = open(os.path.join(root, "tests", "cpp", "reference_binding.h")).read()
    doc = open(os.path.join(root, "INTEGRATION.md")).read()
    assert "```cpp\n" + header + "```\n" in doc
