"""GPU: the reference-side binding of the C ABI (tests/cpp/
reference_binding.h), compiled into tests/cpp/reference_binding_check.cpp
and driven with host buffers, as the
reference's dispatch (src/dispatch/qgemv.cpp:337-365,
src/dispatch/int8_gemm.cpp:67-94) would call it after its own validation.

Checks: every output against the CPU oracle (bit for bit for quantize_int8
and int8_gemm, the 1e-4 normalised contract for qgemv / qgemm); the C ABI
status returned unchanged for every validation and data-dependent failure,
with the outputs left untouched; the variant override
(QUIXICORE_CPU_QGEMV_VARIANT=ref deselects the GPU route).
"""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "quixicore-cpu_amd", "lib", "reference_binding_check")
TOL = 1e-4


@pytest.fixture(scope="module")
def run(qc, oracle, synth, tmp_path_factory):
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is not built (make -C quixicore-cpu_amd)")
    d = tmp_path_factory.mktemp("binding")
    n, k, m = 300, 4096, 5
    w = synth.normal_fast(501, n * k, 0.02).reshape(n, k)
    ins = {}
    for fmt, name in ((1, "q4"), (0, "q8")):
        st, ins[name] = oracle.pack(fmt, w)
        assert st == 0
    ins["x"] = synth.normal_fast(502, m * k).reshape(m, k)
    ins["xq"] = synth.activations_outliers_fast(3, m, k)
    st, ins["w8"], ws = oracle.quantize_int8(synth.normal_fast(503, n * k, 0.02).reshape(n, k))
    ins["ws"] = ws[:, 0].copy()
    rng = np.random.default_rng(504)
    ins["x8"] = rng.integers(-128, 128, (m, k), dtype=np.int8)
    ins["x8"][0, :] = -128
    ins["as"] = rng.uniform(1e-3, 1e-1, m).astype(np.float32)
    ins["rs"] = ins["w8"].astype(np.int32).sum(axis=1).astype(np.int32)
    ins["zp"] = rng.integers(-128, 128, m).astype(np.int32)
    for name, a in ins.items():
        np.ascontiguousarray(a).tofile(d / f"{name}.bin")
    (d / "dims.txt").write_text(f"{n} {k} {m}\n")
    print(f"running reference_binding_check n={n} k={k} m={m}", flush=True)
    env = dict(os.environ)
    env.pop("QUIXICORE_CPU_QGEMV_VARIANT", None)
    subprocess.run([BINARY, str(d)], check=True, timeout=120, env=env)
    status = {}
    for line in (d / "status.txt").read_text().splitlines():
        name, value = line.split()
        status[name] = int(value)

    def out(name, dtype):
        return np.fromfile(d / f"{name}.bin", dtype=dtype)

    return ins, status, out, (n, k, m)


def test_variant_selection(run):
    _, status, _, _ = run
    assert status["available"] == 1
    assert status["selected_default"] == 1
    assert status["selected_ref"] == 0
    assert status["selected_named"] == 1


@pytest.mark.parametrize("fmt,name", [(0, "q8_0"), (1, "q4_0")])
def test_qgemv_qgemm_host_buffers(run, oracle, fmt, name):
    ins, status, out, (n, k, m) = run
    packed = ins["q8" if fmt == 0 else "q4"]
    assert status[f"{name}_qgemv"] == 0
    assert status[f"{name}_qgemm"] == 0
    y = out(f"{name}_qgemv", np.float32)
    y64, wn = oracle.gemv_f64(fmt, packed, ins["x"][0], n, k)
    ok, worst = oracle.within_contract(y, y64, wn, ins["x"][0], TOL)
    assert ok, worst
    Y = out(f"{name}_qgemm", np.float32).reshape(m, n)
    for r in range(m):
        y64, wn = oracle.gemv_f64(fmt, packed, ins["x"][r], n, k)
        ok, worst = oracle.within_contract(Y[r], y64, wn, ins["x"][r], TOL)
        assert ok, (r, worst)


def test_quantize_int8_host_buffers_bit_exact(run, oracle):
    ins, status, out, (n, k, m) = run
    assert status["quantize_rows"] == 0
    st, codes, scales = oracle.quantize_int8(ins["xq"])
    assert np.array_equal(out("quantize_codes", np.int8), codes.reshape(-1))
    assert np.array_equal(out("quantize_scales", np.uint32), scales.reshape(-1).view(np.uint32))
    assert status["quantize_groups"] == 0
    st, codes, scales = oracle.quantize_int8(ins["xq"], 128)
    assert np.array_equal(out("quantize_group_codes", np.int8), codes.reshape(-1))
    assert np.array_equal(out("quantize_group_scales", np.uint32),
                          scales.reshape(-1).view(np.uint32))


@pytest.mark.parametrize("asym", [False, True])
def test_int8_gemm_host_buffers_bit_exact(run, oracle, asym):
    ins, status, out, (n, k, m) = run
    assert status["int8_gemm_azp" if asym else "int8_gemm"] == 0
    st, want = oracle.int8_gemm(ins["w8"], ins["x8"], ins["ws"], ins["as"],
                                ins["rs"] if asym else None, ins["zp"] if asym else None, asym)
    assert st == 0
    got = out("int8_gemm_azp" if asym else "int8_gemm", np.uint32)
    assert np.array_equal(got, want.reshape(-1).view(np.uint32))


def test_statuses_unchanged_and_outputs_untouched(run):
    _, status, out, (n, k, m) = run
    # src/dispatch/qgemv.cpp:125-141,337-349 and kernels/quantization/qgemm_ref.cpp:141-150
    assert status["qgemv_bad_format"] == 2
    assert status["qgemv_bad_k"] == 1
    assert status["qgemv_null_x"] == 3
    assert status["qgemm_null_before_format"] == 3
    assert np.all(out("untouched_qgemv", np.float32) == 7.0)
    # kernels/quantization/quantization_ref.cpp:143-148: non-finite x, before any write
    assert status["quantize_nonfinite"] == 3
    assert np.all(out("untouched_codes", np.int8) == 5)
    assert np.all(out("untouched_scales", np.float32) == 7.0)
    assert status["quantize_bad_group"] == 1
    # src/dispatch/int8_gemm.cpp:72-85: shape, nulls, then finite scales
    assert status["int8_gemm_nan_scale"] == 3
    assert np.all(out("untouched_int8", np.float32) == 7.0)
    assert status["int8_gemm_asym_null"] == 3
    assert status["int8_gemm_bad_shape"] == 1
