"""GPU: the C++ drop-in API (include/quixicore_cpu/*.h) as a reference caller
uses it -- host buffers, synchronous calls, reference Status values -- through
tests/cpp/dropin_check.cpp (built by `make -C quixicore-cpu_amd`).  Its
outputs are checked against the CPU oracle: bit for bit where the GPU path is
bit-identical to the reference (packing, quantizers, int8 GEMMs, qgemv_w8a8,
rms_norm_add_quant_int8 with its partial writes), within the 1e-4 contract for
the f32 GEMV/GEMM family.
"""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "quixicore-cpu_amd", "lib", "dropin_check")
DTYPES = {"f32": np.float32, "u8": np.uint8, "i8": np.int8, "i32": np.int32}
TOL = 1e-4


@pytest.fixture(scope="module")
def run(qc, tmp_path_factory):
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is not built (make -C quixicore-cpu_amd)")
    out = tmp_path_factory.mktemp("dropin")
    print("running dropin_check", flush=True)
    subprocess.run([BINARY, str(out)], check=True, timeout=120)
    arrays, status = {}, {}
    for line in open(out / "manifest.txt"):
        name, kind, value = line.split()
        if kind == "status":
            status[name] = int(value)
        else:
            arrays[name] = np.fromfile(out / f"{name}.bin", dtype=DTYPES[kind])
            assert arrays[name].size == int(value)
    return arrays, status


def _bits_equal(a, b):
    """Same bytes (the program writes flat arrays; the oracle returns shaped ones)."""
    return np.array_equal(np.ascontiguousarray(a).reshape(-1).view(np.uint8),
                          np.ascontiguousarray(b).reshape(-1).view(np.uint8))


def _contract(oracle, fmt, packed, x, y, n, k):
    y64, wn = oracle.gemv_f64(fmt, packed, x, n, k)
    ok, worst = oracle.within_contract(y, y64, wn, x, TOL)
    assert ok, worst


def _act64(v, gelu):
    v = v.astype(np.float64)
    if gelu:
        return 0.5 * v * (1.0 + np.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))
    return v / (1.0 + np.exp(-v))


@pytest.mark.parametrize("fmt,p", [(0, "q8_0_"), (1, "q4_0_")])
def test_dropin_quantized_matmuls(run, oracle, fmt, p):
    a, st = run
    n, k, m = 96, 256, 5
    for name in ("packed_size", "pack", "pack2", "qgemv", "qgemm", "up_gate", "up_gate_gelu",
                 "up_gate_silu", "qkv", "w8a8", "prepare", "prepacked_m5", "prepacked_m70"):
        assert st[p + name] == 0, name
    # qgemv_prepacked is the storage route, which (as in the reference,
    # kernels/quantization/qgemm_canonical.cpp:4275-4291,4647-4653) takes only
    # canonical-layout weights
    assert st[p + "prepacked_gemv"] == 2
    w, w2, x = a[p + "w"].reshape(n, k), a[p + "w2"].reshape(n, k), a[p + "x"].reshape(m, k)
    packed, packed2 = a[p + "packed"], a[p + "packed2"]
    assert _bits_equal(packed, oracle.pack(fmt, w)[1])
    assert _bits_equal(packed2, oracle.pack(fmt, w2)[1])
    _contract(oracle, fmt, packed, x[0], a[p + "qgemv_y"], n, k)
    for name in ("qgemm_y", "prepacked_m5_y"):
        ym = a[p + name].reshape(m, n)
        for r in range(m):
            _contract(oracle, fmt, packed, x[r], ym[r], n, k)
    xl, yl = a[p + "xl"].reshape(70, k), a[p + "prepacked_m70_y"].reshape(70, n)
    for r in range(70):
        _contract(oracle, fmt, packed, xl[r], yl[r], n, k)
    up, gate = a[p + "up"], a[p + "gate"]
    _contract(oracle, fmt, packed, x[0], up, n, k)
    _contract(oracle, fmt, packed2, x[0], gate, n, k)
    for name, gelu in (("act_gelu", True), ("act_silu", False)):
        want = _act64(gate, gelu) * up.astype(np.float64)
        bound = 1e-5 * np.abs(gate.astype(np.float64) * up) + 2e-6 * np.abs(want) + 1e-30
        assert np.all(np.abs(a[p + name] - want) <= bound), name
    row = packed2.size // n
    _contract(oracle, fmt, packed, x[0], a[p + "qkv_q"], n, k)
    _contract(oracle, fmt, packed2[: row * (n // 2)], x[0], a[p + "qkv_k"], n // 2, k)
    _contract(oracle, fmt, packed2[row * (n // 2):], x[0], a[p + "qkv_v"], n // 2, k)
    # RoPE seam: the rotation of the plain projections, in f32; other slots kept
    assert st[p + "qkv_rope"] == 0 and st[p + "qkv_rope_badpos"] == 1
    hd, half, kvd = 16, 8, n // 2
    c, s_ = a[p + "rope_cos"][2 * half:3 * half], a[p + "rope_sin"][2 * half:3 * half]

    def rot(y, heads):
        v = y.reshape(heads, 2, half)
        return np.stack([v[:, 0] * c - v[:, 1] * s_, v[:, 1] * c + v[:, 0] * s_], 1).reshape(-1)

    assert _bits_equal(a[p + "rope_q"], rot(a[p + "qkv_q"], n // hd))
    kc, vc, kc0, vc0 = a[p + "rope_kc"], a[p + "rope_vc"], a[p + "rope_kc0"], a[p + "rope_vc0"]
    assert _bits_equal(kc[kvd:2 * kvd], rot(a[p + "qkv_k"], kvd // hd))
    assert _bits_equal(vc[kvd:2 * kvd], a[p + "qkv_v"])
    for sl in (slice(0, kvd), slice(2 * kvd, 3 * kvd)):
        assert _bits_equal(kc[sl], kc0[sl]) and _bits_equal(vc[sl], vc0[sl])
    st_w8, y_w8 = oracle.gemv_w8a8(fmt, packed, x[0], n, k)
    assert st_w8 == 0 and _bits_equal(a[p + "w8a8_y"], y_w8)


def test_dropin_validation(run):
    _, st = run
    assert st["bad_k"] == 1 and st["null_y"] == 3


def test_dropin_quantizers_and_int8_gemm(run, oracle):
    a, st = run
    x = a["quant_x"].reshape(4, 256)
    for g in (0, 32):
        p = f"quant_g{g}"
        ost, codes, scales = oracle.quantize_int8(x, g)
        assert st[p] == ost == 0
        assert _bits_equal(a[p + "_codes"], codes) and _bits_equal(a[p + "_scales"], scales)
    w, xi = a["i8_w"].reshape(7, 64), a["i8_x"].reshape(5, 64)
    ws, as_, rs, zp = a["i8_ws"], a["i8_as"], a["i8_rs"], a["i8_zp"]
    _, y = oracle.int8_gemm(w, xi, ws, as_)
    assert st["int8_gemm"] == 0 and _bits_equal(a["int8_gemm_y"], y)
    assert st["w8a8"] == 0 and _bits_equal(a["w8a8_y"], y)
    _, y = oracle.int8_gemm(w, xi, ws, as_, row_sum=rs, zp=zp, asymmetric=True)
    assert st["w8a8_azp"] == 0 and _bits_equal(a["w8a8_azp_y"], y)
    xa = a["asym_x"].reshape(3, 200)
    ost, c, s, z = oracle.quantize_int8_asymmetric(xa)
    assert st["asym"] == ost == 0
    assert _bits_equal(a["asym_codes"], c) and _bits_equal(a["asym_scales"], s)
    assert _bits_equal(a["asym_zps"], z)
    _, d = oracle.dequantize_int8_asymmetric(c, s, z)
    assert st["asym_deq"] == 0 and _bits_equal(a["asym_deq_y"], d)


def test_dropin_rms_norm_partial_writes(run, oracle):
    """kernels/norms/norm_quant_ref.cpp: a group with a non-finite normalized
    value keeps the caller's data; host callers see the same partial writes."""
    a, st = run
    x, r = a["norm_x"].reshape(3, 256), a["norm_r"].reshape(3, 256)
    for case, wname, group in (("norm_ok", "norm_w_ok", 32), ("norm_bad", "norm_w_bad", 32)):
        ost, codes, resid, scales = oracle.rms_norm_add_quant_int8(x, r, a[wname], 1e-5, group)
        assert st[case] == ost
        assert _bits_equal(a[case + "_codes"], codes)
        assert _bits_equal(a[case + "_resid"], resid)
        assert _bits_equal(a[case + "_scales"], scales)
    assert st["norm_bad"] == 3
    ost, codes, resid, scales = oracle.rms_norm_add_quant_int8(x, r, a["norm_w_inplace"], 1e-5, 0)
    assert st["norm_inplace"] == ost == 0
    assert _bits_equal(a["norm_inplace_codes"], codes)
    assert _bits_equal(a["norm_inplace_resid"], resid)
    assert _bits_equal(a["norm_inplace_scales"], scales)
