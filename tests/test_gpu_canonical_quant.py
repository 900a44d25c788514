"""GPU: quantize_canonical / dequantize_canonical for the canonical int8
layouts (include/quixicore_cpu/quant_import.h:42-45,53-54;
kernels/quantization/quant_import_ref.cpp:552-681,717-838), and the
canonical W8A8 projections qgemm_prepacked_quantized /
qgemv_prepacked_quantized over them (include/quixicore_cpu/qgemm.h:118-127;
kernels/quantization/qgemm_canonical.cpp:5415-5507).

* The scenario list of tests/cpp/canonical_quant_scenarios.h runs through this
  library's C++ drop-in (quixicore-cpu_amd/lib/canonical_quant_check, host
  buffers) and through the reference's own functions (oracle/_ref).  Every
  status must be equal, and every int8 tensor table (codes, scales, zero
  points, metadata) and decoded output byte-identical; the projections of
  every int8 weight x activation pair meet the 1e-4 normalised contract
  against the f64 product of the decoded operands.  For the layouts this
  GPU path does not compute ("other_" scenarios), the reference's validation
  failures must be the same and where the reference computes, this library
  returns kUnsupportedFormat (2).
* The C ABI beneath them: qc_hip_cint8_dequantize against the oracle's
  restatement of the decode, bit for bit, for symmetric / affine, row and
  group scales, fractional zero points; qc_hip_storage_to_f32 exact for
  f16 / bf16 bit patterns; and both entries' validation statuses.
"""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "quixicore-cpu_amd", "lib", "canonical_quant_check")


def _manifest(directory):
    status, data = {}, {}
    for line in open(os.path.join(directory, "manifest.txt")):
        name, kind, value = line.split()
        if kind == "status":
            status[name] = int(value)
        else:
            data[name] = open(os.path.join(directory, name + ".bin"), "rb").read()
            assert len(data[name]) == int(value)
    return status, data


def test_canonical_quant_scenarios_match_reference(qc, ref, tmp_path):
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is not built (make -C quixicore-cpu_amd)")
    ours, theirs = tmp_path / "ours", tmp_path / "reference"
    ours.mkdir()
    theirs.mkdir()
    print("running canonical_quant_check", flush=True)
    subprocess.run([BINARY, str(ours)], check=True, timeout=120)
    assert ref.canonical_quant_scenarios(str(theirs)) == 0
    s_ours, d_ours = _manifest(ours)
    s_ref, d_ref = _manifest(theirs)
    assert set(s_ours) == set(s_ref)
    assert set(d_ours) == set(d_ref)
    for name, want in s_ref.items():
        got = s_ours[name]
        if name.startswith("other_") and want == 0:
            assert got == 2, (name, got)     # computed by the reference's CPU code only
        else:
            assert got == want, (name, got, want)
    computed = [n for n, v in s_ref.items() if v == 0 and not n.startswith("other_")]
    assert len(computed) >= 16
    for name in d_ref:
        if name.startswith("proj_") and name.endswith("_y"):
            continue                      # f32 sums: checked against the contract below
        assert d_ours[name] == d_ref[name], name
    # the int8 round trips did run and produced data
    assert len(d_ref["sym_row_f32_codes"]) == 48 * 256
    assert len(d_ref["aff_row_f16_zeros"]) == 48 * 4
    # qgemm_prepacked_quantized / qgemv_prepacked_quantized: both libraries'
    # outputs against the f64 product of the decoded operands (byte-identical
    # in both runs, checked above), |y - y64| <= 1e-4 * ||a_row|| * ||w_row||
    n, k, m = 96, 512, 5
    f32 = lambda name: np.frombuffer(d_ours[name], dtype=np.float32)   # noqa: E731
    pairs = 0
    for wname in ("wsym", "wsymg", "waff"):
        w = f32(f"proj_{wname}_dequant").reshape(n, k).astype(np.float64)
        wn = np.linalg.norm(w, axis=1)
        for aname in ("asym", "asymg", "aaff"):
            a = f32(f"proj_{aname}_dequant").reshape(m, k).astype(np.float64)
            y64 = a @ w.T
            bound = 1e-4 * np.linalg.norm(a, axis=1)[:, None] * wn[None, :]
            for d in (d_ours, d_ref):
                y = np.frombuffer(d[f"proj_{wname}_{aname}_y"], dtype=np.float32).reshape(m, n)
                assert np.all(np.abs(y - y64) <= bound), (wname, aname, d is d_ours)
            if wname == "wsym":
                y = np.frombuffer(d_ours[f"proj_gemv_{aname}_y"], dtype=np.float32)
                assert np.all(np.abs(y - y64[0]) <= bound[0]), ("gemv", aname)
            pairs += 1
    assert pairs == 9
    assert np.all(np.frombuffer(d_ours["proj_untouched"], dtype=np.float32) == 7.0)


@pytest.mark.parametrize("affine,groups,fractional", [(False, 1, False), (False, 8, False),
                                                       (True, 1, False), (True, 32, False),
                                                       (True, 4, True)])
def test_cint8_dequantize_bit_exact(qc, oracle, dev, affine, groups, fractional):
    """out = scale * (code - zero), each step rounded in f32, against the
    oracle's restatement of the reference's decode (oracle.cint8_dequant)."""
    import torch
    rows, cols = 300, 1024
    rng = np.random.default_rng(groups + 10 * affine)
    codes = rng.integers(-128, 128, (rows, cols), dtype=np.int8)
    scales = (rng.random(rows * groups, dtype=np.float32) * 1e-2 + 1e-6).astype(np.float32)
    zeros = None
    if affine:
        zeros = rng.integers(-128, 128, rows * groups).astype(np.float32)
        if fractional:
            zeros = (zeros + rng.random(rows * groups, dtype=np.float32)).astype(np.float32)
    C = torch.from_numpy(codes).to(dev)
    S = torch.from_numpy(scales).to(dev)
    Z = None if zeros is None else torch.from_numpy(zeros).to(dev)
    w = qc.cint8_weights(C, S, Z, rows, cols, groups)
    out = torch.full((rows, cols), 7.0, device=dev)
    print(f"cint8_dequantize affine={affine} groups={groups} fractional={fractional}", flush=True)
    assert qc.cint8_dequantize_raw(w, out) == 0
    want = oracle.cint8_dequant(codes, scales, zeros, rows, cols, groups)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_storage_to_f32_exact(qc, dev):
    import torch
    rng = np.random.default_rng(1616)
    bits = rng.integers(0, 1 << 16, 1 << 16, dtype=np.uint32).astype(np.uint16)
    bits[:1 << 10] = np.arange(1 << 10, dtype=np.uint16)          # subnormals and zero
    bits[-4:] = [0x7c00, 0xfc00, 0x7e00, 0x8000]                   # inf, -inf, nan, -0
    X = torch.from_numpy(bits.view(np.int16).copy()).to(dev)
    out = torch.empty(bits.size, device=dev)
    assert qc.storage_to_f32_raw(X, 1, bits.size, out) == 0
    want = bits.view(np.float16).astype(np.float32)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32)[~np.isnan(want)],
                          want.view(np.uint32)[~np.isnan(want)])
    assert np.isnan(got[np.isnan(want)]).all()
    assert qc.storage_to_f32_raw(X, 2, bits.size, out) == 0
    want = (bits.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_new_entry_validation(qc, dev):
    import torch
    t = torch.zeros(64, device=dev)
    c = torch.zeros(64, dtype=torch.int8, device=dev)
    assert qc.storage_to_f32_raw(t, 1, 0, t) == 1
    assert qc.storage_to_f32_raw(t, 5, 16, t) == 2
    assert qc.storage_to_f32_raw(None, 1, 16, t) == 3
    ok = qc.cint8_weights(c, t, None, 8, 8, 2)
    assert qc.cint8_dequantize_raw(qc.cint8_weights(c, t, None, 0, 8, 1), t) == 1
    assert qc.cint8_dequantize_raw(qc.cint8_weights(c, t, None, 8, 8, 3), t) == 1
    assert qc.cint8_dequantize_raw(qc.cint8_weights(c, None, None, 8, 8, 1), t) == 3
    assert qc.cint8_dequantize_raw(ok, None) == 3
    assert qc.cint8_dequantize_raw(ok, t) == 0


@pytest.mark.parametrize("m,n,k,affine", [(512, 4096, 4096, False), (512, 4096, 4096, True),
                                          (1, 14336, 4096, False), (70, 300, 1024, True)])
def test_quantized_gemm_mfma_route_is_int8_gemm(qc, oracle, synth, dev, m, n, k, affine):
    """Symmetric row-scaled weights x row-scaled activations (no zero points,
    or integer ones): qc_hip_cint8_quantized_gemm gives exactly int8_gemm's
    bits on the same codes and scales (the AZP form with the weights' row
    sums for affine activations), which the int8 GEMM tests pin bit for bit
    against the reference."""
    import torch
    print(f"cint8 quantized gemm mfma m={m} n={n} k={k} affine={affine}", flush=True)
    st, wq, ws = oracle.quantize_int8(synth.normal_fast(71 + n, n * k, 0.02).reshape(n, k))
    x = synth.activations_outliers_fast(3, m, k)
    W, WS = torch.from_numpy(wq).to(dev), torch.from_numpy(ws[:, 0].copy()).to(dev)
    if affine:
        codes, scales, zps = qc.quantize_int8_asymmetric(torch.from_numpy(x).to(dev))
        zf = zps.float()
    else:
        codes, scales = qc.quantize_int8(torch.from_numpy(x).to(dev))
        scales = scales[:, 0].contiguous()
        zps, zf = None, None
    w = qc.cint8_weights(W, WS, None, n, k, 1)
    a = qc.cint8_weights(codes, scales, zf, m, k, 1)
    y = torch.full((m, n), 7.0, device=dev)
    assert qc.cint8_quantized_gemm_raw(w, a, y, zps) == 0
    rs = W.to(torch.int32).sum(dim=1).to(torch.int32) if affine else None
    want = qc.int8_gemm(W, codes, WS, scales, rs, zps, affine)
    assert torch.equal(y.view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("wgroups,waffine,agroups,aaffine,int_zeros",
                         [(8, False, 1, False, False), (1, True, 1, False, False),
                          (1, False, 4, True, False), (1, False, 1, True, False),
                          (16, True, 2, True, False)])
def test_quantized_gemm_generic_route(qc, oracle, dev, wgroups, waffine, agroups, aaffine,
                                      int_zeros):
    """Group scales, affine weights or activation zero points given only as
    floats: the f32 decode-and-FMA kernel, against the f64 product of the
    exactly decoded operands within the 1e-4 normalised contract."""
    import torch
    m, n, k = 9, 700, 2048
    print(f"cint8 quantized gemm generic wg={wgroups} wa={waffine} ag={agroups} aa={aaffine}",
          flush=True)
    rng = np.random.default_rng(wgroups * 7 + agroups)
    wc = rng.integers(-128, 128, (n, k), dtype=np.int8)
    ac = rng.integers(-128, 128, (m, k), dtype=np.int8)
    wsc = (rng.random(n * wgroups, dtype=np.float32) * 1e-2 + 1e-5).astype(np.float32)
    asc = (rng.random(m * agroups, dtype=np.float32) * 1e-1 + 1e-4).astype(np.float32)
    wz = rng.integers(-20, 21, n * wgroups).astype(np.float32) if waffine else None
    az = rng.integers(-20, 21, m * agroups).astype(np.float32) if aaffine else None
    T = lambda a: None if a is None else torch.from_numpy(a).to(dev)   # noqa: E731
    keep = [T(wc), T(wsc), T(wz), T(ac), T(asc), T(az)]
    w = qc.cint8_weights(keep[0], keep[1], keep[2], n, k, wgroups)
    a = qc.cint8_weights(keep[3], keep[4], keep[5], m, k, agroups)
    y = torch.full((m, n), 7.0, device=dev)
    assert qc.cint8_quantized_gemm_raw(w, a, y) == 0
    wh = oracle.cint8_dequant(wc, wsc, wz, n, k, wgroups).astype(np.float64)
    ah = oracle.cint8_dequant(ac, asc, az, m, k, agroups).astype(np.float64)
    y64 = ah @ wh.T
    bound = 1e-4 * np.linalg.norm(ah, axis=1)[:, None] * np.linalg.norm(wh, axis=1)[None, :]
    assert np.all(np.abs(y.cpu().numpy() - y64) <= bound)


def test_quantized_gemm_validation(qc, dev):
    import torch
    t = torch.zeros(64, device=dev)
    c = torch.zeros(64, dtype=torch.int8, device=dev)
    w = qc.cint8_weights(c, t, None, 8, 8, 1)
    assert qc.cint8_quantized_gemm_raw(w, qc.cint8_weights(c, t, None, 2, 16, 1), t) == 1
    assert qc.cint8_quantized_gemm_raw(w, qc.cint8_weights(c, t, None, 0, 8, 1), t) == 1
    assert qc.cint8_quantized_gemm_raw(w, qc.cint8_weights(c, t, None, 2, 8, 3), t) == 1
    assert qc.cint8_quantized_gemm_raw(w, qc.cint8_weights(None, t, None, 2, 8, 1), t) == 3
    assert qc.cint8_quantized_gemm_raw(w, qc.cint8_weights(c, t, None, 2, 8, 1), None) == 3
