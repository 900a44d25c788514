"""GPU: quantize_canonical / dequantize_canonical for the canonical int8
layouts (include/quixicore_cpu/quant_import.h:42-45,53-54;
kernels/quantization/quant_import_ref.cpp:552-681,717-838).

* The scenario list of tests/cpp/canonical_quant_scenarios.h runs through this
  library's C++ drop-in (quixicore-cpu_amd/lib/canonical_quant_check, host
  buffers) and through the reference's own functions (oracle/_ref).  Every
  status must be equal, and every int8 tensor table (codes, scales, zero
  points, metadata) and decoded output byte-identical.  For the layouts this
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
        assert d_ours[name] == d_ref[name], name
    # the int8 round trips did run and produced data
    assert len(d_ref["sym_row_f32_codes"]) == 48 * 256
    assert len(d_ref["aff_row_f16_zeros"]) == 48 * 4


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
