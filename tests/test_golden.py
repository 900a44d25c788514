"""CPU: the committed fixtures of tests/golden (written by
tests/golden/make_fixtures.py).

* The seeded synthetic streams that the GPU tests use at the BASELINE
  configs' full sizes hash to the committed SHA-256 values.
* The oracle reproduces, bit for bit, the outputs the reference's own
  compiled functions gave on the small golden inputs: q8_0 / q4_0 packing
  (including an all-zero block and an fp16-subnormal scale), the x86 GEMV
  routes (q8_0_gemv_ref, gguf_gemv_avx2's q4_rows, q4_0_gemv_ref), qgemm,
  quantize_int8 (per row and per 32-group) and the dispatched int8_gemm with
  and without the zero-point correction.  These hold without oracle/_ref.
"""
import hashlib
import json
import os

import numpy as np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden():
    return np.load(os.path.join(HERE, "reference_vectors.npz"), allow_pickle=False)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


def test_synthetic_streams_match_committed_hashes():
    import sys
    sys.path.insert(0, HERE)
    from make_fixtures import streams
    want = json.load(open(os.path.join(HERE, "synthetic_sha256.json")))
    got = {name: a for name, a in streams()}
    assert set(got) == set(want)
    for name, a in got.items():
        assert list(a.shape) == want[name]["shape"], name
        assert str(a.dtype) == want[name]["dtype"], name
        assert hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest() == \
            want[name]["sha256"], name


def test_oracle_pack_and_gemv_match_reference_vectors(oracle):
    g = _golden()
    w, x = g["w"], g["x"]
    n, k = w.shape
    for fmt, name in ((oracle.Q8_0, "q8_0"), (oracle.Q4_0, "q4_0")):
        st, packed = oracle.pack(fmt, w)
        assert st == 0
        assert np.array_equal(packed, g[f"{name}_packed"]), name
        y = oracle.gemv(fmt, packed, x[0], n, k)
        assert np.array_equal(_bits(y), _bits(g[f"{name}_gemv"])), name
        rows = np.stack([oracle.gemv(fmt, packed, x[r], n, k) for r in range(x.shape[0])])
        assert np.array_equal(_bits(rows), _bits(g[f"{name}_qgemm"])), name
    y = oracle.gemv(oracle.Q4_0, g["q4_0_packed"], x[0], n, k, order="portable")
    assert np.array_equal(_bits(y), _bits(g["q4_0_gemv_portable"]))
    # the all-zero q4_0 block keeps the reference's -0 scale (fp16 0x8000)
    assert g["q4_0_packed"][0] == 0x00 and g["q4_0_packed"][1] == 0x80


def test_oracle_quantize_int8_matches_reference_vectors(oracle):
    g = _golden()
    st, codes, scales = oracle.quantize_int8(g["qi8_x"])
    assert st == 0
    assert np.array_equal(codes, g["qi8_codes"])
    assert np.array_equal(_bits(scales), _bits(g["qi8_scales"]))
    st, codes, scales = oracle.quantize_int8(g["qi8_x"], group_size=32)
    assert st == 0
    assert np.array_equal(codes, g["qi8_group32_codes"])
    assert np.array_equal(_bits(scales), _bits(g["qi8_group32_scales"]))
    assert not np.any(g["qi8_codes"][2]) and g["qi8_scales"][2, 0] == 0.0


def test_oracle_int8_gemm_matches_reference_vectors(oracle):
    g = _golden()
    st, y = oracle.int8_gemm(g["i8_w"], g["i8_x"], g["i8_ws"], g["i8_as"])
    assert st == 0
    assert np.array_equal(_bits(y), _bits(g["i8_y"]))
    st, y = oracle.int8_gemm(g["i8_w"], g["i8_x"], g["i8_ws"], g["i8_as"], g["i8_rs"],
                             g["i8_zp"], True)
    assert st == 0
    assert np.array_equal(_bits(y), _bits(g["i8_y_azp"]))
