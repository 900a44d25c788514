"""Pins the CPU oracle (oracle/qc_oracle.c) before anything is checked against it.

Each oracle function is checked against at least one thing a plausible
mistake would break:
  * fp16 codec       -- exhaustive against numpy's IEEE float16 conversions and
                        the reference's known answers (tests/correctness/
                        test_qgemv.cpp:79-97).
  * q8_0/q4_0 pack   -- byte-identical to the reference's own packers compiled
                        from source (oracle/_ref), on random data and on the
                        edge cases the reference tests (subnormal scale, zero
                        block, non-finite rejection, rounding ties), and to the
                        committed golden fixtures.
  * unpack           -- exact products d*q checked against numpy.
  * f32 GEMV orders  -- bit-identical to the reference's q8_0_gemv_ref, the
                        AVX2 q4_rows route and the portable q4_0 kernel.
  * f64 contract     -- against numpy float64 matmul of the unpacked weights.
  * quantize_int8    -- bit-identical to the reference's quantize_int8 and its
                        known answer (test_quantization.cpp:100-111).
  * qgemv_w8a8       -- bit-identical to the reference's q4_0/q8_0
                        gemv_w8a8_ref (oracle/_ref); the reference test's own
                        xorshift case within its tight f64 oracle
                        (test_qgemv_w8a8.cpp:57-116); a numpy float32
                        restatement of the per-block order; the codes equal
                        quantize_int8 with 32-element groups; validation order
                        (test_qgemv_w8a8.cpp:126-134).
  * int8 GEMM        -- bit-identical to the reference's dispatched int8_gemm
                        over its own test grid (test_int8_gemm.cpp:106-116),
                        numpy int64 matmul, and the known answers
                        {0, -1.5} / AZP {-5, -2} (test_projection_ops.cpp:81-97).
  * rms_norm_add_quant_int8 -- bit-identical to the reference's function
                        (oracle/_ref) over random shapes, groups, eps, scales
                        spanning 60 decades, invalid groups (overflowing or
                        non-finite weights, NaN inputs) and every validation
                        case; the reference test's own known answer
                        (test_remaining_ops.cpp:197-215), its codes worked by
                        hand; residual_out = x + residual exactly; per group
                        max |code| = 127 and codes within half a step of the
                        float64 normalized values.
  * qgemv_qkv_rope_kv -- bit-identical to the reference's function (oracle/_ref)
                        on random q8_0/q4_0 shapes, positions and slots
                        (slot -1 included) with the caches' other slots left
                        as they were, and on every validation case; the
                        reference test's known answer (test_remaining_ops.cpp:
                        217-257: a 90-degree rotation gives (-q1, q0) exactly);
                        at a zero angle the outputs are the plain row orders'
                        GEMV outputs bit for bit; each rotated pair keeps its
                        f64 norm.
  * canonical int8 projections (cint8_dequant / cint8_project_f64) -- the
                        reference's own prepared storage projections
                        (qgemm_prepacked_*_storage, oracle/_ref) over every
                        scenario of tests/cpp/storage_scenarios.h (symmetric
                        and affine, channel and group scales, f32/f16/bf16,
                        bias + every activation, gate/up, SwiGLU, Q/K/V,
                        RoPE with cache slots) stay within the normalised
                        contract of the f64 restatement; a hand-worked case.
  * quantize_int8_asymmetric / dequantize -- bit-identical to the reference's
                        functions on random rows and on the out-of-range
                        conversions (1-ulp spreads); the reference test's
                        known answers (test_quantization.cpp:113-136), both
                        rows worked by hand; round trip within half a step.
"""
import math

import numpy as np
import pytest

from conftest import xorshift32_unit


# ------------------------------------------------------------------ fp16 ---

def test_fp16_decode_exhaustive(oracle):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([oracle.fp16_to_fp32(int(c)) for c in codes], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))


def test_fp16_encode_matches_ieee(oracle):
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e-3),
        (rng.standard_normal(20000) * 1e4).astype(np.float32),
        np.ldexp(rng.uniform(1, 2, 20000), rng.integers(-30, 17, 20000)).astype(np.float32),
        # halfway points between adjacent halves (ties to even)
        ((np.arange(0, 4096, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -24)),
        np.array([65504, 65519.996, 65520, 65536, 1e30, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                  -0.0, 0.0, np.inf, -np.inf], dtype=np.float32),
    ]).astype(np.float32)
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.fp32_to_fp16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)
    assert oracle.fp32_to_fp16(float("nan")) == 0x7E00


def test_fp16_reference_known_answers(oracle):
    # tests/correctness/test_qgemv.cpp:79-97
    rt = lambda v: oracle.fp16_to_fp32(oracle.fp32_to_fp16(v))
    assert rt(1.0) == 1.0 and rt(0.5) == 0.5 and rt(0.0) == 0.0 and rt(65504.0) == 65504.0
    assert oracle.fp32_to_fp16(math.ldexp(1.0, -14)) == 0x0400
    assert oracle.fp32_to_fp16(math.ldexp(1.0, -15)) == 0x0200
    assert oracle.fp32_to_fp16(math.ldexp(1.0, -24)) == 0x0001
    assert oracle.fp32_to_fp16(math.ldexp(1.0, -25)) == 0x0000
    assert oracle.fp32_to_fp16(-math.ldexp(1.0, -24)) == 0x8001
    v = np.float32(0.0123456)
    assert abs(rt(float(v)) - v) / v < 1e-3


# ------------------------------------------------------------------ pack ---

def _edge_weights(k=32):
    rows = [
        np.full(k, 1e-3, np.float32),                     # fp16-subnormal scale
        np.zeros(k, np.float32),                          # all-zero block
        np.linspace(-1, 1, k, dtype=np.float32),
        np.where(np.arange(k) % 2 == 0, 1.0, -1.0).astype(np.float32),
        (np.arange(k, dtype=np.float32) - 16) * np.float32(0.5),  # many ties
        np.full(k, -7.25, np.float32),
        np.array([3.0e38] + [1.0] * (k - 1), np.float32),        # scale overflows fp16
    ]
    return np.stack(rows)


@pytest.mark.parametrize("fmt", [0, 1])
def test_pack_matches_reference(oracle, ref, fmt):
    for seed, (n, k) in enumerate([(1, 32), (3, 64), (5, 96), (33, 512), (17, 4096)]):
        w = (np.random.default_rng(seed).standard_normal((n, k)) * 0.02).astype(np.float32)
        st, got = oracle.pack(fmt, w)
        rst, want = ref.pack(fmt, w)
        assert st == 0 and rst == 0
        assert np.array_equal(got, want), (fmt, n, k)
    w = _edge_weights()
    st, got = oracle.pack(fmt, w)
    rst, want = ref.pack(fmt, w)
    assert st == 0 and rst == 0 and np.array_equal(got, want)


def test_pack_reference_edge_cases(oracle):
    # sizes: 34 / 18 bytes per 32 weights (test_qgemv.cpp:116-122)
    assert oracle.packed_size(0, 4, 64) == (0, 4 * 2 * 34)
    assert oracle.packed_size(1, 4, 64) == (0, 4 * 2 * 18)
    assert oracle.packed_size(0, 4, 33)[0] == 1
    assert oracle.packed_size(0, 0, 32)[0] == 1
    assert oracle.packed_size(0, 1 << 62, 128)[0] == 1
    assert oracle.packed_size(5, 4, 64)[0] == 2
    # non-finite rejection (test_qgemv.cpp:124-140)
    for fmt in (0, 1):
        for bad in (np.nan, np.inf):
            w = np.ones((1, 32), np.float32)
            w[0, 7] = bad
            assert oracle.pack(fmt, w)[0] == 3
    # subnormal fp16 scale keeps the block (test_qgemv.cpp:199-216)
    st, p = oracle.pack(0, np.full((1, 32), 1e-3, np.float32))
    dq = oracle.unpack(0, p, 1, 32)
    assert dq[0, 0] != 0 and abs(dq[0, 0] - 1e-3) < 1e-5
    # all-zero q4_0 block: d = -0.0 (0x8000) and every nibble 8
    st, p = oracle.pack(1, np.zeros((1, 32), np.float32))
    assert p[0] == 0x00 and p[1] == 0x80 and np.all(p[2:] == 0x88)


@pytest.mark.parametrize("fmt", [0, 1])
def test_unpack_is_exact_product(oracle, fmt):
    w = (np.random.default_rng(3).standard_normal((7, 128)) * 0.02).astype(np.float32)
    st, p = oracle.pack(fmt, w)
    blocks = p.reshape(7, 4, 34 if fmt == 0 else 18)
    d = blocks[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float64)
    if fmt == 0:
        q = blocks[:, :, 2:].view(np.int8).astype(np.float64)
    else:
        b = blocks[:, :, 2:].astype(np.int64)
        q = np.concatenate([(b & 15) - 8, (b >> 4) - 8], axis=2).astype(np.float64)
    want = (d[:, :, None] * q).reshape(7, 128)
    assert np.array_equal(oracle.unpack(fmt, p, 7, 128).astype(np.float64), want)


# ------------------------------------------------------------------ GEMV ---

def test_gemv_orders_match_reference(oracle, ref):
    for fmt in (0, 1):
        for seed, (n, k) in enumerate([(1, 32), (33, 512), (129, 2048), (64, 4096)]):
            rng = np.random.default_rng(100 + seed)
            w = rng.standard_normal((n, k)).astype(np.float32)
            x = rng.standard_normal(k).astype(np.float32)
            _, p = oracle.pack(fmt, w)
            got = oracle.gemv(fmt, p, x, n, k)
            want = ref.gemv(fmt, p, x, n, k)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (fmt, n, k)
            if fmt == 1:
                got = oracle.gemv(fmt, p, x, n, k, order="portable")
                want = ref.gemv(fmt, p, x, n, k, portable=True)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gemv_f64_contract_oracle(oracle):
    for fmt in (0, 1):
        rng = np.random.default_rng(11)
        n, k = 33, 512
        w = rng.standard_normal((n, k)).astype(np.float32)
        x = rng.standard_normal(k).astype(np.float32)
        _, p = oracle.pack(fmt, w)
        y64, wn = oracle.gemv_f64(fmt, p, x, n, k)
        dq = oracle.unpack(fmt, p, n, k).astype(np.float64)
        assert np.allclose(y64, dq @ x.astype(np.float64), rtol=1e-13, atol=1e-12)
        assert np.allclose(wn, np.linalg.norm(dq, axis=1), rtol=1e-13)
        # reference tolerance against the f32 route (test_qgemv.cpp:291-295)
        y = oracle.gemv(fmt, p, x, n, k)
        assert np.all(np.abs(y - y64) <= 1e-5 + 1e-4 * np.abs(y64))


def test_reference_rng_shapes(oracle):
    # the reference's own q4_0 contract case (test_qgemv.cpp:142-182)
    n, k = 33, 512
    vals = xorshift32_unit(0xD1B54A32, n * k + k)
    w, x = vals[: n * k].reshape(n, k), vals[n * k:]
    _, p = oracle.pack(1, w)
    y = oracle.gemv(1, p, x, n, k)
    y64, _ = oracle.gemv_f64(1, p, x, n, k)
    assert np.all(np.abs(y - y64) <= 1e-5 + 1e-4 * np.abs(y64))


# ------------------------------------------------------------ qgemv_w8a8 ---

def _w8a8_cases():
    rng = np.random.default_rng(21)
    for fmt in (0, 1):
        for n, k in ((1, 32), (17, 256), (40, 4096), (3, 14336)):
            w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
            x = rng.standard_normal(k).astype(np.float32)
            if k >= 64:
                x[:32] = 0.0                                       # all-zero block
                x[32:64] = (np.arange(32, dtype=np.float32) - 16) * np.float32(0.5)   # ties
            if k >= 128:
                x[64:96] *= np.float32(1e-30)                       # tiny block
                x[96:128] *= np.float32(1e20)                       # huge block
            yield fmt, n, k, w, x


def test_gemv_w8a8_matches_reference(oracle, ref):
    for fmt, n, k, w, x in _w8a8_cases():
        st, p = oracle.pack(fmt, w)
        assert st == 0
        st, got = oracle.gemv_w8a8(fmt, p, x, n, k)
        assert st == 0
        want = ref.gemv_w8a8(fmt, p, x, n, k)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (fmt, n, k)


def test_gemv_w8a8_numpy_restatement(oracle):
    """Independent float32 restatement: codes from quantize_int8 with 32-element
    groups, exact integer block dots, then sum = sum + (dot * d_w) * d_x in
    block order."""
    for fmt, n, k, w, x in _w8a8_cases():
        if k > 4096:
            continue
        _, p = oracle.pack(fmt, w)
        st, codes, scales = oracle.quantize_int8(x.reshape(1, k), 32)
        assert st == 0
        nb = k // 32
        blocks = p.reshape(n, nb, oracle.BLOCK_BYTES[fmt])
        d = blocks[:, :, 0:2].copy().view(np.float16).astype(np.float32).reshape(n, nb)
        if fmt == 0:
            q = blocks[:, :, 2:].view(np.int8).astype(np.int64)
        else:
            nib = blocks[:, :, 2:].astype(np.int64)
            q = np.concatenate([(nib & 15) - 8, (nib >> 4) - 8], axis=2)
        dots = np.einsum("nbj,bj->nb", q, codes.reshape(nb, 32).astype(np.int64))
        y = np.zeros(n, dtype=np.float32)
        for b in range(nb):
            y = y + (dots[:, b].astype(np.float32) * d[:, b]) * scales[0, b]
        st, got = oracle.gemv_w8a8(fmt, p, x, n, k)
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32)), (fmt, n, k)


def test_gemv_w8a8_reference_test_case(oracle):
    """tests/correctness/test_qgemv_w8a8.cpp:57-116: Rng(1234) weights then x,
    n=96, k=256, within atol 1e-4 + rtol 1e-4 of the dequantized f64 oracle."""
    n, k = 96, 256
    vals = xorshift32_unit(1234, n * k + k)
    w, x = vals[: n * k].reshape(n, k), vals[n * k:]
    for fmt in (1, 0):
        _, p = oracle.pack(fmt, w)
        st, y = oracle.gemv_w8a8(fmt, p, x, n, k)
        assert st == 0
        ref64 = oracle.gemv_w8a8_f64(fmt, p, x, n, k)
        assert np.all(np.abs(y.astype(np.float64) - ref64) <= 1e-4 + 1e-4 * np.abs(ref64))


def test_gemv_w8a8_validation(oracle):
    """Status order of src/dispatch/qgemv_w8a8.cpp:99-105,130-143 and the
    reference test's cases (test_qgemv_w8a8.cpp:126-134)."""
    n, k = 96, 256
    vals = xorshift32_unit(1234, n * k + k)
    w, x = vals[: n * k].reshape(n, k), vals[n * k:].copy()
    _, p = oracle.pack(1, w)
    assert oracle.gemv_w8a8(1, p, x, n, k + 1)[0] == 1
    assert oracle.gemv_w8a8(1, None, x, n, k)[0] == 3
    assert oracle.gemv_w8a8(7, p, x, n, k)[0] == 2
    assert oracle.gemv_w8a8(7, p, x, n, k + 1)[0] == 2      # format before shape
    x[7] = np.nan
    assert oracle.gemv_w8a8(1, p, x, n, k)[0] == 3


# --------------------------------------------------------- quantize_int8 ---

def test_quantize_int8_matches_reference(oracle, ref, synth):
    cases = [
        synth.activations_with_outliers(3, 16, 4096),
        np.zeros((2, 64), np.float32),
        (np.arange(-64, 64, dtype=np.float32) * np.float32(0.5)).reshape(2, 64),
        np.random.default_rng(5).standard_normal((3, 96)).astype(np.float32) * np.float32(1e-30),
    ]
    for x in cases:
        for group in (0, 32):
            st, c, s = oracle.quantize_int8(x, group)
            rst, rc, rs = ref.quantize_int8(x, group)
            assert st == rst == 0
            assert np.array_equal(c, rc) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))


def test_quantize_int8_known_answers(oracle):
    # test_quantization.cpp:100-111: group int8 endpoints
    x = np.array([[-2.0, -0.5, 0.0, 2.0], [1.0, 2.0, 3.0, 4.0]], np.float32)
    st, c, s = oracle.quantize_int8(x, 2)
    assert st == 0 and c[0, 0] == -127 and c[0, 3] == 127 and c[1, 3] == 127
    # closed form, by hand: row max 4 -> scale 4/127, codes rint(x*127/4)
    st, c, s = oracle.quantize_int8(x, 0)
    assert s[1, 0] == np.float32(4.0) / np.float32(127.0)
    assert list(c[1]) == [32, 64, 95, 127]
    # validation
    assert oracle.quantize_int8(np.zeros((2, 6), np.float32), 4)[0] == 1
    bad = np.ones((2, 4), np.float32)
    bad[1, 2] = np.inf
    assert oracle.quantize_int8(bad)[0] == 3


# ------------------------------------------------------------- int8 GEMM ---

def _ref_grid_case(m, n, k, asym, state):
    def u32():
        state[0] ^= (state[0] << 13) & 0xFFFFFFFF
        state[0] ^= state[0] >> 17
        state[0] ^= (state[0] << 5) & 0xFFFFFFFF
        return state[0]
    w = np.array([u32() & 255 for _ in range(n * k)], np.uint8).view(np.int8).reshape(n, k)
    x = np.array([u32() & 255 for _ in range(m * k)], np.uint8).view(np.int8).reshape(m, k)
    w[0, 0] = -1
    x[0, 0] = -128
    ws = (np.float32(0.001) * np.arange(1, n + 1, dtype=np.float32)).astype(np.float32)
    as_ = (np.float32(0.002) * np.arange(1, m + 1, dtype=np.float32)).astype(np.float32)
    rs = w.astype(np.int32).sum(axis=1).astype(np.int32)
    zp = (np.arange(m, dtype=np.int32) - 2) if asym else np.zeros(m, np.int32)
    return w, x, ws, as_, rs, zp.astype(np.int32)


def test_int8_gemm_matches_reference_grid(oracle, ref):
    # tests/correctness/test_int8_gemm.cpp:106-116
    state = [0x9E3779B9]
    for m in range(1, 6):
        for n in range(1, 6):
            for k in (1, 15, 16, 17, 63, 64, 65, 100, 1408):
                for asym in (False, True):
                    w, x, ws, as_, rs, zp = _ref_grid_case(m, n, k, asym, state)
                    st, y = oracle.int8_gemm(w, x, ws, as_, rs, zp, asym)
                    rst, ry = ref.int8_gemm(w, x, ws, as_, rs, zp, asym)
                    assert st == rst == 0
                    assert np.array_equal(y.view(np.uint32), ry.view(np.uint32)), (m, n, k, asym)
                    acc = x.astype(np.int64) @ w.astype(np.int64).T
                    if asym:
                        acc -= zp[:, None].astype(np.int64) * rs[None, :]
                    want = (acc.astype(np.float32) * ws[None, :]) * as_[:, None]
                    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_int8_gemm_known_answers(oracle):
    w = np.array([[1, 2, -1, 3], [-2, 1, 0, 2]], np.int8)
    x = np.array([[2, -1, 3, 1]], np.int8)
    ws = np.array([0.5, 0.25], np.float32)
    as_ = np.array([2.0], np.float32)
    st, y = oracle.int8_gemm(w, x, ws, as_)
    assert st == 0 and abs(y[0, 0] - 0.0) < 1e-6 and abs(y[0, 1] + 1.5) < 1e-6
    st, y = oracle.int8_gemm(w, x, ws, as_, np.array([5, 1], np.int32),
                             np.array([1], np.int32), True)
    assert st == 0 and abs(y[0, 0] + 5.0) < 1e-6 and abs(y[0, 1] + 2.0) < 1e-6
    ws_bad = np.array([np.nan, 1.0], np.float32)
    assert oracle.int8_gemm(w, x, ws_bad, as_)[0] == 3


def test_int8_gemm_entries(oracle):
    rng = np.random.default_rng(9)
    w = rng.integers(-128, 128, (37, 200), dtype=np.int8)
    x = rng.integers(-128, 128, (19, 200), dtype=np.int8)
    ws = rng.uniform(0.001, 0.01, 37).astype(np.float32)
    as_ = rng.uniform(0.001, 0.01, 19).astype(np.float32)
    st, y = oracle.int8_gemm(w, x, ws, as_)
    rows = rng.integers(0, 19, 50)
    cols = rng.integers(0, 37, 50)
    acc, ye = oracle.int8_gemm_entries(w, x, ws, as_, rows, cols)
    assert np.array_equal(acc, (x.astype(np.int64) @ w.astype(np.int64).T)[rows, cols])
    assert np.array_equal(ye.view(np.uint32), y[rows, cols].view(np.uint32))


# ------------------------------------------------ rms_norm_add_quant_int8 ---

def _bits_equal(a, b):
    """(status, arrays...) tuples equal, the arrays bit for bit."""
    return a[0] == b[0] and all(
        np.array_equal(np.ascontiguousarray(p).view(np.uint8), np.ascontiguousarray(q).view(np.uint8))
        for p, q in zip(a[1:], b[1:]))


def test_rms_norm_add_quant_known_answer(oracle):
    # test_remaining_ops.cpp:197-215: x = {1,2,3,4}, residual = 1, weight = 1
    x = np.array([[1, 2, 3, 4]], np.float32)
    st, c, ro, sc = oracle.rms_norm_add_quant_int8(x, np.ones((1, 4), np.float32),
                                                   np.ones(4, np.float32))
    assert st == 0 and ro[0, 3] == 5.0
    # by hand: values {2,3,4,5}, codes rint(v / 5 * 127) = {51, 76, 102, 127}
    assert list(c[0]) == [51, 76, 102, 127]
    inv = np.float32(1.0 / np.sqrt(54.0 / 4.0 + np.float64(np.float32(1e-5))))
    assert sc[0, 0] == np.float32(np.float32(5.0) * inv) / np.float32(127.0)
    # dequantized within the reference test's 0.02 of rms_norm_add
    ref = np.array([2, 3, 4, 5], np.float64) / np.sqrt(54.0 / 4 + 1e-5)
    assert np.all(np.abs(c[0] * np.float64(sc[0, 0]) - ref) <= 0.02)


def _norm_case(rng, rows, hidden, decades=30):
    sc = 10.0 ** rng.uniform(-decades, decades)
    x = (rng.standard_normal((rows, hidden)) * sc).astype(np.float32)
    r = (rng.standard_normal((rows, hidden)) * sc).astype(np.float32)
    w = rng.standard_normal(hidden).astype(np.float32)
    return x, r, w


def test_rms_norm_add_quant_matches_reference(oracle, ref):
    rng = np.random.default_rng(11)
    for trial in range(120):
        hidden = int(rng.choice([4, 32, 96, 128, 1000, 4096]))
        group = int(rng.choice([0, hidden, 4, 32])) if hidden % 32 == 0 else 0
        eps = float(rng.choice([1e-5, 0.0, 1e-6]))
        x, r, w = _norm_case(rng, int(rng.integers(1, 5)), hidden)
        assert _bits_equal(oracle.rms_norm_add_quant_int8(x, r, w, eps, group),
                           ref.rms_norm_add_quant_int8(x, r, w, eps, group))


def test_rms_norm_add_quant_invalid_groups_match_reference(oracle, ref):
    rng = np.random.default_rng(12)
    x, r, w = _norm_case(rng, 3, 64, 1)
    w[5] = np.float32(3e38)
    w[40] = np.inf
    for group in (0, 32, 16):
        a = oracle.rms_norm_add_quant_int8(x, r, w, 1e-5, group)
        assert a[0] == 3 and _bits_equal(a, ref.rms_norm_add_quant_int8(x, r, w, 1e-5, group))
    x[1, 3] = np.nan
    a = oracle.rms_norm_add_quant_int8(x, r, np.ones(64, np.float32), 1e-5, 16)
    assert a[0] == 3 and np.all(a[3][1] == oracle.SCALE_SENTINEL)
    assert _bits_equal(a, ref.rms_norm_add_quant_int8(x, r, np.ones(64, np.float32), 1e-5, 16))
    for eps, group in ((1e-5, 5), (float("nan"), 0), (-1.0, 0), (1e-5, -32), (float("inf"), 0)):
        assert oracle.rms_norm_add_quant_int8(x, r, w, eps, group)[0] == 1
        assert ref.rms_norm_add_quant_int8(x, r, w, eps, group)[0] == 1


def test_rms_norm_add_quant_properties(oracle):
    rng = np.random.default_rng(13)
    for hidden, group in ((4096, 0), (4096, 32), (96, 0), (256, 128)):
        x, r, w = _norm_case(rng, 3, hidden, 20)
        st, c, ro, sc = oracle.rms_norm_add_quant_int8(x, r, w, 1e-5, group)
        assert st == 0
        assert np.array_equal(ro.view(np.uint32), (x + r).view(np.uint32))
        v = ro.astype(np.float64)
        n64 = v / np.sqrt(np.mean(v * v, axis=1, keepdims=True) + np.float64(np.float32(1e-5)))
        n64 = n64 * w.astype(np.float64)
        g = hidden if group == 0 else group
        cg = c.reshape(3, hidden // g, g).astype(np.float64)
        scg = sc.reshape(3, hidden // g, 1).astype(np.float64)
        assert np.all(np.abs(cg).max(axis=2) == 127)
        err = np.abs(cg * scg - n64.reshape(3, hidden // g, g))
        assert np.all(err <= scg * (0.5 + 1e-4))


# ------------------------------------------------ quantize_int8_asymmetric ---

def test_quantize_int8_asymmetric_known_answers(oracle):
    # test_quantization.cpp:113-124 and, by hand: row 0 scale 4/255, zero
    # rint(-128 + 127.5) = 0, codes rint({-127.5, -31.875, 0, 127.5}) clamped;
    # row 1 scale 3/255, zero -128 - 85 = -213, codes {85, 170, 255, 340} - 213
    x = np.array([[-2.0, -0.5, 0.0, 2.0], [1.0, 2.0, 3.0, 4.0]], np.float32)
    st, c, s, z = oracle.quantize_int8_asymmetric(x)
    assert st == 0
    assert list(c[0]) == [-128, -32, 0, 127] and list(c[1]) == [-128, -43, 42, 127]
    assert list(z) == [0, -213]
    assert s[0] == np.float32(4.0 / 255.0) and s[1] == np.float32(3.0 / 255.0)
    st, d = oracle.dequantize_int8_asymmetric(c, s, z)
    assert st == 0 and abs(d[0, 0] + 2.0) <= 0.02 and abs(d[0, 3] - 2.0) <= 0.02
    # test_quantization.cpp:125-136: {-FLT_MAX, FLT_MAX} keeps distinct endpoints
    fmax = np.finfo(np.float32).max
    st, c, s, z = oracle.quantize_int8_asymmetric(np.array([[-fmax, fmax]], np.float32))
    assert st == 0 and np.isfinite(s[0]) and s[0] > 0 and list(c[0]) == [-128, 127]
    # constant row: scale max(|v| / 127, 1e-7), zero -128 - v / scale
    st, c, s, z = oracle.quantize_int8_asymmetric(np.full((1, 3), 2.54, np.float32))
    assert s[0] == np.float32(np.float64(np.float32(2.54)) / 127.0) and z[0] == -255
    bad = np.ones((2, 4), np.float32)
    bad[1, 1] = np.nan
    assert oracle.quantize_int8_asymmetric(bad)[0] == 3


def test_quantize_int8_asymmetric_matches_reference(oracle, ref):
    rng = np.random.default_rng(14)
    cases = [np.array([[0.99999994, 1.0]], np.float32),       # out-of-range zero point
             np.array([[1e-30, 1e-30], [0.0, -0.0]], np.float32),
             np.array([[-3.4028235e38, 3.4028235e38]], np.float32)]
    for trial in range(150):
        rows, dim = int(rng.integers(1, 5)), int(rng.integers(1, 300))
        x = (rng.standard_normal((rows, dim)) * 10.0 ** rng.uniform(-40, 38)).astype(np.float32)
        if trial % 5 == 0:
            x[:, :] = x[:, :1]
        if trial % 7 == 0:
            x += np.float32(rng.uniform(-1e3, 1e3))
        cases.append(x)
    for x in cases:
        a = oracle.quantize_int8_asymmetric(x)
        b = ref.quantize_int8_asymmetric(x)
        assert _bits_equal(a, b)
        assert _bits_equal(oracle.dequantize_int8_asymmetric(*a[1:]),
                           ref.dequantize_int8_asymmetric(*b[1:]))


def test_quantize_int8_asymmetric_round_trip(oracle):
    rng = np.random.default_rng(15)
    x = (rng.standard_normal((8, 512)) * 3.0 + 1.0).astype(np.float32)
    st, c, s, z = oracle.quantize_int8_asymmetric(x)
    st2, d = oracle.dequantize_int8_asymmetric(c, s, z)
    assert st == st2 == 0
    assert np.all(np.abs(d - x) <= s[:, None] * 0.5001)
    assert np.all(c.min(axis=1) == -128) and np.all(c.max(axis=1) >= 126)


# ------------------------------------------------------- qgemv_qkv_rope_kv ---

def _rope_inputs(oracle, fmt, qh, kvh, hd, k, max_pos, seed):
    rng = np.random.default_rng(seed)
    packs = []
    for rows in (qh * hd, kvh * hd, kvh * hd):
        st, p = oracle.pack(fmt, (0.02 * rng.standard_normal((rows, k))).astype(np.float32))
        assert st == 0
        packs.append(p)
    x = rng.standard_normal(k).astype(np.float32)
    ang = rng.uniform(-np.pi, np.pi, (max_pos, hd // 2))
    return packs, x, np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def test_qkv_rope_kv_matches_reference(oracle, ref):
    for case, (fmt, qh, kvh, hd, k, slots, pos, slot) in enumerate(
            [(0, 4, 2, 8, 64, 3, 5, 1), (1, 4, 2, 8, 64, 3, 0, 2), (1, 8, 2, 64, 512, 2, 7, -1),
             (0, 2, 1, 6, 96, 4, 3, 0), (1, 3, 3, 2, 32, 1, 1, 0)]):
        packs, x, c, sn = _rope_inputs(oracle, fmt, qh, kvh, hd, k, 8, 300 + case)
        kc0 = np.arange(slots * kvh * hd, dtype=np.float32)     # other slots must survive
        args = (fmt, *packs, x, c, sn, qh, kvh, hd, k, slots, 8, pos, slot)
        got = oracle.qkv_rope_kv(*args, key_cache=kc0, value_cache=-kc0)
        want = ref.qkv_rope_kv(*args, key_cache=kc0, value_cache=-kc0)
        assert got[0] == want[0] == 0
        for g, w in zip(got[1:], want[1:]):
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), case
        kvd = kvh * hd
        keep = np.ones(slots * kvd, bool)
        if slot >= 0:
            keep[slot * kvd:(slot + 1) * kvd] = False
        assert np.array_equal(got[2][keep], kc0[keep]) and np.array_equal(got[3][keep], -kc0[keep])


def test_qkv_rope_kv_validation_matches_reference(oracle, ref):
    packs, x, c, sn = _rope_inputs(oracle, 0, 2, 1, 4, 64, 4, 9)
    good = dict(query_heads=2, kv_heads=1, head_dim=4, input_dim=64, slots=2, max_position=4,
                position=1, slot=0)
    cases = [dict(head_dim=3), dict(position=4), dict(position=-1), dict(slot=2), dict(slot=-2),
             dict(query_heads=0), dict(slots=0), dict(input_dim=48), dict(input_dim=40),
             dict(kv_heads=-1), dict(max_position=1)]
    # q8_0 / q4_0, and an id past the reference's QuantFormat list (the
    # reference implements its other formats; this build reports them unsupported)
    for fmt in (0, 1, 37):
        for over in cases + [dict()]:
            a = dict(good, **over)
            args = (fmt, *packs, x, c, sn, a["query_heads"], a["kv_heads"], a["head_dim"],
                    a["input_dim"], a["slots"], a["max_position"], a["position"], a["slot"])
            if fmt in (0, 1) and not over:
                continue
            got, want = oracle.qkv_rope_kv(*args)[0], ref.qkv_rope_kv(*args)[0]
            assert got == want, (fmt, over, got, want)
            assert got != 0


def test_qkv_rope_kv_reference_test_case(oracle):
    # tests/correctness/test_remaining_ops.cpp:217-257
    n, k = 2, 32
    proj = np.array([(i % 5 - 2) * 0.1 for i in range(n * k)], np.float32).reshape(n, k)
    act = np.array([(i % 7 - 3) * 0.2 for i in range(k)], np.float32)
    st, p = oracle.pack(0, proj)
    assert st == 0
    qv = oracle.gemv(0, p, act, n, k)
    cos, sin = np.array([1, 0], np.float32), np.array([0, 1], np.float32)
    st, q, kc, vc = oracle.qkv_rope_kv(0, p, p, p, act, cos, sin, 1, 1, 2, k, 2, 2, 1, 1)
    assert st == 0
    assert q[0] == -qv[1] and q[1] == qv[0]
    assert kc[2] == -qv[1] and kc[3] == qv[0] and vc[2] == qv[0] and vc[3] == qv[1]
    assert np.all(kc[:2] == 0) and np.all(vc[:2] == 0)
    st = oracle.qkv_rope_kv(0, p, p, p, act, cos, sin, 1, 1, 2, k, 2, 2, 2, 1)[0]
    assert st == 1


def test_qkv_rope_kv_properties(oracle):
    for fmt in (0, 1):
        qh, kvh, hd, k = 3, 2, 8, 128
        packs, x, c, sn = _rope_inputs(oracle, fmt, qh, kvh, hd, k, 3, 40 + fmt)
        c[1], sn[1] = 1.0, 0.0                                  # zero angle at position 1
        st, q, kc, vc = oracle.qkv_rope_kv(fmt, *packs, x, c, sn, qh, kvh, hd, k, 1, 3, 1, 0)
        assert st == 0
        plain = [oracle.gemv(fmt, packs[i], x, rows, k, order="portable" if fmt else "reference")
                 for i, rows in enumerate((qh * hd, kvh * hd, kvh * hd))]
        assert np.array_equal(q.view(np.uint32), plain[0].view(np.uint32))
        assert np.array_equal(kc.view(np.uint32), plain[1].view(np.uint32))
        assert np.array_equal(vc.view(np.uint32), plain[2].view(np.uint32))
        # a rotation keeps each (d, d + half) pair's length
        st, q, kc, _ = oracle.qkv_rope_kv(fmt, *packs, x, c, sn, qh, kvh, hd, k, 1, 3, 2, 0)
        for out, heads in ((q, qh), (kc, kvh)):
            o = out.reshape(heads, 2, hd // 2).astype(np.float64)
            p = plain[0 if out is q else 1].reshape(heads, 2, hd // 2).astype(np.float64)
            assert np.allclose(np.hypot(o[:, 0], o[:, 1]), np.hypot(p[:, 0], p[:, 1]),
                               rtol=1e-6, atol=1e-9)


# ------------------------------------------------- canonical int8 projections ---

def test_cint8_oracle_matches_reference_scenarios(oracle, ref, tmp_path):
    import storage_eval
    assert ref.storage_scenarios(tmp_path) == 0
    status, bad = storage_eval.check(oracle, tmp_path)
    assert not bad, bad[:10]
    assert len(status) > 100


def test_cint8_dequant_known_answer(oracle):
    # two rows, four columns, groups of two; affine zero points
    codes = np.array([[1, -2, 3, 127], [-128, 0, 5, -5]], np.int8)
    scales = np.array([0.5, 2.0, 0.25, 1.0], np.float32)
    zeros = np.array([1.0, -1.0, 0.0, 2.0], np.float32)
    w = oracle.cint8_dequant(codes, scales, zeros, 2, 4, 2)
    assert w.tolist() == [[0.0, -1.5, 8.0, 256.0], [-32.0, 0.0, 3.0, -7.0]]
    y, wn = oracle.cint8_project_f64(np.array([[1, 2, 3, 4]], np.float32), w)
    assert y.tolist() == [[0 - 3 + 24 + 1024, -32 + 0 + 9 - 28]]
    assert np.allclose(wn, np.linalg.norm(w.astype(np.float64), axis=1))
