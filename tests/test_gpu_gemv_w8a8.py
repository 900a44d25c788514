"""GPU parity: qgemv_w8a8 (activation-quantizing GEMV) through the C ABI.

The reference defines the output bit for bit (per-32-block int8 activations,
exact integer block dots, y[r] = sum_b (float(dot) * d_w) * d_x in block
order; kernels/quantization/qgemv_w8a8_ref.cpp:18-41,120-177), and the GPU
path reproduces that order, so every comparison here is bitwise against the
oracle, which tests/test_oracle.py pins bitwise to the reference's compiled
gemv_w8a8_ref.
"""
import numpy as np
import pytest

from conftest import xorshift32_unit

pytestmark = pytest.mark.gpu


def _weights(oracle, synth, fmt, n, k, seed):
    w = synth.normal_fast(seed, n * k, 0.02).reshape(n, k)
    st, packed = oracle.pack(fmt, w)
    assert st == 0
    return packed


def _run(qc, dev, fmt, packed, x, n, k, w_offset=0, x_offset=0):
    import torch
    pbuf = torch.zeros(packed.size + w_offset, dtype=torch.uint8, device=dev)
    pbuf[w_offset:] = torch.from_numpy(packed).to(dev)
    xbuf = torch.zeros(k + x_offset, dtype=torch.float32, device=dev)
    xbuf[x_offset:] = torch.from_numpy(x).to(dev)
    y = torch.full((n,), 7.0, dtype=torch.float32, device=dev)
    st = qc.qgemv_w8a8_raw(fmt, pbuf[w_offset:], xbuf[x_offset:], y, n, k)
    return st, y.cpu().numpy()


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("fmt,n,k", [(0, 4096, 4096), (1, 14336, 4096), (1, 4096, 14336),
                                     (0, 14336, 4096), (0, 96, 256), (1, 33, 8192),
                                     (0, 7, 20480), (1, 300, 64), (1, 1000, 1408),
                                     (0, 5, 96), (1, 3, 32), (1, 129, 16448)])
def test_qgemv_w8a8_bit_exact(qc, oracle, synth, dev, fmt, n, k):
    print(f"qgemv_w8a8 fmt={fmt} n={n} k={k}", flush=True)
    packed = _weights(oracle, synth, fmt, n, k, 300 + n + k)
    x = synth.normal_fast(400 + k, k)
    st, want = oracle.gemv_w8a8(fmt, packed, x, n, k)
    assert st == 0
    st, got = _run(qc, dev, fmt, packed, x, n, k)
    assert st == 0
    assert np.array_equal(_bits(got), _bits(want))
    st, again = _run(qc, dev, fmt, packed, x, n, k)
    assert st == 0 and np.array_equal(_bits(again), _bits(got))


def test_qgemv_w8a8_reference_case(qc, oracle, dev):
    """tests/correctness/test_qgemv_w8a8.cpp:57-116 (Rng(1234), n=96, k=256)."""
    n, k = 96, 256
    vals = xorshift32_unit(1234, n * k + k)
    w, x = vals[: n * k].reshape(n, k), vals[n * k:]
    for fmt in (1, 0):
        _, packed = oracle.pack(fmt, w)
        _, want = oracle.gemv_w8a8(fmt, packed, x, n, k)
        st, got = _run(qc, dev, fmt, packed, x, n, k)
        assert st == 0 and np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("w_offset,x_offset", [(2, 0), (0, 1), (6, 3)])
def test_qgemv_w8a8_misaligned(qc, oracle, synth, dev, w_offset, x_offset):
    """Unaligned weights take the one-wave-per-row kernel, unaligned x the
    scalar activation loads; the bits do not change."""
    fmt, n, k = 1, 70, 4096
    packed = _weights(oracle, synth, fmt, n, k, 555)
    x = synth.normal_fast(556, k)
    _, want = oracle.gemv_w8a8(fmt, packed, x, n, k)
    st, got = _run(qc, dev, fmt, packed, x, n, k, w_offset, x_offset)
    assert st == 0 and np.array_equal(_bits(got), _bits(want))


def test_qgemv_w8a8_every_rows_per_wave(qc, oracle, synth, dev):
    """Every rows-per-wave variant, bit for bit: whole-line items restaged
    through LDS (q8_0, and q4_0 from 4 rows per wave) and per-lane records,
    whole items (K = 4096) and partial ones (K = 1408: 22 pairs of 64)."""
    n = 1000
    try:
        for k in (4096, 1408):
            for fmt in (0, 1):
                packed = _weights(oracle, synth, fmt, n, k, 600 + fmt + k)
                x = synth.normal_fast(602 + k, k)
                _, want = oracle.gemv_w8a8(fmt, packed, x, n, k)
                for rows in (1, 2, 4, 7, 8, 14):
                    print(f"qgemv_w8a8 fmt={fmt} k={k} rows_per_wave={rows}", flush=True)
                    qc.set_gemv_rows_per_wave(rows)
                    st, got = _run(qc, dev, fmt, packed, x, n, k)
                    assert st == 0 and np.array_equal(_bits(got), _bits(want)), (k, rows)
    finally:
        qc.set_gemv_rows_per_wave(0)


def test_qgemv_w8a8_edge_activations(qc, oracle, synth, dev):
    """All-zero blocks, rounding ties, a single huge or tiny value per block,
    subnormals, and the largest finite floats."""
    n, k = 257, 1024
    x = synth.normal_fast(700, k)
    x[:32] = 0.0
    x[32:64] = (np.arange(32, dtype=np.float32) - 16) * np.float32(0.5)
    x[64:96] = np.float32(1e-3)
    x[70] = np.float32(1e30)
    x[96:128] = np.float32(1e-40) * np.arange(32, dtype=np.float32)
    x[128:160] = np.float32(3e38) * np.sign(x[128:160])
    x[160:192] = np.float32(127.0) * (np.arange(32, dtype=np.float32) - 15.5) / 16.0
    for fmt in (0, 1):
        packed = _weights(oracle, synth, fmt, n, k, 701 + fmt)
        _, want = oracle.gemv_w8a8(fmt, packed, x, n, k)
        st, got = _run(qc, dev, fmt, packed, x, n, k)
        assert st == 0 and np.array_equal(_bits(got), _bits(want))


def test_qgemv_w8a8_nonfinite(qc, oracle, synth, dev):
    """Synchronous form (no status word): status 3 before any work, y
    untouched (src/dispatch/qgemv_w8a8.cpp:138-142).  Asynchronous form: the
    status word reads 3 and the outputs are NaN."""
    import torch
    n, k = 64, 512
    packed = _weights(oracle, synth, 1, n, k, 800)
    x = synth.normal_fast(801, k)
    x[100] = np.nan
    assert oracle.gemv_w8a8(1, packed, x, n, k)[0] == 3
    st, got = _run(qc, dev, 1, packed, x, n, k)
    assert st == 3 and np.all(got == 7.0)
    for bad in (np.nan, np.inf, -np.inf):
        x[100] = bad
        P = torch.from_numpy(packed).to(dev)
        X = torch.from_numpy(x).to(dev)
        y = torch.zeros(n, dtype=torch.float32, device=dev)
        status = torch.zeros(1, dtype=torch.int32, device=dev)
        assert qc.qgemv_w8a8_raw(1, P, X, y, n, k, status) == 0
        torch.cuda.synchronize()
        assert int(status.item()) == 3
        assert torch.all(torch.isnan(y))
